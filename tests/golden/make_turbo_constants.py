"""Writes tests/golden/turbo_constants_d{64,128}.npz: the TurboQuant
constants (rotation Pi, QJL matrix S, Lloyd-Max centroids / boundaries) as
raw fp32 arrays, generated with numpy RandomState + LAPACK QR + scipy as
samfurr/foveated_kv src/foveated_kv/turbo_constants.py:29-100 specifies.
Committed because LAPACK QR bits can differ between builds; the tests pin
them independently (QR uniqueness, orthogonality, the textbook quantiser)
and check that the runtime constants still equal these files.

    python tests/golden/make_turbo_constants.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import turbo  # noqa: E402

for d in (64, 128):
    c = turbo.constants(d)
    np.savez(os.path.join(HERE, f"turbo_constants_d{d}.npz"), **c)
    print(d, c["centroids"], c["boundaries"])

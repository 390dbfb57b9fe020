"""Convert the reference's six legacy attention fixtures to .npz.

Source: samfurr/foveated_kv tests/fixtures/{foveal_only,gqa_mixed,mixed_small,
spike_case,long_context,qwen7b_shape}.pt -- golden vectors from the deleted
3-tier PyTorch reference (docs/phase1_plan.md:109-114).  They are loaded as
data only (torch.load(weights_only=True)); no reference code is imported or
run.  The output files are the committed fixtures; this script only needs to
run again if the conversion changes.

Usage: python tests/golden/make_legacy_fixtures.py [/root/reference]
"""

import os
import sys

import numpy as np
import torch
from torch.torch_version import TorchVersion

NAMES = ["foveal_only", "gqa_mixed", "mixed_small", "spike_case", "long_context", "qwen7b_shape"]


def main(ref_root):
    torch.serialization.add_safe_globals([TorchVersion])
    out_dir = os.path.dirname(os.path.abspath(__file__))
    for name in NAMES:
        path = os.path.join(ref_root, "tests", "fixtures", f"{name}.pt")
        d = torch.load(path, weights_only=True)
        arrays = {}
        for k, v in d["inputs"].items():
            if isinstance(v, torch.Tensor):
                arrays[k] = v.numpy()
            elif isinstance(v, (int, float)):
                arrays[k] = np.array(v, np.float64)
        arrays["ref_output"] = d["ref_output"].numpy()
        arrays["ref_spike_flags"] = d["ref_spike_flags"].numpy().astype(np.int32)
        arrays["ref_spike_tokens"] = d["ref_spike_tokens"].numpy().astype(np.int64)
        np.savez_compressed(os.path.join(out_dir, f"legacy_{name}.npz"), **arrays)
        print("wrote", name, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")

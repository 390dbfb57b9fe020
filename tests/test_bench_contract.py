"""The benchmark's contract on the CPU: a request for more than one GPU exits
with a message, and the algorithmic byte counts behind `value` and
`roofline.achieved` equal the figures the survey derives from the
reference's tier formulas for every benchmark configuration (its section 8d:
C1 0.13 MB, C2 7.74 MB, C3 8K / 16K / 32K 119.45 / 238.78 / 477.43 MB, C5
119.88 MB with its 128 decode rows)."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from foveated_kv_amd import synthetic, tier_cache  # noqa: E402


def _run(args, env_extra=None):
    env = dict(os.environ)
    env.update(env_extra or {})
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")] + args, capture_output=True, text=True,
                          env=env, timeout=120)


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], None), (["--gpus", "8"], None), ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_exits_with_a_message(args, env):
    r = _run(args, env)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def _tiers(S):
    tb = tier_cache.TierConfig().tier_boundaries(S)
    return tb["R_actual"], tb["far_count"]


@pytest.mark.parametrize("name,n_dec,expected", [
    ("c1_qwen05b_512", None, 130_208),
    ("c2_7b_4k", None, 7_735_296),
    ("c3_7b_8k_b8", None, 119_457_056),
    ("c3_7b_16k_b8", None, 238_780_960),
    ("c3_7b_32k_b8", None, 477_428_768),
    ("c5_70b_64k", None, 119_359_744),   # the benchmark's line: the first decode step
    ("c5_70b_64k", 128, 119_884_032),    # the survey's figure: the last of 128 steps
])
def test_algorithmic_bytes_of_the_configurations(name, n_dec, expected):
    B, Hq, Hkv, D, S, nd = synthetic.CONFIGS[name]
    R, F = _tiers(S)
    assert bench.algorithmic_bytes(B, Hq, Hkv, D, R, F, nd if n_dec is None else n_dec) == expected


def test_algorithmic_bytes_turbo_c4():
    B, Hq, Hkv, D, S, nd = synthetic.CONFIGS["c4_turbo_8k_b4"]
    R, F = _tiers(S)
    # 92 far bytes per token at D = 128: 32 index + 16 sign + 4 norm/gamma + 32 value + 8 scale bytes
    assert bench.algorithmic_bytes_turbo(1, 8, 1, 128, 0, 1, 0) - bench.algorithmic_bytes_turbo(
        1, 8, 1, 128, 0, 0, 0) == 92
    assert bench.algorithmic_bytes_turbo(B, Hq, Hkv, D, R, F, nd) == 35_191_200


def test_group32_bytes_add_the_group_scales():
    B, Hq, Hkv, D, S, nd = synthetic.CONFIGS["c3_7b_16k_b8"]
    R, F = _tiers(S)
    # three more fp16 scale / zero pairs per far token (4 groups instead of 1)
    assert (bench.algorithmic_bytes(B, Hq, Hkv, D, R, F, nd, v_group=32) -
            bench.algorithmic_bytes(B, Hq, Hkv, D, R, F, nd)) == B * Hkv * F * 12 == 11_324_928

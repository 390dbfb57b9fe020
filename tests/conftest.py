import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI library)")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle._load()
    return oracle


def pytest_sessionfinish(session, exitstatus):
    """With FKV_PARITY_LOG set, tabulate the margins the GPU parity cases
    logged (tests/_parity.py) into <log>.md beside the log."""
    import json

    path = os.environ.get("FKV_PARITY_LOG")
    if not path or not os.path.exists(path):
        return
    rows = [json.loads(line) for line in open(path) if line.strip()]
    cols = ["maxabs_kernel", "cos_kernel", "maxabs_formulation", "cos_formulation", "flagged", "spike_ties"]
    out = [f"# GPU parity margins ({len(rows)} cases; tolerance max-abs 2e-3, cosine 0.9999)", "",
           "| test | case | " + " | ".join(cols) + " | other |", "|---|---|" + "---|" * (len(cols) + 1)]

    def fmt(v):
        return f"{v:.3e}" if isinstance(v, float) else str(v)

    for r in rows:
        cells = []
        for c in cols:
            v = r.get(c, "")
            cells.append(f"{v:.3e}" if c.startswith("maxabs") and v != "" else
                         f"{v:.8f}" if c.startswith("cos") and v != "" else str(v))
        other = ", ".join(f"{k} {fmt(v)}" for k, v in r.items() if k not in cols and k not in ("test", "case"))
        out.append(f"| `{r['test'].split('::')[-1]}` | {r['case']} | " + " | ".join(cells) + f" | {other} |")
    # sharp cases are held to the bar beyond the fp16 output's own rounding (tests/_parity.py)
    plain = [r for r in rows if "maxabs_kernel" in r and "beyond_output_rounding" not in r]
    sharp = [r for r in rows if "beyond_output_rounding" in r]
    if plain:
        worst = max(r["maxabs_kernel"] for r in plain)
        lowest = min(r["cos_kernel"] for r in plain)
        out += ["", f"Largest max-abs vs the kernel oracle: {worst:.3e}; lowest cosine: {lowest:.8f}."]
    if sharp:
        out += [f"Sharp-softmax cases: largest error beyond the fp16 output rounding "
                f"{max(r['beyond_output_rounding'] for r in sharp):.3e} (raw max-abs up to "
                f"{max(r['maxabs_kernel'] for r in sharp):.3e}, the output's own rounding)."]
    with open(os.path.splitext(path)[0] + ".md", "w") as f:
        f.write("\n".join(out) + "\n")

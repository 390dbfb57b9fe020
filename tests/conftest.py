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
           "| test | case | " + " | ".join(cols) + " |", "|---|---|" + "---|" * len(cols)]
    for r in rows:
        cells = []
        for c in cols:
            v = r.get(c, "")
            cells.append(f"{v:.3e}" if c.startswith("maxabs") and v != "" else
                         f"{v:.8f}" if c.startswith("cos") and v != "" else str(v))
        out.append(f"| `{r['test'].split('::')[-1]}` | {r['case']} | " + " | ".join(cells) + " |")
    worst = max((r["maxabs_kernel"] for r in rows if "maxabs_kernel" in r), default=None)
    lowest = min((r["cos_kernel"] for r in rows if "cos_kernel" in r), default=None)
    if worst is not None:
        out += ["", f"Largest max-abs vs the kernel oracle: {worst:.3e}; lowest cosine: {lowest:.8f}."]
    with open(os.path.splitext(path)[0] + ".md", "w") as f:
        f.write("\n".join(out) + "\n")

"""Writes tests/golden/small_plan.tcff and small_plan.json (a regression pin of the plan
compiler + .tcff writer): a 1-D input, a dense linear layer, a sparse wave with shared rows
and a residual.  Run from the repository root:  python tests/golden/make_golden.py

The same file is independently produced by oracle/plan_oracle.py (checked in
tests/test_plan.py), so the fixture is pinned by two implementations, not only by itself.
"""
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))


def _graph(wavec):
    rng = np.random.default_rng(2024)
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", 80, 1, 72, is_1d=True)
    w = (rng.standard_normal((48, 80)) * 0.1).astype(np.float32)
    b = (rng.standard_normal(48) * 0.1).astype(np.float32)
    g.add_linear("fc", "x", "h", 80, 48, w, b, act="relu")
    rows = rng.integers(0, 48, size=(2, 40)).astype(np.uint32)
    ws = (rng.standard_normal((32, 40)) * 0.1).astype(np.float16)
    bs = (rng.standard_normal(32) * 0.1).astype(np.float16)
    g.add_sparse_wave("sp", "h", "y", rows, ws, bs, cluster=16, act="gelu", res_blob="h")
    g.set_output("y")
    return g


def oracle_graph(po):
    """The same graph for oracle/plan_oracle.py (same generator draws)."""
    rng = np.random.default_rng(2024)
    g = po.Graph()
    g.input("x", 80, 1, 72, True)
    w = (rng.standard_normal((48, 80)) * 0.1).astype(np.float32)
    b = (rng.standard_normal(48) * 0.1).astype(np.float32)
    g.linear("fc", "x", "h", 80, 48, w.astype(np.float16).view(np.uint16),
             b.astype(np.float16).view(np.uint16), act=1)
    rows = rng.integers(0, 48, size=(2, 40)).astype(np.uint32)
    ws = (rng.standard_normal((32, 40)) * 0.1).astype(np.float16)
    bs = (rng.standard_normal(32) * 0.1).astype(np.float16)
    g.sparse("sp", "h", "y", rows, ws.view(np.uint16), bs.view(np.uint16), cluster=16, act=5,
             residual="h")
    g.output = "y"
    return g


def build_tcff(wavec, path) -> bytes:
    g = _graph(wavec)
    plan = g.compile()
    plan.save_tcff(path, "Golden")
    return Path(path).read_bytes()


def summary_fields(wavec) -> dict:
    plan = _graph(wavec).compile()
    s = plan.summary
    return {"canvas_elems": s["canvas_elems"], "output_shape": s["output_shape"],
            "cmds": [{k: c[k] for k in ("name", "Cout", "B", "B_raw", "S", "src_off", "y_off")}
                     for c in s["cmds"]]}


if __name__ == "__main__":
    from snntome_amd import wavec

    data = build_tcff(wavec, HERE / "small_plan.tcff")
    (HERE / "small_plan.json").write_text(json.dumps(summary_fields(wavec), indent=1) + "\n")
    print(f"wrote small_plan.tcff ({len(data)} bytes) and small_plan.json")

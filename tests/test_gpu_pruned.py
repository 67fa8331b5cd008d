"""Pruned projections on the GPU: every neuron keeps its own clusters; the compiler's
pattern-sorted tiles (zero-filled unions, cout_map stores, empty slots) must give the same
outputs as the per-neuron formulation evaluated by the fp64 oracle."""
import numpy as np
import pytest

from snntome_amd import synth

from wave_cases import PATH_IDS, TOL, stride_of

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("path", ["auto", "valu"])
@pytest.mark.parametrize("n_cl,K,S,tile,cout,act,res", [
    (4, 2, 64, 64, 448, "silu", False),
    (11, 6, 32, 16, 200, None, True),
    (6, 3, 32, 32, 97, "gelu", False),
])
def test_pruned_wave_matches_per_neuron_oracle(wavec, orc, tuning, path, n_cl, K, S, tile,
                                               cout, act, res):
    if path != "auto":
        tuning("path", PATH_IDS[path])
    rng = np.random.default_rng(n_cl * 7 + K)
    C, tokens = n_cl * S, 100
    pick = np.argsort(rng.random((cout, n_cl)), axis=1)[:, :K]
    starts = (pick * S).astype(np.uint32)
    w = synth.normal_f16(rng, (cout, K * S), 0.05)
    b = synth.normal_f16(rng, (cout,), 0.05)
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", C, 1, tokens, is_1d=True)
    g.add_pruned_wave("p", "x", "y", starts, S, w, b, tile=tile, act=act,
                      res_blob="x" if res else None)
    plan = g.compile()
    plan.init_gpu()
    rep = plan.exec_report()["waves"]
    _log(f"[pruned {n_cl}/{K} S={S} tile={tile} {path}] parts "
         f"{[(r['path'], r['cout'], r['K']) for r in rep]}")
    if path == "valu":
        assert {r["path"] for r in rep} == {"valu_gather_dot"}
    elif tile >= 16 and S % 32 == 0:
        assert {r["path"] for r in rep} <= {"mfma_tile", "mfma_dma"}
    plan.fill_input_uniform(5)
    plan.execute(1)
    st = stride_of(tokens)
    canvas = plan.read_canvas(0, int(plan.summary["canvas_elems"]))
    x0 = int(plan.cmds[0]["src_off"])
    seg = (x0 + starts.astype(np.uint64) * st).ravel()
    # per-neuron formulation; with a residual the cout_map epilogue is act(v + r) (act = none here)
    ref = orc.wave_f64(canvas, seg, w, b, None, K, S, 1, st, st, st, act,
                       res_off=x0 if res else None)
    y0 = int(plan.cmds[0]["y_off"])
    y = canvas[y0:y0 + cout * st].view(np.float16).reshape(cout, st).astype(np.float64)
    err = orc.rel_err(y, ref)
    _log(f"  rel err {err:.3e}")
    assert err <= TOL

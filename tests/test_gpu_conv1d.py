"""Token-shifted 1-D taps on the GPU: 1-D convolutions compiled through the reference ABI
(wavec_add_conv2d on a 1-D input, kh = 1, kw = 3 / 5) gather at element offsets
ch_base + dx (reference wavec/k44_plan_types.hpp:593-595, kernel44_rocm_pack.cuh:57-66), which
sit off the 8-byte grid for odd dx.  Checked against the fp64 oracle evaluated on the canvas the
wave read, with the tap offsets built here from the reference formula (not from the plan)."""
import numpy as np
import pytest

from wave_cases import TOL, stride_of

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _conv1d_plan(wavec, rng, cin, cout, kw, W, act, residual):
    """x -> linear (so the convolution's input is not at canvas offset 0) -> 1-D conv."""
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", cin, 1, W, is_1d=True)
    w0 = (rng.standard_normal((cin, cin)) * 0.2).astype(np.float32)
    b0 = (rng.standard_normal(cin) * 0.1).astype(np.float32)
    g.add_linear("pre", "x", "h", cin, cin, w0, b0, act="relu")
    wc = (rng.standard_normal((cout, cin, 1, kw)) * 0.05).astype(np.float32)
    bc = (rng.standard_normal(cout) * 0.05).astype(np.float32)
    g.add_conv2d("conv", "h", "y", cin, cout, 1, kw, wc, bc, stride=1, pad=kw // 2, act=act,
                 res_blob="h" if residual else None)
    return g.compile(), wc, bc


@pytest.mark.parametrize("kw", [3, 5])
@pytest.mark.parametrize("W", [100, 128, 256])
@pytest.mark.parametrize("residual", [False, True])
def test_token_shifted_conv1d_matches_oracle(wavec, orc, kw, W, residual):
    rng = np.random.default_rng(kw * 1000 + W + residual)
    cin = 64
    cout = cin if residual else 48
    act = "silu"
    plan, wc, bc = _conv1d_plan(wavec, rng, cin, cout, kw, W, act, residual)
    plan.init_gpu()
    rep = plan.exec_report()["waves"][1]
    _log(f"[conv1d kw={kw} W={W} res={residual}] path={rep['path']} K={rep['K']} S={rep['S']} "
         f"misaligned={rep['misaligned']} phase_order={rep['phase_order']}")
    assert rep["misaligned"] and rep["phase_order"]
    assert (rep["K"], rep["S"]) == (kw, cin)  # kw segments of cin consecutive channels
    plan.fill_input_uniform(17)
    plan.execute_range(0, 1)
    n = int(plan.summary["canvas_elems"])
    canvas = plan.read_canvas(0, n)  # what the convolution reads
    plan.execute_range(1, 1)
    c = plan.cmds[1]
    st = stride_of(W)
    h_off = int(c["src_off"])
    # Reference gather offsets: channel base + tap shift dx = kx - kw // 2 (synapse ch*kw + kx).
    syn = np.array([h_off + ch * st + (kx - kw // 2) for ch in range(cin) for kx in range(kw)],
                   dtype=np.uint64)
    w16 = wc.reshape(cout, cin * kw).astype(np.float16)
    ref = orc.wave_f64(canvas, syn, w16, bc.astype(np.float16), None, cin * kw, 1, cout, st,
                       st, st, act, res_off=h_off if residual else None)
    y = plan.read_canvas(int(c["y_off"]), cout * st).view(np.float16).reshape(cout, st)
    # Columns whose taps stay inside the input tensor's own rows (past them the wave reads the
    # next tensor, which is its own output: those columns are unspecified, as in the reference).
    lim = W if W + kw // 2 <= st else W - kw // 2
    err = orc.rel_err(y[:, :lim].astype(np.float64), ref[:, :lim])
    _log(f"[conv1d kw={kw} W={W} res={residual}] rel err {err:.3e} over {cout} x {lim}")
    assert err <= TOL


@pytest.mark.parametrize("cout", [64, 128])
@pytest.mark.parametrize("W", [100, 256])
@pytest.mark.parametrize("residual", [False, True])
def test_token_shifted_conv1d_on_mfma(wavec, orc, tuning, cout, W, residual):
    """A dense token-shifted 1-D convolution (cin 256, kw 3: 3 segments of 256 channels, two of
    them off the 16-byte grid by one element) runs on the matrix cores: the register-staged MFMA
    tile kernel loads the aligned 16-byte chunks around each lane's tokens and shifts them into
    place.  Both this path and the VALU funnel-shift gather (tuning path=0) are checked against
    the fp64 oracle with tap offsets from the reference formula."""
    rng = np.random.default_rng(cout + W + 7 * residual)
    cin, kw = 256, 3
    cout = cin if residual else cout
    act = "gelu"
    for mode in ("mfma", "valu"):
        tuning("path", -1 if mode == "mfma" else 0)
        plan, wc, bc = _conv1d_plan(wavec, np.random.default_rng(cout + W + 7 * residual), cin,
                                    cout, kw, W, act, residual)
        plan.init_gpu()
        rep = plan.exec_report()["waves"][1]
        _log(f"[conv1d mfma cin={cin} cout={cout} W={W} res={residual} {mode}] "
             f"path={rep['path']} K={rep['K']} S={rep['S']} ksplit={rep['ksplit']}")
        if mode == "mfma":
            assert rep["path"] == "mfma_tile" and "shifted into place" in rep["why"], rep
        else:
            assert rep["path"] == "valu_gather_dot" and rep["misaligned"], rep
        assert (rep["K"], rep["S"]) == (kw, cin)
        plan.fill_input_uniform(23)
        plan.execute_range(0, 1)
        canvas = plan.read_canvas(0, int(plan.summary["canvas_elems"]))
        plan.execute_range(1, 1)
        c = plan.cmds[1]
        st = stride_of(W)
        h_off = int(c["src_off"])
        syn = np.array([h_off + ch * st + (kx - kw // 2) for ch in range(cin) for kx in range(kw)],
                       dtype=np.uint64)
        w16 = wc.reshape(cout, cin * kw).astype(np.float16)
        ref = orc.wave_f64(canvas, syn, w16, bc.astype(np.float16), None, cin * kw, 1, cout, st,
                           st, st, act, res_off=h_off if residual else None)
        y = plan.read_canvas(int(c["y_off"]), cout * st).view(np.float16).reshape(cout, st)
        lim = W if W + kw // 2 <= st else W - kw // 2
        err = orc.rel_err(y[:, :lim].astype(np.float64), ref[:, :lim])
        _log(f"[conv1d mfma cin={cin} cout={cout} W={W} res={residual} {mode}] rel err {err:.3e}")
        assert err <= TOL
        plan.release_gpu()

"""Multi-wave plans (config 4): waves read earlier waves' outputs through the canvas."""
import numpy as np
import pytest

from snntome_amd import synth

from wave_cases import TOL, stride_of

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _wave_inputs(plan, wl, i, st):
    """Canvas element offset of every channel of wave i's (concatenated) input."""
    cmds = plan.cmds
    x0 = int(cmds[0]["src_off"])
    offs = [x0 + np.arange(wl.substrate, dtype=np.uint64) * st]
    for t in range(i):
        y = int(cmds[t]["y_off"])
        offs.append(y + np.arange(wl.waves[t].cout, dtype=np.uint64) * st)
    return np.concatenate(offs)


def test_config4_full_plan_wavewise(wavec, orc):
    """Full config 4 (8 waves x 4,096 neurons x 16 x S=128, batch 128): after one end-to-end
    run, every output of every wave (all 4,096 neurons x 128 tokens) is checked against the
    oracle evaluated on the canvas that wave read."""
    wl = synth.config4()
    _log(f"[c4] {wl.description}")
    plan = synth.build_graph(wl, wavec).compile()
    plan.init_gpu()
    rep = plan.exec_report()["waves"]
    assert [w["path"] for w in rep] == ["valu_gather_dot"] * 8
    assert all((w["K"], w["S"]) == (16, 128) for w in rep)
    plan.fill_input_uniform(wl.seed)
    plan.execute(1)
    st = stride_of(wl.tokens)
    canvas = plan.read_canvas(0, int(plan.summary["canvas_elems"]))
    for i, w in enumerate(wl.waves):
        chan = _wave_inputs(plan, wl, i, st)
        seg = chan[w.starts.astype(np.int64)].ravel()
        ref = orc.wave_f64(canvas, seg, w.weights, w.bias, None, w.K, w.S, 1, st, st, st,
                           w.act)
        y0 = int(plan.cmds[i]["y_off"])
        y = canvas[y0:y0 + w.cout * st].view(np.float16).reshape(w.cout, st)
        err = orc.rel_err(y.astype(np.float64), ref)
        _log(f"[c4] wave {i}: rel err {err:.3e}")
        assert err <= TOL


def test_multiwave_chain_end_to_end(wavec, orc):
    """Reduced 8-wave plan evaluated end to end by the oracle alone (fp16 rounding between
    waves, as on the canvas) and compared with the GPU's final wave."""
    wl = synth.config4(waves=8, width=4096, neurons=256, K=8, S=64, tokens=128)
    plan = synth.build_graph(wl, wavec).compile()
    plan.init_gpu()
    plan.fill_input_uniform(wl.seed)
    plan.execute(1)
    st = stride_of(wl.tokens)
    gpu = plan.read_canvas(0, int(plan.summary["canvas_elems"]))
    ref_canvas = np.zeros_like(gpu)
    x0 = int(plan.cmds[0]["src_off"])
    ref_canvas[x0:x0 + wl.substrate * st] = synth.substrate_rows(
        wl.seed, np.arange(wl.substrate), st, valid=wl.tokens).view(np.uint16).ravel()
    for i, w in enumerate(wl.waves):
        chan = _wave_inputs(plan, wl, i, st)
        seg = chan[w.starts.astype(np.int64)].ravel()
        out = orc.wave_f64(ref_canvas, seg, w.weights, w.bias, None, w.K, w.S, 1, st, st, st,
                           w.act)
        y0 = int(plan.cmds[i]["y_off"])
        ref_canvas[y0:y0 + w.cout * st] = out.astype(np.float32).astype(np.float16).view(
            np.uint16).ravel()
    last = len(wl.waves) - 1
    y0 = int(plan.cmds[last]["y_off"])
    n = wl.waves[last].cout * st
    y = gpu[y0:y0 + n].view(np.float16).astype(np.float64)
    r = ref_canvas[y0:y0 + n].view(np.float16).astype(np.float64)
    err = orc.rel_err(y, r)
    _log(f"[c4-chain] final wave rel err {err:.3e}")
    assert err <= TOL
    # and the plan output read through the reference entry point shape
    assert tuple(plan.summary["output_shape"]) == (wl.waves[last].cout, 1, wl.tokens)

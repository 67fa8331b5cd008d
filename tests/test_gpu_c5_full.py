"""Config 5 — the LLM-shaped decoder — at its real size on the GPU (16 layers, d 2048, FFN 5632,
vocab 32,000; 16 requests x 512-token prefill; decode one token per request), checked node by
node against the CPU oracle at the north_star bound (tests/llm_check.py):

  * the prefill plan command by command (every sub-wave, union tile and token op launched
    alone) and run by run (the whole-plan schedule: group launches over 8,192 tokens), on three
    64-token windows of every tensor (first request start, a request boundary, last tokens);
  * a full-width 16-layer decode step after a real prefill hand-over, command by command and
    run by run (folded multiplies, relocated operands, RMSNorm + token shift kernels);
  * the whole decode plan, folded and replayed as a HIP graph, against the plan with nothing
    folded launched kernel by kernel: ids and logits bit for bit over several steps.
"""
import numpy as np
import pytest

from llm_check import PlanChecker
from snntome_amd import synth

pytestmark = pytest.mark.gpu

FULL = synth.LLMSpec()
WINDOWS = [(0, 64), (4064, 64), (8128, 64)]
DECODE_STEPS = 3


def _log(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def c5(wavec):
    _log("[c5 full] building weights and the prefill plan")
    wts = synth.llm_weights(FULL)
    pre = synth.build_llm_graph(FULL, wts, decode=False, wavec_mod=wavec).compile()
    pre.init_gpu()
    n = FULL.requests * FULL.prompt
    ids = np.random.default_rng(55).integers(0, FULL.vocab, n).astype(np.uint32)
    return wts, pre, ids


def _head(plan):
    return next(c for c in plan.cmds if c["name"].split("/")[0] == "head")


def test_c5_prefill_full_size_commandwise(c5):
    wts, pre, ids = c5
    PlanChecker(pre, FULL, wts, ids.size, False, WINDOWS, log=_log).run(
        "commands", ids, "c5 prefill full size")


def test_c5_prefill_full_size_runwise_equals_whole_plan(c5):
    """Run by run through the whole-plan schedule; then the whole plan in one call reproduces
    the run-wise logits windows and ids bit for bit."""
    wts, pre, ids = c5
    rep = pre.exec_report()
    _log(f"[c5 prefill] {len(rep['runs'])} runs, {len(rep['groups'])} group launches, "
         f"largest group {max(len(g) for g in rep['groups'])} waves")
    chk = PlanChecker(pre, FULL, wts, ids.size, False, WINDOWS, log=_log)
    chk.run("runs", ids, "c5 prefill full size")
    h = _head(pre)
    logits = chk.rows(h["y_off"], h["logical_Cout"])
    got_ids = pre.get_ids(ids.size)
    pre.set_ids(ids)
    pre.execute(1)
    assert np.array_equal(chk.rows(h["y_off"], h["logical_Cout"]).view(np.uint16),
                          logits.view(np.uint16))
    assert np.array_equal(pre.get_ids(ids.size), got_ids)


@pytest.fixture(scope="module")
def c5_decode(c5, wavec):
    """Decode plans handed over from one whole-plan prefill run: 'cmd' and 'run' (defaults),
    'graph' (kernel by kernel, HIP-graph replay), 'unfused' (tuning switch fuse=0), 'prog'
    (tuning program=1: whole-plan runs as the persistent decode launch) and 'prog_ref' (kernel by
    kernel, compared with 'prog' only)."""
    wts, pre, ids = c5
    pre.set_ids(ids)
    pre.execute(1)
    plans = {}
    for name in ("cmd", "run", "graph", "unfused", "prog", "prog_ref"):
        wavec.reset_tuning()
        if name == "unfused":
            wavec.set_tuning("fuse", 0)
        if name in ("graph", "prog_ref"):
            wavec.set_tuning("program", 0)
        if name == "prog":
            wavec.set_tuning("program", 1)
        p = synth.build_llm_graph(FULL, wts, decode=True, wavec_mod=wavec).compile()
        p.init_gpu()
        synth.llm_handoff(FULL, pre, p)
        plans[name] = p
    wavec.reset_tuning()
    return wts, plans


def test_c5_decode_step_full_size_commandwise(c5_decode):
    wts, plans = c5_decode
    p = plans["cmd"]
    R = FULL.requests
    PlanChecker(p, FULL, wts, R, True, log=_log).run("commands", p.get_ids(R),
                                                      "c5 decode full size")


def test_c5_decode_step_full_size_runwise(c5_decode):
    wts, plans = c5_decode
    p = plans["run"]
    rep = p.exec_report()
    n_mul = sum(a["fused"] and a["type"] == "SWIGLU_MUL_1D" for a in rep["aux"])
    n_shift = sum(a["fused"] and a["type"] == "TOKEN_SHIFT_1D" for a in rep["aux"])
    moved = sum(w["y_off_run"] != w["y_off"] for w in rep["waves"])
    _log(f"[c5 decode] {len(rep['runs'])} runs: {n_mul} multiplies folded, {n_shift} token "
         f"shifts run by their RMSNorm, {moved} sub-waves store to relocated operands")
    assert n_mul == 3 * FULL.layers and n_shift == FULL.layers
    R = FULL.requests
    PlanChecker(p, FULL, wts, R, True, log=_log).run("runs", p.get_ids(R),
                                                      "c5 decode full size")


def test_c5_decode_graph_folded_matches_unfused_full_size(c5_decode):
    """The default decode plan (folded multiplies, RMSNorm + token shift kernels, group launches)
    replayed as a HIP graph, against the plan with nothing folded launched kernel by kernel:
    ids and logits bit for bit after every step."""
    _, plans = c5_decode
    g, u = plans["graph"], plans["unfused"]
    assert not any(a["fused"] for a in u.exec_report()["aux"])
    g.use_graph(True)
    R = FULL.requests
    hg, hu = _head(g), _head(u)
    for step in range(DECODE_STEPS):
        g.execute(1)
        u.execute(1)
        ids_g, ids_u = g.get_ids(R), u.get_ids(R)
        lg = g.read_canvas(int(hg["y_off"]), FULL.vocab * 64)
        lu = u.read_canvas(int(hu["y_off"]), FULL.vocab * 64)
        _log(f"[c5 decode graph vs unfused] step {step}: ids {ids_g[:4].tolist()}...")
        assert np.array_equal(ids_g, ids_u), step
        # logits of the batch's token columns (columns past it are unspecified)
        assert np.array_equal(lg.reshape(FULL.vocab, 64)[:, :R], lu.reshape(FULL.vocab, 64)[:, :R]), step


def test_c5_decode_program_matches_runwise_full_size(c5_decode):
    """The persistent decode launch at full size (16 layers) against the kernel-by-kernel plan
    that the run-wise checker verifies node by node: both start from the same hand-over and
    take the same ids every step; logits agree to a few fp16 ulps of the largest logit (the
    projections sum their contractions in another order), ids wherever the top two logits are
    clearly apart."""
    _, plans = c5_decode
    p, u = plans["prog"], plans["prog_ref"]
    rep = p.exec_report()["program"]
    _log(f"[c5 decode program] {rep}")
    assert rep["active"], rep["why"]
    R = FULL.requests
    hp, hu = _head(p), _head(u)
    ids = p.get_ids(R)
    assert np.array_equal(ids, u.get_ids(R))
    for step in range(DECODE_STEPS):
        p.set_ids(ids)
        u.set_ids(ids)
        p.execute(1)
        u.execute(1)
        lp = p.read_canvas(int(hp["y_off"]), FULL.vocab * 64).view(np.float16)
        lu = u.read_canvas(int(hu["y_off"]), FULL.vocab * 64).view(np.float16)
        lp = lp.reshape(FULL.vocab, 64)[:, :R].astype(np.float64)
        lu = lu.reshape(FULL.vocab, 64)[:, :R].astype(np.float64)
        scale = np.abs(lu).max()
        err = np.abs(lp - lu).max() / scale
        srt = np.sort(lu, axis=0)
        clear = (srt[-1] - srt[-2]) > 0.05 * scale
        _log(f"[c5 decode program] step {step}: max|d| / max|logit| = {err:.3e}, "
             f"{int(clear.sum())} of {R} ids with a clear margin")
        assert err <= 1e-2, step
        assert np.array_equal(p.get_ids(R)[clear], u.get_ids(R)[clear]), step
        ids = u.get_ids(R)

"""The persistent decode launch (kernels/k44_program.hip, tuning program=1): a decode-sized plan runs
every whole-plan execution as one launch whose stages wait on device-scope completion counters.  Checked here:
which plans take it, its logits against the kernel-by-kernel plan and the fp64 oracle, greedy
decoding with the device-side id history, and a stage wait past its time limit (forced from the
host with a zero limit) reported as an error, after which the plan runs correctly again."""
import numpy as np
import pytest

from oracle import llm_oracle as lo
from snntome_amd import synth

pytestmark = pytest.mark.gpu

TINY = synth.LLMSpec(layers=2, d=256, ffn=384, vocab=640, S=64, requests=2, prompt=64,
                     decode_steps=4, seed=9)
# Full config-5 widths, 2 layers (the oracle's fp64 forward stays within seconds).
WIDE = synth.LLMSpec(layers=2)
# Relative to the largest logit (as the other end-to-end decode tests).
E2E_TOL = 1e-2


def _log(msg):
    print(msg, flush=True)


def _head(plan):
    return next(c for c in plan.cmds if c["name"].split("/")[0] == "head")


def _logits(plan, spec, R):
    h = _head(plan)
    x = plan.read_canvas(int(h["y_off"]), spec.vocab * 64).view(np.float16)
    return x.reshape(spec.vocab, 64)[:, :R].astype(np.float64)


def _decode_plan(spec, wts, wavec, tuning, program):
    tuning("program", 1 if program else -1)
    p = synth.build_llm_graph(spec, wts, decode=True, wavec_mod=wavec).compile()
    p.init_gpu()
    return p


def test_program_taken_by_decode_plans_only(wavec, tuning):
    wts = synth.llm_weights(TINY)
    dec = _decode_plan(TINY, wts, wavec, tuning, True)
    rep = dec.exec_report()
    _log(f"[program] decode: {rep['program']}")
    assert rep["program"]["active"] and rep["launches_per_run"] == 1
    # every run is a stage; an argmax adds its final stage
    assert rep["program"]["stages"] == len(rep["runs"]) + 1
    pre = synth.build_llm_graph(TINY, wts, decode=False, wavec_mod=wavec).compile()
    pre.init_gpu()
    prep = pre.exec_report()["program"]
    _log(f"[program] prefill: {prep}")
    assert not prep["active"]
    assert "decode-sized" in prep["why"] or "no program form" in prep["why"]
    off = _decode_plan(TINY, wts, wavec, tuning, False).exec_report()["program"]
    assert not off["active"] and "program=1" in off["why"]


@pytest.mark.parametrize("spec", [TINY, WIDE], ids=["tiny", "wide"])
def test_program_matches_launches_and_oracle(wavec, tuning, spec):
    """Same ids every step into a persistent-launch plan and a kernel-by-kernel plan (zero
    token-shift history in both): logits agree within the end-to-end bound, step after step
    (the shift state carries over), and the first step's logits match the fp64 oracle."""
    wts = synth.llm_weights(spec)
    prog = _decode_plan(spec, wts, wavec, tuning, True)
    ref = _decode_plan(spec, wts, wavec, tuning, False)
    assert prog.exec_report()["program"]["active"]
    R = spec.requests
    rng = np.random.default_rng(17)
    for step in range(3):
        ids = rng.integers(0, spec.vocab, R).astype(np.uint32)
        for p in (prog, ref):
            p.set_ids(ids)
            p.execute(1)
        lp, lr = _logits(prog, spec, R), _logits(ref, spec, R)
        scale = np.abs(lr).max()
        err = np.abs(lp - lr).max() / scale
        srt = np.sort(lr, axis=0)
        clear = (srt[-1] - srt[-2]) > 0.05 * scale
        _log(f"[program {spec.d}] step {step}: max|d| / max|logit| = {err:.3e}, "
             f"{int(clear.sum())} of {R} clear ids")
        assert err <= E2E_TOL, step
        assert np.array_equal(prog.get_ids(R)[clear], ref.get_ids(R)[clear]), step
        if step == 0:
            zero = [np.zeros((spec.d, spec.rf - 1, 64), np.float16) for _ in range(spec.layers)]
            want = lo.llm_forward(spec, wts, ids, decode=True, shift_state=zero)
            w = want.tensors["logits"][:, :R].astype(np.float64)
            e2 = np.abs(lp - w).max() / np.abs(w).max()
            _log(f"[program {spec.d}] against the fp64 oracle: {e2:.3e}")
            assert e2 <= E2E_TOL
            ws = np.sort(w, axis=0)
            wclear = (ws[-1] - ws[-2]) > 0.05
            assert np.array_equal(prog.get_ids(R)[wclear], want.ids[wclear])


def test_program_greedy_history_and_repeats(wavec, tuning):
    """Greedy decoding over the device-side id history: the persistent launch's ids equal the
    argmax of its own logits every step, the history holds them in order, and repeating the
    same start reproduces every step bit for bit (counters, sums and keys return to zero)."""
    spec = TINY
    steps = 5
    wts = synth.llm_weights(spec)
    R = spec.requests
    ids0 = np.random.default_rng(23).integers(0, spec.vocab, R).astype(np.uint32)
    runs = []
    for rep in range(2):
        p = _decode_plan(spec, wts, wavec, tuning, True)
        p.set_history(steps)
        p.set_ids(ids0)
        got_ids, got_logits = [], []
        for s in range(steps):
            p.execute(1)
            lg = _logits(p, spec, R)
            ids = p.get_ids(R)
            assert np.array_equal(ids, lo.argmax(lg.astype(np.float16), R)), (rep, s)
            got_ids.append(ids)
            got_logits.append(lg)
        hist = p.get_history(steps, R)
        assert np.array_equal(hist, np.stack(got_ids))
        runs.append((np.stack(got_ids), np.stack(got_logits)))
        p.release_gpu()
    assert np.array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1], runs[1][1])
    _log(f"[program greedy] ids {runs[0][0].tolist()}")


def test_program_wait_limit_reported_then_recovers(wavec, tuning):
    """A zero wait limit (set from the host) makes the first stage wait that is not already
    satisfied give up: the launch ends normally, wavec_gpu_execute returns -1 naming the stage,
    and the plan initialised again with the default limit computes the right logits."""
    spec = TINY
    wts = synth.llm_weights(spec)
    R = spec.requests
    ids = np.random.default_rng(29).integers(0, spec.vocab, R).astype(np.uint32)
    ref = _decode_plan(spec, wts, wavec, tuning, False)
    ref.set_ids(ids)
    ref.execute(1)
    want = _logits(ref, spec, R)
    tuning("program", 1)
    tuning("prog_spin_ms", 0)
    p = synth.build_llm_graph(spec, wts, decode=True, wavec_mod=wavec).compile()
    p.init_gpu()
    assert p.exec_report()["program"]["active"]
    p.set_ids(ids)
    with pytest.raises(RuntimeError, match="abandoned"):
        p.execute(1)
    _log(f"[program wait limit] {wavec.last_error()}")
    tuning("prog_spin_ms", -1)
    p.release_gpu()
    p.init_gpu()  # rebuilt with the default limit
    assert p.exec_report()["program"]["active"]
    p.set_ids(ids)
    p.execute(1)
    got = _logits(p, spec, R)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err <= E2E_TOL

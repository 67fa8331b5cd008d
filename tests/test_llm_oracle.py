"""Pins of the CPU restatement of the token ops and the LLM-shaped decoder (oracle/llm_oracle.py)
against brute-force loops, closed forms and invariants, so that a dropped term, a shifted index
or a swapped operand in the oracle fails here before it is used to judge the device."""
import numpy as np
import pytest

from oracle import llm_oracle as lo
from snntome_amd import synth


def _f16(rng, shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def test_rmsnorm_closed_forms():
    # constant column c -> sign(c) / sqrt(1 + eps/c^2); one-hot column -> sqrt(D)
    D = 64
    x = np.zeros((D, 4), np.float16)
    x[:, 0] = 2.0
    x[:, 1] = -0.5
    x[7, 2] = 1.0
    y = lo.rmsnorm(x).astype(np.float64)
    assert np.allclose(y[:, 0], 1.0, atol=1e-3) and np.allclose(y[:, 1], -1.0, atol=1e-3)
    assert abs(y[7, 2] - np.sqrt(D)) < 8e-3 and np.count_nonzero(y[:, 2]) == 1
    assert np.all(y[:, 3] == 0)  # all-zero column stays zero (eps keeps it finite)
    g = np.linspace(0.5, 1.5, D).astype(np.float16)
    yg = lo.rmsnorm(x, g).astype(np.float64)
    assert np.allclose(yg[:, 0], g.astype(np.float64), atol=2e-3)


def test_rmsnorm_scale_invariance():
    rng = np.random.default_rng(0)
    x = _f16(rng, (96, 16))
    a = lo.rmsnorm(x, eps=0.0)
    b = lo.rmsnorm((x.astype(np.float32) * 4).astype(np.float16), eps=0.0)  # exact scale by 4
    assert np.array_equal(a, b)


def test_mul_exact_product():
    rng = np.random.default_rng(1)
    a, b = _f16(rng, (8, 64)), _f16(rng, (8, 64))
    # a product of two fp16 is exact in fp32, so one fp16 rounding of it is the answer
    exp = (a.astype(np.float32) * b.astype(np.float32)).astype(np.float16)
    assert np.array_equal(lo.mul(a, b), exp)
    assert not np.array_equal(lo.mul(a, b), lo.mul(a, b[:, ::-1]))


def _shift_loops(x, mu, seq_len, valid):
    D, T = x.shape
    rf = mu.shape[1]
    y = np.zeros((D, T))
    for c in range(D):
        for t in range(valid):
            r0 = (t // seq_len) * seq_len
            for i in range(rf):
                if t - i >= r0:
                    y[c, t] += float(mu[c, i]) * float(x[c, t - i])
    return y.astype(np.float16)


def test_token_shift_brute_force_and_state():
    rng = np.random.default_rng(2)
    D, seq, req, rf = 5, 7, 3, 4
    valid = seq * req
    x = _f16(rng, (D, 64))
    x[:, valid:] = 0
    mu = _f16(rng, (D, rf))
    y, st = lo.token_shift(x, mu, seq, valid)
    assert np.array_equal(y, _shift_loops(x, mu, seq, valid))
    # an impulse at the first token of request 1 spreads to exactly its next rf-1 tokens
    imp = np.zeros((D, 64), np.float16)
    imp[:, seq] = 1.0
    yi, _ = lo.token_shift(imp, np.ones((D, rf), np.float16), seq, valid)
    assert np.array_equal(np.nonzero(yi[0])[0], np.arange(seq, seq + rf))
    for r in range(req):
        for i in range(rf - 1):
            assert np.array_equal(st[:, i, r], x[:, r * seq + seq - 1 - i])
    assert not st[:, :, req:].any()
    # requests shorter than rf - 1: older slots hold zeros, not the previous request's tokens
    y2, st2 = lo.token_shift(x, mu, 2, 20)
    assert np.array_equal(y2, _shift_loops(x, mu, 2, 20))
    assert np.array_equal(st2[:, 0, 3], x[:, 7]) and np.array_equal(st2[:, 1, 3], x[:, 6])
    assert not st2[:, 2:, :].any()


def test_token_shift_decode_continues_prefill():
    """Prefill of P tokens then one decode step == prefill of P+1 tokens at position P."""
    rng = np.random.default_rng(3)
    D, P, req, rf = 6, 9, 4, 3
    xs = _f16(rng, (D, req, P + 1))
    mu = _f16(rng, (D, rf))
    pre = np.zeros((D, 64), np.float16)
    pre[:, :req * P] = xs[:, :, :P].reshape(D, req * P)
    _, st = lo.token_shift(pre, mu, P, req * P)
    dec = np.zeros((D, 64), np.float16)
    dec[:, :req] = xs[:, :, P]
    yd, st2 = lo.token_shift_decode(dec, mu, st, req)
    full = np.zeros((D, 64), np.float16)
    full[:, :req * (P + 1)] = xs.reshape(D, req * (P + 1))
    yf, stf = lo.token_shift(full, mu, P + 1, req * (P + 1))
    assert np.array_equal(yd[:, :req], yf[:, P::P + 1][:, :req])
    assert np.array_equal(st2[:, :, :req], stf[:, :, :req])


def test_embed_and_argmax():
    rng = np.random.default_rng(4)
    table = _f16(rng, (50, 8))
    ids = np.array([3, 49, 0, 77], dtype=np.int64)  # 77 >= vocab -> zero column
    y = lo.embed(table, ids, 64)
    assert np.array_equal(y[:, 0], table[3]) and np.array_equal(y[:, 1], table[49])
    assert not y[:, 3:].any()
    x = np.zeros((6, 64), np.float16)
    x[2, 0] = x[4, 0] = 1.0  # tie -> lowest index
    x[5, 1] = 0.5
    x[:, 1] -= np.float16(1.0)
    assert list(lo.argmax(x, 2)) == [2, 5]


def test_project_matches_dense_gather():
    rng = np.random.default_rng(5)
    D, T, S, tile, K = 32, 64, 4, 2, 3
    x = _f16(rng, (D, T))
    starts = rng.integers(0, D // S, size=(3, K)) * S
    w = _f16(rng, (6, K * S), 0.3)
    b = _f16(rng, 6, 0.1)
    y = lo.project(x, starts, S, tile, w, b, "none").astype(np.float64)
    for j in range(6):
        rows = (starts[j // tile][:, None] + np.arange(S)[None, :]).ravel()
        ref = w[j].astype(np.float64) @ x[rows].astype(np.float64) + float(b[j])
        assert np.allclose(y[j], ref, rtol=1e-3, atol=1e-3)
    yr = lo.project(x, starts, S, tile, w, b, "relu", res=x[:6]).astype(np.float64)
    assert np.allclose(yr, np.maximum(y, 0) + x[:6].astype(np.float64), atol=4e-3)


TINY = synth.LLMSpec(layers=2, d=256, ffn=384, vocab=640, S=64, requests=2, prompt=32,
                     decode_steps=3, seed=9)


def test_llm_decode_continues_prefill():
    """The decoder has no attention, so decoding token P of each request from the prefill state
    equals a prefill of P+1 tokens, bit for bit in the oracle."""
    wts = synth.llm_weights(TINY)
    rng = np.random.default_rng(6)
    R, P = TINY.requests, TINY.prompt
    toks = rng.integers(0, TINY.vocab, size=(R, P + 1))
    pre = lo.llm_forward(TINY, wts, toks[:, :P].ravel(), decode=False)
    dec = lo.llm_forward(TINY, wts, toks[:, P], decode=True, shift_state=pre.shift_state)
    import dataclasses
    longer = dataclasses.replace(TINY, prompt=P + 1)
    full = lo.llm_forward(longer, wts, toks.ravel(), decode=False)
    assert np.array_equal(dec.tensors["logits"][:, :R], full.tensors["logits"][:, P::P + 1][:, :R])
    assert np.array_equal(dec.ids, full.ids[P::P + 1])


def test_llm_spec_accounting():
    s = synth.LLMSpec()
    kd, kf = s.kept(s.d) * s.S, s.kept(s.ffn) * s.S
    assert (kd, kf) == (1024, 3072)  # 2 of 4 and 6 of 11 clusters of 512
    assert s.nnz_per_token == s.layers * (4 * s.d * kd + 2 * s.ffn * kd + s.d * kf) + s.vocab * kd
    w = synth.llm_weights(TINY)
    for p in w.proj[0].values():
        st = np.sort(p.starts.astype(np.int64), axis=1)
        assert np.all(np.diff(st, axis=1) > 0)  # distinct clusters per neuron
        assert np.all(p.starts % TINY.S == 0)
        assert p.starts.shape[0] == p.weights.shape[0]  # per-neuron patterns
        assert len({tuple(r) for r in st.tolist()}) > 1


@pytest.mark.parametrize("act", [None, "relu", "sigmoid", "silu", "leaky_relu", "gelu"])
@pytest.mark.parametrize("res", [False, True])
def test_project_dense_equals_scalar_oracle(orc, act, res):
    """The dense float64 restatement used by the full-size checks equals the scalar fp64 oracle
    (orc_wave_f64) to float64 rounding, for every activation, with and without residual; a
    shifted cluster start or a dropped bias in the dense form is caught."""
    rng = np.random.default_rng(17 + (act is None) + 2 * res)
    n_cl, S, K, cout, T = 7, 16, 3, 50, 40
    D = n_cl * S
    pick = np.argsort(rng.random((cout, n_cl)), axis=1)[:, :K]
    starts = (pick * S).astype(np.uint32)
    w = _f16(rng, (cout, K * S), 0.2)
    b = _f16(rng, (cout,), 0.3)
    x = _f16(rng, (D, T))
    r = _f16(rng, (cout, T)) if res else None
    want = lo.project(x, starts, S, 1, w, b, act, r, f64=True)
    got = lo.project_dense_f64(x, starts, S, w, b, act, r, block=16)
    assert np.max(np.abs(got - want) / (np.abs(want) + 1e-2)) < 1e-12
    # planted mistakes in the dense form are visible at the tolerance of the device checks
    bad = starts.copy()
    bad[0, 0] = S * next(c for c in range(n_cl) if c not in pick[0])  # another cluster
    moved = lo.project_dense_f64(x, bad, S, w, b, act, r)
    assert orc.rel_err(moved, want) > 2e-3
    no_bias = lo.project_dense_f64(x, starts, S, w, np.zeros_like(b), act, r)
    assert orc.rel_err(no_bias, want) > 2e-3


def test_project_dense_rejects_overlapping_clusters():
    x = np.zeros((64, 8), np.float16)
    starts = np.array([[0, 8]], np.uint32)  # clusters of 16 overlap on rows 8..15
    with pytest.raises(ValueError):
        lo.project_dense_f64(x, starts, 16, np.zeros((1, 32), np.float16), np.zeros(1, np.float16),
                             None)

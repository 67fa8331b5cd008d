"""Pins the CPU oracle (oracle/wave_oracle.c) before anything is checked against it.

Each function is checked against something the mathematics or a published source fixes:
exhaustive fp16 tables vs numpy's IEEE conversion, published FNV-1a-64 and SplitMix64 known
answers, a hand-written WMMA tile layout, an independent numpy float64 evaluation of the wave,
closed-form activation values, and planted mistakes that the tolerance metric must catch.
"""
import math

import numpy as np
import pytest

from snntome_amd import synth


# ------------------------------------------------------------------------------------ fp16
def test_f16_to_f32_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint32)
    ours = np.array([orc.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_roundtrip_every_half(orc):
    """Every finite half survives float -> half exactly (incl. subnormals and +-0)."""
    for b in range(65536):
        h = np.uint16(b).view(np.float16)
        if np.isnan(h):
            continue
        assert orc.f32_to_f16(float(h)) == b


def test_f32_to_f16_rne_random_and_ties(orc):
    rng = np.random.default_rng(0)
    # random f32 bit patterns across the whole range (numpy's conversion is IEEE RNE)
    u = rng.integers(0, 2**32, size=20000, dtype=np.uint64).astype(np.uint32)
    f = u.view(np.float32)
    f = f[~np.isnan(f)]
    with np.errstate(over="ignore"):
        f16 = f.astype(np.float16).view(np.uint16)
    ours = np.array([orc.f32_to_f16(float(x)) for x in f], dtype=np.uint16)
    assert np.array_equal(ours, f16)
    # exact midpoints between consecutive halves round to the even neighbour
    h = np.arange(0x0001, 0x7bff, 97, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)  # representable in f32
    want = np.where(h % 2 == 0, h, h + 1)
    got = np.array([orc.f32_to_f16(float(m)) for m in mid], dtype=np.uint16)
    assert np.array_equal(got, want)


def test_f32_to_f16_special_cases(orc):
    assert orc.f32_to_f16(65504.0) == 0x7BFF
    assert orc.f32_to_f16(65519.99) == 0x7BFF
    assert orc.f32_to_f16(65520.0) == 0x7C00  # ties away from max -> even (Inf)
    assert orc.f32_to_f16(float("inf")) == 0x7C00
    assert orc.f32_to_f16(float("-inf")) == 0xFC00
    assert orc.f32_to_f16(2.0**-25) == 0x0000  # tie between 0 and 2^-24 -> 0
    assert orc.f32_to_f16(2.0**-25 * 1.0000001) == 0x0001
    assert orc.f32_to_f16(-(2.0**-24)) == 0x8001
    assert orc.f32_to_f16(-0.0) == 0x8000
    # NaN rule of k44_plan_types.hpp:40-44: sign | 0x7c00 | (mantissa >> 13) | 1
    for bits in (0x7FC00000, 0x7F800001, 0xFFC12345, 0x7FFFE000):
        want = ((bits >> 16) & 0x8000) | 0x7C00 | ((bits & 0x7FFFFF) >> 13) | 1
        assert orc.f32bits_to_f16(bits) == want


# ------------------------------------------------------------------------------------ hashes
FNV_KAT = {b"": 0xCBF29CE484222325, b"a": 0xAF63DC4C8601EC8C, b"foobar": 0x85944171F73967E8}


def test_fnv1a64_published_answers(orc):
    from oracle import plan_oracle

    for msg, h in FNV_KAT.items():
        assert orc.fnv1a64(msg) == h
        assert plan_oracle.fnv1a64(msg) == h


def test_splitmix64_published_sequence(orc):
    # SplitMix64 seeded with 0: the first three outputs (Vigna's reference generator).
    seq = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    golden = 0x9E3779B97F4A7C15
    for k, want in enumerate(seq):
        state = (k * golden) & 0xFFFFFFFFFFFFFFFF
        assert orc.splitmix64(state) == want
        assert int(synth.splitmix64(np.uint64(state))) == want


def test_substrate_generator_host_paths_agree(orc):
    """numpy generator (product) == C generator (oracle), bit for bit, incl. padding tokens."""
    rng = np.random.default_rng(1)
    pos = rng.integers(0, 40_000_000, size=64)
    x = synth.substrate_rows(123, pos, 64, valid=50).view(np.uint16)
    for i, p in enumerate(pos[:16]):
        for t in (0, 1, 31, 49):
            assert x[i, t] == orc.substrate_f16(123, int(p), t)
    assert not x[:, 50:].any()
    vals = x[:, :50].view(np.float16).astype(np.float32)
    assert vals.min() >= -1.0 and vals.max() <= 1.0
    assert abs(vals.mean()) < 0.05 and 0.5 < vals.std() * math.sqrt(3) < 1.1
    comp = orc.fill_segments(123, pos[:4], 3, 50, 64)
    for i in range(4):
        for s in range(3):
            assert np.array_equal(comp[i * 3 + s], synth.substrate_rows(123, [pos[i] + s], 64,
                                                                        valid=50).view(np.uint16)[0])


# ------------------------------------------------------------------------------------ WMMA order
def test_wmma_order_hand_example(orc):
    """Cout=16, B=64: vector g holds row (g % 32) & 15, columns 16*(g//32) + 8*((g%32)>>4)."""
    cout, B = 16, 64
    w = (np.arange(cout)[:, None] * 100 + np.arange(B)[None, :]).astype(np.uint16)
    vec = orc.raw_to_wmma(w).reshape(-1, 8)
    assert list(vec[0]) == list(range(0, 8))          # row 0, cols 0..7
    assert list(vec[1]) == list(range(100, 108))      # row 1, cols 0..7
    assert list(vec[15]) == list(range(1500, 1508))   # row 15, cols 0..7
    assert list(vec[16]) == list(range(8, 16))        # row 0, cols 8..15 (upper half-lanes)
    assert list(vec[31]) == list(range(1508, 1516))   # row 15, cols 8..15
    assert list(vec[32]) == list(range(16, 24))       # next K tile: row 0, cols 16..23
    assert list(vec[127]) == list(range(1556, 1564))  # last tile: row 15, cols 56..63


def test_wmma_order_is_a_bijection(orc):
    rng = np.random.default_rng(3)
    for cout, B in ((16, 64), (48, 96), (128, 512)):
        w = rng.integers(0, 65535, size=(cout, B), dtype=np.uint16)
        iw = orc.raw_to_wmma(w)
        assert np.array_equal(np.sort(iw.ravel()), np.sort(w.ravel()))
        assert np.array_equal(orc.wmma_to_raw(iw, cout, B), w)


# ------------------------------------------------------------------------------------ activations
def test_activation_closed_forms(orc):
    a = orc.lib().orc_act
    assert a(-1.5, 1) == 0.0 and a(2.5, 1) == 2.5
    assert a(0.0, 2) == 0.5 and abs(a(2.0, 2) - 1 / (1 + math.exp(-2))) < 1e-15
    assert a(0.0, 3) == 0.0 and abs(a(1.0, 3) - 1 / (1 + math.exp(-1))) < 1e-15
    assert a(-2.0, 4) == pytest.approx(-0.2) and a(3.0, 4) == 3.0
    assert a(0.0, 5) == 0.0
    assert a(1.0, 5) == pytest.approx(0.8413447460685429, abs=1e-15)  # Phi(1)
    assert a(-1.0, 5) == pytest.approx(-0.15865525393145707, abs=1e-15)
    assert a(30.0, 5) == 30.0 and abs(a(-30.0, 5)) < 1e-100
    assert a(7.0, 0) == 7.0


# ------------------------------------------------------------------------------------ wave oracle
def _np_wave(x, seg, w, bias, K, S, cluster, step, tokens, act, resid=None, cmap=None):
    """Independent evaluation: explicit numpy gather + float64 matmul."""
    xf = x.view(np.float16).astype(np.float64)
    cout = w.shape[0]
    W = w.view(np.float16).astype(np.float64)
    out = np.empty((cout, tokens))
    for j in range(cout):
        rows = np.concatenate([seg[(j // cluster) * K + k] + step * np.arange(S)
                               for k in range(K)]).astype(np.int64)
        G = xf[rows[:, None] + np.arange(tokens)[None, :]]
        v = W[j] @ G + (0 if bias is None else float(bias.view(np.float16)[j]))
        r = 0.0 if resid is None else resid[j]
        f = {0: lambda z: z, 1: lambda z: np.maximum(z, 0), 2: lambda z: 1 / (1 + np.exp(-z)),
             3: lambda z: z / (1 + np.exp(-z)), 4: lambda z: np.where(z > 0.1 * z, z, 0.1 * z),
             5: lambda z: 0.5 * z * (1 + np.vectorize(math.erf)(z / math.sqrt(2)))}[act]
        out[j] = f(v + r) if cmap is not None else f(v) + r
    return out


@pytest.mark.parametrize("act", [0, 1, 2, 3, 4, 5])
def test_wave_f64_matches_numpy(orc, act):
    rng = np.random.default_rng(act)
    C, tokens, cout, K, S, cl = 300, 40, 12, 3, 5, 2
    stride = 64
    x = synth.substrate_rows(9, np.arange(C), stride, valid=tokens).view(np.uint16).ravel()
    seg = (rng.integers(0, C - S, size=(cout // cl) * K) * stride).astype(np.uint64)
    w = synth.normal_f16(rng, (cout, K * S), 0.3)
    b = synth.normal_f16(rng, (cout,), 0.3)
    got = orc.wave_f64(x, seg, w, b, None, K, S, cl, stride, tokens, stride, act)
    want = _np_wave(x, seg, w, b, K, S, cl, stride, tokens, act)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_wave_f64_residual_and_cmap_epilogues(orc):
    rng = np.random.default_rng(5)
    C, tokens, cout, K, S = 200, 64, 8, 2, 4
    stride = 64
    x = synth.substrate_rows(2, np.arange(C), stride).view(np.uint16).ravel()
    seg = (rng.integers(0, C - S, size=cout * K) * stride).astype(np.uint64)
    w = synth.normal_f16(rng, (cout, K * S), 0.5)
    b = synth.normal_f16(rng, (cout,), 0.5)
    res_off = 50 * stride  # residual = substrate channels 50.. (as a canvas region)
    resid = x.view(np.float16).astype(np.float64)[res_off:res_off + cout * stride]
    resid = resid.reshape(cout, stride)[:, :tokens]
    # no cout_map: y = act(v) + r
    got = orc.wave_f64(x, seg, w, b, None, K, S, 1, stride, tokens, stride, 3, res_off=res_off)
    assert np.allclose(got, _np_wave(x, seg, w, b, K, S, 1, stride, tokens, 3, resid=resid))
    # with cout_map: y = act(v + r[cmap[j]]), residual read at the remapped channel
    cmap = rng.permutation(cout).astype(np.uint16)
    got = orc.wave_f64(x, seg, w, b, cmap, K, S, 1, stride, tokens, stride, 3, res_off=res_off)
    want = _np_wave(x, seg, w, b, K, S, 1, stride, tokens, 3, resid=resid[cmap], cmap=cmap)
    assert np.allclose(got, want)


def test_wave_f32_omp_within_tolerance(orc):
    rng = np.random.default_rng(8)
    C, tokens, cout, K, S = 4096, 256, 64, 4, 16
    stride = 256
    x = synth.substrate_rows(4, np.arange(C), stride).view(np.uint16).ravel()
    seg = (rng.integers(0, C - S, size=cout * K) * stride).astype(np.uint64)
    w = synth.normal_f16(rng, (cout, K * S), 0.05)
    b = synth.normal_f16(rng, (cout,), 0.01)
    canvas = np.concatenate([x, np.zeros(cout * stride, np.uint16)])
    orc.wave_f32_omp(canvas, seg, w, b, None, K, S, 1, stride, tokens, stride, 1, y_off=x.size)
    y = canvas[x.size:].view(np.float16).astype(np.float64).reshape(cout, stride)
    ref = orc.wave_f64(x, seg, w, b, None, K, S, 1, stride, tokens, stride, 1)
    assert orc.rel_err(y, ref) <= 2e-3


def test_tolerance_catches_planted_mistakes(orc):
    """A dropped segment, a wrong segment start, a transposed (reversed) synapse order or a
    missing bias must each violate the 2e-3 bound — the metric is not vacuous."""
    rng = np.random.default_rng(11)
    C, tokens, cout, K, S = 2048, 64, 32, 4, 16
    stride = 64
    x = synth.substrate_rows(6, np.arange(C), stride).view(np.uint16).ravel()
    seg = (rng.integers(0, C - S, size=cout * K) * stride).astype(np.uint64)
    w = synth.normal_f16(rng, (cout, K * S), 0.05)
    b = synth.normal_f16(rng, (cout,), 0.01)
    ref = orc.wave_f64(x, seg, w, b, None, K, S, 1, stride, tokens, stride, 0)
    dropped = orc.wave_f64(x, seg, w[:, : (K - 1) * S].copy(), b, None, K - 1, S, 1, stride,
                           tokens, stride, 0)
    seg2 = seg.copy()
    seg2[0] += stride
    shifted = orc.wave_f64(x, seg2, w, b, None, K, S, 1, stride, tokens, stride, 0)
    reversed_w = orc.wave_f64(x, seg, w[:, ::-1].copy(), b, None, K, S, 1, stride, tokens,
                              stride, 0)
    no_bias = orc.wave_f64(x, seg, w, None, None, K, S, 1, stride, tokens, stride, 0)
    for bad in (dropped, shifted, reversed_w, no_bias):
        assert orc.rel_err(bad, ref) > 2e-3

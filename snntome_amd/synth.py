"""Synthetic workloads of the wave hot path (the configurations the benchmark and tests use).

Every generator is seeded and deterministic.  The substrate generator is counter based, so any
position row can be produced on its own, on the host (numpy, here) or on the device
(wavec_gpu_fill_input_uniform), with bit-identical fp16 values:
    x(pos, t) = fp16_rne((int32(h >> 40) - 2^23) * 2^-23),
    h = splitmix64(((pos << 20) | t) ^ splitmix64(seed))
Weights and biases are normal draws from numpy's PCG64 generator, rounded to fp16 (RNE).
"""

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(x) -> np.ndarray:
    """SplitMix64 output for state x (vectorised, wrapping uint64 arithmetic)."""
    with np.errstate(over="ignore"):
        z = np.asarray(x, dtype=np.uint64) + _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def substrate_rows(seed: int, positions, tokens: int, valid: Optional[int] = None) -> np.ndarray:
    """fp16 rows [len(positions), tokens] of the synthetic substrate (tokens >= valid are 0)."""
    pos = np.asarray(positions, dtype=np.uint64).reshape(-1, 1)
    t = np.arange(tokens, dtype=np.uint64).reshape(1, -1)
    with np.errstate(over="ignore"):
        mix = splitmix64(np.uint64(seed))
        h = splitmix64(((pos << np.uint64(20)) | t) ^ mix)
    q = (h >> np.uint64(40)).astype(np.int64) - (1 << 23)
    x = (q.astype(np.float32) * np.float32(1.0 / 8388608.0)).astype(np.float16)
    if valid is not None and valid < tokens:
        x[:, valid:] = 0
    return x


def normal_f16(rng: np.random.Generator, shape, sigma: float) -> np.ndarray:
    return (rng.standard_normal(shape, dtype=np.float64) * sigma).astype(np.float16)


@dataclass
class WaveSpec:
    """One wave: neuron j reads K segments of S consecutive substrate positions."""
    name: str
    cout: int
    K: int
    S: int
    cluster: int
    starts: np.ndarray  # [cout/cluster, K] uint32, positions in the wave's input tensor
    weights: np.ndarray  # [cout, K*S] fp16
    bias: np.ndarray  # [cout] fp16
    act: str
    sources: List[str] = field(default_factory=list)  # input tensor(s) (concatenated)

    @property
    def nnz(self) -> int:
        return self.cout * self.K * self.S


@dataclass
class Workload:
    name: str
    substrate: int  # positions of the plan input
    tokens: int  # batch (tokens per position)
    seed: int  # substrate seed
    waves: List[WaveSpec]
    description: str = ""

    @property
    def flops(self) -> float:
        return float(sum(2 * w.nnz * self.tokens for w in self.waves))


def _aligned_starts(rng, n, hi_exclusive, align):
    """Uniform random starts in {0, align, 2 align, ...} below hi_exclusive."""
    slots = hi_exclusive // align
    return (rng.integers(0, slots, size=n, dtype=np.int64) * align).astype(np.uint32)


def config1(seed: int = 1) -> Workload:
    """Single wave, plumbing: substrate 65,536 x batch 64; 4,096 neurons x 8 clusters of S=64,
    8-aligned uniform starts; W ~ N(0, 0.02), b ~ N(0, 0.01), ReLU."""
    rng = np.random.default_rng(seed)
    C, N, K, S = 65536, 4096, 8, 64
    st = _aligned_starts(rng, N * K, C - S + 1, 8).reshape(N, K)
    w = normal_f16(rng, (N, K * S), 0.02)
    b = normal_f16(rng, (N,), 0.01)
    return Workload("c1_plumbing", C, 64, seed + 100,
                    [WaveSpec("wave0", N, K, S, 1, st, w, b, "relu", ["x"])],
                    "65,536 x 64 substrate; 4,096 neurons x 8 clusters x S=64; ReLU")


def config2(seed: int = 2, neurons: int = 65536, substrate: int = 40_000_000) -> Workload:
    """Ultra-sparse gather-bound wave: substrate 40,000,000 x batch 256; 65,536 neurons x 4
    clusters of S=16, 16-aligned uniform starts; W ~ N(0, 0.05), b ~ N(0, 0.01), ReLU."""
    rng = np.random.default_rng(seed)
    K, S = 4, 16
    st = _aligned_starts(rng, neurons * K, substrate - S + 1, 16).reshape(neurons, K)
    w = normal_f16(rng, (neurons, K * S), 0.05)
    b = normal_f16(rng, (neurons,), 0.01)
    return Workload("c2_ultra_sparse", substrate, 256, seed + 100,
                    [WaveSpec("wave0", neurons, K, S, 1, st, w, b, "relu", ["x"])],
                    f"{substrate:,} x 256 substrate; {neurons:,} neurons x 4 clusters x S=16; ReLU")


def config3(seed: int = 3, neurons: int = 16384, substrate: int = 1 << 20,
            tokens: int = 512) -> Workload:
    """Dense-cluster wave: substrate 1,048,576 x batch 512; 16,384 neurons x 16 clusters of
    S=512; tiles of 64 neurons share 64-aligned starts; W ~ N(0, 0.02), b ~ N(0, 0.01), GELU."""
    rng = np.random.default_rng(seed)
    K, S, T = 16, 512, 64
    st = _aligned_starts(rng, (neurons // T) * K, substrate - S + 1, 64).reshape(neurons // T, K)
    w = normal_f16(rng, (neurons, K * S), 0.02)
    b = normal_f16(rng, (neurons,), 0.01)
    return Workload("c3_dense_cluster", substrate, tokens, seed + 100,
                    [WaveSpec("wave0", neurons, K, S, T, st, w, b, "gelu", ["x"])],
                    f"{substrate:,} x {tokens} substrate; {neurons:,} neurons x 16 x S=512, "
                    "64-neuron shared tiles; GELU")


def config4(seed: int = 4, waves: int = 8, width: int = 32768, neurons: int = 4096,
            K: int = 16, S: int = 128, tokens: int = 128) -> Workload:
    """Multi-wave plan: 8 waves over a 32,768-wide input, 4,096 neurons each, 16 clusters of
    S=128 per neuron: 8 clusters from the immediately preceding tensor (the input for wave 0)
    and 8 uniform over all earlier tensors (input + previous waves, chosen proportional to
    width); starts 8-aligned inside the chosen tensor so no cluster straddles two tensors.
    W ~ N(0, 0.02), b ~ N(0, 0.01), ReLU, batch 128."""
    rng = np.random.default_rng(seed)
    names = ["x"] + [f"y{i}" for i in range(waves)]
    widths = [width] + [neurons] * waves
    offs = np.concatenate([[0], np.cumsum(widths)]).astype(np.int64)
    specs = []
    half = K // 2
    for i in range(waves):
        srcs = names[: i + 1]  # wave i reads the concatenation [x, y0 .. y(i-1)]
        prev = i  # index of the immediately preceding tensor in srcs
        st = np.empty((neurons, K), dtype=np.uint32)
        st[:, :half] = offs[prev] + _aligned_starts(rng, neurons * half, widths[prev] - S + 1,
                                                    8).reshape(neurons, half)
        p = np.asarray(widths[: i + 1], dtype=np.float64)
        pick = rng.choice(i + 1, size=(neurons, K - half), p=p / p.sum())
        for t in range(i + 1):
            m = pick == t
            st[:, half:][m] = offs[t] + _aligned_starts(rng, int(m.sum()), widths[t] - S + 1, 8)
        w = normal_f16(rng, (neurons, K * S), 0.02)
        b = normal_f16(rng, (neurons,), 0.01)
        specs.append(WaveSpec(f"wave{i}", neurons, K, S, 1, st, w, b, "relu", srcs))
    return Workload("c4_multi_wave", width, tokens, seed + 100, specs,
                    f"{waves}-wave plan over a {width:,}-wide input; {neurons} neurons/wave x "
                    f"{K} x S={S}; batch {tokens}; ReLU")


def build_graph(wl: Workload, wavec_mod=None, kv_cache_max_seq: int = 0):
    """WaveGraph for a workload: 1-D input 'x' [substrate, tokens]; wave i writes 'y{i}'."""
    if wavec_mod is None:
        from . import wavec as wavec_mod
    g = wavec_mod.WaveGraph(kv_cache_max_seq=kv_cache_max_seq)
    g.add_input("x", wl.substrate, 1, wl.tokens, is_1d=True)
    for i, w in enumerate(wl.waves):
        src = w.sources[0] if len(w.sources) == 1 else f"cat{i}"
        if len(w.sources) > 1:
            g.add_concat(f"cat{i}", w.sources, src)
        g.add_cluster_wave(w.name, src, f"y{i}", w.starts, w.S, w.weights, w.bias,
                           cluster=w.cluster, act=w.act)
    g.set_output(f"y{len(wl.waves) - 1}")
    return g


def distinct_positions(starts: np.ndarray, S: int) -> int:
    """Number of distinct substrate positions covered by [start, start + S) segments."""
    s = np.sort(np.asarray(starts, dtype=np.int64).ravel())
    if s.size == 0:
        return 0
    ends = s + S
    run_end = np.maximum.accumulate(ends)
    new = np.ones_like(s, dtype=bool)
    new[1:] = s[1:] >= run_end[:-1]
    # covered = sum over merged runs of (end - start)
    idx = np.flatnonzero(new)
    run_starts = s[idx]
    run_ends = np.append(run_end[idx[1:] - 1], run_end[-1])
    return int(np.sum(run_ends - run_starts))


def compulsory_bytes(wl: Workload, wave: WaveSpec) -> int:
    """Algorithmic HBM bytes of one wave: distinct substrate rows x tokens x 2 + weights
    (2 B/synapse) + segment starts (4 B each) + bias (2 B) + outputs (2 B x tokens)."""
    u = distinct_positions(wave.starts, wave.S)
    return (2 * wl.tokens * u + 2 * wave.nnz + 4 * wave.starts.size + 2 * wave.cout
            + 2 * wave.cout * wl.tokens)


# ---------------------------------------------------------------------------------------------
# Config 5: LLM-shaped compiled decoder
# ---------------------------------------------------------------------------------------------
@dataclass
class LLMSpec:
    """LLM-shaped decoder compiled to waves.  Per layer (x: [d][tokens], fp16 canvas tensors):
        u = RMSNorm(x);  s = TokenShift_rf(u)        (causal, per request; carried state in decode)
        q = sigmoid(Wq s);  k = silu(Wk s);  v = Wv s;  m = q * (k * v)
        x = x + Wo m
        n = RMSNorm(x);  h = silu(Wg n) * (Wu n);  x = x + Wd h
    then logits = Whead RMSNorm(x), next id = argmax.  Every projection is a pruned wave: its
    input row is cut into clusters of S consecutive channels and every neuron keeps its own
    random `keep` fraction of them (2 of 4 for d-wide inputs, 6 of 11 for FFN-wide inputs at the
    default sizes); the compiler groups neurons into pattern-sorted tiles of `tile` for MFMA.
    RMSNorm gamma = 1."""
    layers: int = 16
    d: int = 2048
    ffn: int = 5632
    vocab: int = 32000
    S: int = 512
    keep: float = 0.5
    tile: int = 64
    rf: int = 4
    requests: int = 16
    prompt: int = 512
    decode_steps: int = 128
    seed: int = 5

    def kept(self, fan: int) -> int:
        n = fan // self.S
        return max(1, int(np.ceil(n * self.keep - 1e-9)))

    @property
    def nnz_per_token(self) -> int:
        kd, kf = self.kept(self.d) * self.S, self.kept(self.ffn) * self.S
        per_layer = 4 * self.d * kd + 2 * self.ffn * kd + self.d * kf
        return self.layers * per_layer + self.vocab * kd


@dataclass
class Projection:
    starts: np.ndarray  # [cout, K] uint32 first input channel of each cluster neuron j keeps
    weights: np.ndarray  # [cout, K*S] fp16
    bias: np.ndarray  # [cout] fp16


def _projection(rng, spec: LLMSpec, fan_in: int, cout: int) -> Projection:
    n_cl = fan_in // spec.S
    K = spec.kept(fan_in)
    pick = np.argsort(rng.random((cout, n_cl)), axis=1)[:, :K]  # K distinct clusters per neuron
    starts = (pick * spec.S).astype(np.uint32)  # random order: the compiler sorts them
    sigma = 1.0 / np.sqrt(K * spec.S)
    w = (rng.standard_normal((cout, K * spec.S), dtype=np.float32) * np.float32(sigma)).astype(
        np.float16)
    b = (rng.standard_normal(cout, dtype=np.float32) * np.float32(0.01)).astype(np.float16)
    return Projection(starts, w, b)


@dataclass
class LLMWeights:
    embed: np.ndarray  # [vocab, d] fp16
    mix: List[np.ndarray]  # per layer [d, rf] fp16 (rows sum to ~1)
    proj: List[dict]  # per layer {"q","k","v","o","g","u","dn"} -> Projection
    head: Projection


def llm_weights(spec: LLMSpec) -> LLMWeights:
    rng = np.random.default_rng(spec.seed)
    embed = rng.standard_normal((spec.vocab, spec.d), dtype=np.float32).astype(np.float16)
    mix, proj = [], []
    for _ in range(spec.layers):
        m = rng.random((spec.d, spec.rf), dtype=np.float32) + np.float32(0.05)
        m[:, 0] += np.float32(spec.rf)  # the current token dominates the mix
        mix.append((m / m.sum(axis=1, keepdims=True)).astype(np.float16))
        p = {}
        for name in ("q", "k", "v", "o"):
            p[name] = _projection(rng, spec, spec.d, spec.d)
        p["g"] = _projection(rng, spec, spec.d, spec.ffn)
        p["u"] = _projection(rng, spec, spec.d, spec.ffn)
        p["dn"] = _projection(rng, spec, spec.ffn, spec.d)
        proj.append(p)
    head = _projection(rng, spec, spec.d, spec.vocab)
    return LLMWeights(embed, mix, proj, head)


def build_llm_graph(spec: LLMSpec, wts: LLMWeights, decode: bool, wavec_mod=None):
    """Prefill (decode=False: requests x prompt tokens) or decode (one token per request)."""
    if wavec_mod is None:
        from . import wavec as wavec_mod
    T = spec.requests if decode else spec.requests * spec.prompt
    seq = 1 if decode else spec.prompt
    g = wavec_mod.WaveGraph(kv_cache_max_seq=0, fold_rmsnorm_gamma=True)
    g.add_input("tok", 1, 1, T, is_1d=True)
    g.add_embedding("embed", "tok", "x0", wts.embed)
    ones = np.ones(spec.d, np.float32)

    def proj(name, src, out, p: Projection, act=None, res=None):
        g.add_pruned_wave(name, src, out, p.starts, spec.S, p.weights, p.bias, tile=spec.tile,
                          act=act, res_blob=res)

    x = "x0"
    for l in range(spec.layers):
        P = wts.proj[l]
        g.add_rmsnorm(f"l{l}.n1", x, f"l{l}.u", spec.d, ones)
        g.add_token_shift(f"l{l}.shift", f"l{l}.u", f"l{l}.s", wts.mix[l], seq, decode=decode)
        proj(f"l{l}.q", f"l{l}.s", f"l{l}.q", P["q"], act="sigmoid")
        proj(f"l{l}.k", f"l{l}.s", f"l{l}.k", P["k"], act="silu")
        proj(f"l{l}.v", f"l{l}.s", f"l{l}.v", P["v"])
        g.add_swiglu(f"l{l}.kv", f"l{l}.k", f"l{l}.v", f"l{l}.kv")
        g.add_swiglu(f"l{l}.m", f"l{l}.q", f"l{l}.kv", f"l{l}.m")
        proj(f"l{l}.o", f"l{l}.m", f"l{l}.x1", P["o"], res=x)
        g.add_rmsnorm(f"l{l}.n2", f"l{l}.x1", f"l{l}.n", spec.d, ones)
        proj(f"l{l}.g", f"l{l}.n", f"l{l}.g", P["g"], act="silu")
        proj(f"l{l}.u", f"l{l}.n", f"l{l}.up", P["u"])
        g.add_swiglu(f"l{l}.h", f"l{l}.g", f"l{l}.up", f"l{l}.h")
        proj(f"l{l}.dn", f"l{l}.h", f"l{l}.x2", P["dn"], res=f"l{l}.x1")
        x = f"l{l}.x2"
    g.add_rmsnorm("final.n", x, "z", spec.d, ones)
    proj("head", "z", "logits", wts.head)
    g.add_argmax("argmax", "logits", "next")
    g.set_output("logits")
    return g


def llm_handoff(spec: LLMSpec, prefill, decode) -> None:
    """Device-side hand-over from a finished prefill plan to the decode plan: every layer's
    token-shift state block, and the argmax id of each request's last prompt token as the
    first decode input."""
    pre = {c["name"]: c for c in prefill.cmds if c["type"] == "TOKEN_SHIFT_1D"}
    n = spec.d * (spec.rf - 1) * 64
    for c in decode.cmds:
        if c["type"] != "TOKEN_SHIFT_1D":
            continue
        decode.copy_canvas_from(prefill, int(c["state_off"]), int(pre[c["name"]]["state_off"]), n)
    decode.copy_ids_from(prefill, 0, spec.prompt - 1, spec.prompt, spec.requests)

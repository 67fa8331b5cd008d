"""CPU restatement of the 1-D token ops and of the LLM-shaped decoder — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module, as the
checker.  Every tensor is channel-major fp16 [channels, tokens] (the canvas layout); every
function computes in float64 and rounds once to fp16 (round to nearest even) where the device
stores a tensor (f64=True / *_f64 return the value before that rounding), so the device differs from it only by fp32 arithmetic and single roundings.

Reference citations:
  rmsnorm   kernels/common/kernel44_valu_pack.cuh:104-134 (k44_valu_rmsnorm_tile64_f16_kernel):
            y = x * rsqrt(sum_c x^2 / D + eps) * gamma
  mul       kernels/common/kernel44_valu_pack.cuh:135-143 (k44_valu_swiglu_tile64_f16_kernel):
            y = gate * up (SiLU fused into the gate projection's epilogue,
            wavec/k44_wave_compiler.hpp:1024-1049 emits SWIGLU_MUL_1D after it)
  project   the K44 wave of wave_oracle.c (orc_wave_f64) on a compact canvas
  project_dense_f64
            the same projection as one float64 matrix product (for full-size checks, where the
            scalar orc_wave_f64 is too slow); pinned against `project` in tests/test_llm_oracle.py
  token_shift, embed, argmax: build extensions with no reference counterpart; pinned in
            tests/test_llm_oracle.py against brute-force loops and closed forms.
"""
from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

from . import oracle as orc
from .cnn_oracle import act as act_f64

F16 = np.float16


def rmsnorm_f64(x: np.ndarray, gamma: Optional[np.ndarray] = None,
                eps: float = 1e-5) -> np.ndarray:
    """x: [D, T] fp16 -> float64 before the store (reference kernel44_valu_pack.cuh:104-134)."""
    xf = x.astype(np.float64)
    inv = 1.0 / np.sqrt((xf * xf).sum(axis=0) / x.shape[0] + np.float64(np.float32(eps)))
    g = np.ones(x.shape[0]) if gamma is None else gamma.astype(np.float64)
    return xf * inv[None, :] * g[:, None]


def rmsnorm(x: np.ndarray, gamma: Optional[np.ndarray] = None, eps: float = 1e-5) -> np.ndarray:
    return rmsnorm_f64(x, gamma, eps).astype(F16)


def mul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Element-wise product (reference kernel44_valu_pack.cuh:135-143)."""
    return (a.astype(np.float64) * b.astype(np.float64)).astype(F16)


def token_shift(x: np.ndarray, mu: np.ndarray, seq_len: int, valid: int, f64: bool = False):
    """Prefill: y[c][t] = sum_{i<rf, i<=pos} mu[c][i] * x[c][t-i], pos = t % seq_len, for the
    first `valid` tokens (requests of seq_len tokens; padding columns y = 0).  Returns (y, state)
    with state [D, rf-1, 64]: state[c][i][r] = x[c][r*seq_len + seq_len-1-i] (the newest rf-1
    inputs of request r, newest first) for i < seq_len; all other entries are 0."""
    D, T = x.shape
    rf = mu.shape[1]
    xf = x.astype(np.float64)
    m = mu.astype(np.float64)
    y = np.zeros((D, T), dtype=np.float64)
    if valid % seq_len == 0:  # whole requests: tap i shifts every request by i tokens
        R = valid // seq_len
        xr = xf[:, :valid].reshape(D, R, seq_len)
        yr = y[:, :valid].reshape(D, R, seq_len)
        for i in range(min(rf, seq_len)):
            yr[:, :, i:] += m[:, i, None, None] * xr[:, :, :seq_len - i]
    else:
        t = np.arange(valid)
        pos = t % seq_len
        for i in range(rf):
            ok = pos >= i
            y[:, t[ok]] += m[:, i:i + 1] * xf[:, t[ok] - i]
    state = np.zeros((D, max(rf - 1, 0), 64), dtype=F16)
    for r in range(valid // seq_len):
        for i in range(min(rf - 1, seq_len)):  # slots before the request start stay 0
            state[:, i, r] = x[:, r * seq_len + seq_len - 1 - i]
    return (y if f64 else y.astype(F16)), state


def token_shift_decode(x: np.ndarray, mu: np.ndarray, state: np.ndarray, valid: int,
                       f64: bool = False):
    """Decode: token t is request t; y = mu[:,0]*x + sum_{i>=1} mu[:,i]*state[:,i-1,t]; the
    returned state has x as newest entry and the older entries moved one place back."""
    D, T = x.shape
    rf = mu.shape[1]
    m = mu.astype(np.float64)
    y = np.zeros((D, T), dtype=np.float64)
    y[:, :valid] = m[:, :1] * x[:, :valid].astype(np.float64)
    for i in range(1, rf):
        y[:, :valid] += m[:, i:i + 1] * state[:, i - 1, :valid].astype(np.float64)
    new = state.copy()
    if rf > 1:
        new[:, 1:, :valid] = state[:, :-1, :valid]
        new[:, 0, :valid] = x[:, :valid]
    return (y if f64 else y.astype(F16)), new


def embed(table: np.ndarray, ids: np.ndarray, stride: int) -> np.ndarray:
    """y[c][t] = table[ids[t]][c]; ids >= vocab and padding tokens give 0."""
    V, D = table.shape
    y = np.zeros((D, stride), dtype=F16)
    for t, i in enumerate(ids):
        if i < V:
            y[:, t] = table[i]
    return y


def argmax(x: np.ndarray, valid: int) -> np.ndarray:
    """Lowest channel index of the maximum of every valid token column (fp16 compare)."""
    return np.argmax(x[:, :valid].astype(np.float32), axis=0).astype(np.uint32)


def project(x: np.ndarray, starts: np.ndarray, S: int, tile: int, w: np.ndarray, b: np.ndarray,
            act, res: Optional[np.ndarray] = None, f64: bool = False) -> np.ndarray:
    """Dendritic-cluster projection through orc_wave_f64: neuron j of tile j//tile sums
    w[j][k*S+s] * x[starts[j//tile][k] + s][t]; y = fp16(act(v) [+ res])."""
    D, T = x.shape
    canvas = x.view(np.uint16).ravel()
    res_off = None
    if res is not None:
        canvas = np.concatenate([canvas, res.view(np.uint16).ravel()])
        res_off = x.size
    K = starts.shape[1]
    seg = (starts.astype(np.uint64) * np.uint64(T)).ravel()
    out = orc.wave_f64(canvas, seg, w, b, None, K, S, tile, T, T, T, act, res_off=res_off)
    return out if f64 else out.astype(F16)


def project_dense_f64(x: np.ndarray, starts: np.ndarray, S: int, w: np.ndarray, b: np.ndarray,
                      act, res: Optional[np.ndarray] = None, block: int = 4096) -> np.ndarray:
    """`project` with per-neuron clusters (tile 1), before the fp16 store, computed as one float64
    matrix product: neuron j's K disjoint clusters are scattered into row j of a dense [cout, D]
    weight matrix, v = W x + b, y = act(v) [+ res].  Rows are processed in blocks of `block`."""
    D, T = x.shape
    cout, K = starts.shape
    cols = (starts.astype(np.int64)[:, :, None] + np.arange(S, dtype=np.int64)).reshape(cout, K * S)
    if cols.size and cols.max() >= D:
        raise ValueError("a cluster reaches past the input rows")
    srt = np.sort(cols, axis=1)
    if np.any(srt[:, 1:] == srt[:, :-1]):
        raise ValueError("a neuron reads one input row twice (clusters overlap)")
    xf = x.astype(np.float64)
    out = np.empty((cout, T), dtype=np.float64)
    for r0 in range(0, cout, block):
        r1 = min(cout, r0 + block)
        Wd = np.zeros((r1 - r0, D), dtype=np.float64)
        np.put_along_axis(Wd, cols[r0:r1], w[r0:r1].astype(np.float64), axis=1)
        v = Wd @ xf + b[r0:r1].astype(np.float64)[:, None]
        y = act_f64(v, act)
        if res is not None:
            y = y + res[r0:r1].astype(np.float64)
        out[r0:r1] = y
    return out


@dataclass
class LLMState:
    tensors: Dict[str, np.ndarray]  # name -> [C, stride] fp16 (every op output of one run)
    shift_state: List[np.ndarray]  # per layer [d, rf-1, 64] fp16
    ids: np.ndarray  # argmax of the last tensor, [valid] uint32


def llm_forward(spec, wts, tok_ids: np.ndarray, decode: bool,
                shift_state: Optional[List[np.ndarray]] = None) -> LLMState:
    """One run of the decoder built by snntome_amd.synth.build_llm_graph (same op order and
    tensor names) on token ids `tok_ids` (prefill: requests*prompt ids, request-major)."""
    valid = len(tok_ids)
    T = (valid + 63) // 64 * 64
    seq = 1 if decode else spec.prompt
    ts: Dict[str, np.ndarray] = {}
    x = embed(wts.embed, np.asarray(tok_ids, dtype=np.int64), T)
    ts["x0"] = x
    states = []

    def proj(p, src, act=None, res=None):  # per-neuron clusters: index row = neuron
        return project(src, p.starts, spec.S, 1, p.weights, p.bias, act, res)

    for l in range(spec.layers):
        P = wts.proj[l]
        u = rmsnorm(x)
        if decode:
            s, st = token_shift_decode(u, wts.mix[l], shift_state[l], valid)
        else:
            s, st = token_shift(u, wts.mix[l], seq, valid)
        states.append(st)
        q = proj(P["q"], s, "sigmoid")
        k = proj(P["k"], s, "silu")
        v = proj(P["v"], s)
        kv = mul(k, v)
        m = mul(q, kv)
        x1 = proj(P["o"], m, res=x)
        n = rmsnorm(x1)
        g = proj(P["g"], n, "silu")
        up = proj(P["u"], n)
        h = mul(g, up)
        x2 = proj(P["dn"], h, res=x1)
        ts.update({f"l{l}.u": u, f"l{l}.s": s, f"l{l}.q": q, f"l{l}.k": k, f"l{l}.v": v,
                   f"l{l}.kv": kv, f"l{l}.m": m, f"l{l}.x1": x1, f"l{l}.n": n, f"l{l}.g": g,
                   f"l{l}.up": up, f"l{l}.h": h, f"l{l}.x2": x2})
        x = x2
    z = rmsnorm(x)
    logits = proj(wts.head, z)
    ts["z"] = z
    ts["logits"] = logits
    return LLMState(ts, states, argmax(logits, valid))

"""ctypes binding of the C oracle (wave_oracle.c) — TEST INFRASTRUCTURE ONLY.

Functions mirror wave_oracle.c; see that file for the reference citations of each.
"""
import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_dp = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32bits_to_f16.restype = ctypes.c_uint16
        L.orc_f32bits_to_f16.argtypes = [ctypes.c_uint32]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_bf16_to_f32.restype = ctypes.c_float
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_fnv1a64.restype = ctypes.c_uint64
        L.orc_fnv1a64.argtypes = [_u8p, ctypes.c_size_t]
        L.orc_raw_to_wmma.argtypes = [_u16p, _u16p, ctypes.c_uint32, ctypes.c_uint32]
        L.orc_wmma_to_raw.argtypes = [_u16p, _u16p, ctypes.c_uint32, ctypes.c_uint32]
        L.orc_splitmix64.restype = ctypes.c_uint64
        L.orc_splitmix64.argtypes = [ctypes.c_uint64]
        L.orc_substrate_f16.restype = ctypes.c_uint16
        L.orc_substrate_f16.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32]
        L.orc_fill_substrate.argtypes = [_u16p, ctypes.c_uint64, ctypes.c_uint64,
                                         ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint64]
        L.orc_fill_segments.argtypes = [_u16p, ctypes.c_uint64, _u64p, ctypes.c_uint64,
                                        ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64]
        L.orc_act.restype = ctypes.c_double
        L.orc_act.argtypes = [ctypes.c_double, ctypes.c_int]
        L.orc_wave_f64.restype = ctypes.c_int
        L.orc_wave_f64.argtypes = [_u16p, _u64p, _u16p, _u16p, _u16p, ctypes.c_uint32,
                                   ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64,
                                   ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_uint64, _u32p, ctypes.c_uint32, _dp]
        L.orc_wave_f32_omp.restype = ctypes.c_int
        L.orc_wave_f32_omp.argtypes = [_u16p, _u64p, _u16p, _u16p, _u16p, ctypes.c_uint32,
                                       ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                       ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint64,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_uint64,
                                       ctypes.c_uint64, ctypes.c_int]
        _lib = L
    return _lib


def _p(a, t):
    return None if a is None else a.ctypes.data_as(t)


def f32_to_f16(x: float) -> int:
    return int(lib().orc_f32_to_f16(float(x)))


def f32bits_to_f16(bits: int) -> int:
    return int(lib().orc_f32bits_to_f16(int(bits)))


def f16_to_f32(h: int) -> float:
    return float(lib().orc_f16_to_f32(int(h)))


def fnv1a64(data: bytes) -> int:
    buf = np.frombuffer(data, dtype=np.uint8).copy() if data else np.zeros(1, np.uint8)
    return int(lib().orc_fnv1a64(_p(buf, _u8p), len(data)))


def raw_to_wmma(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w).view(np.uint16)
    out = np.empty_like(w)
    lib().orc_raw_to_wmma(_p(out, _u16p), _p(w, _u16p), w.shape[0], w.shape[1])
    return out


def wmma_to_raw(w: np.ndarray, cout: int, B: int) -> np.ndarray:
    w = np.ascontiguousarray(w).view(np.uint16).reshape(cout, B)
    out = np.empty_like(w)
    lib().orc_wmma_to_raw(_p(out, _u16p), _p(w, _u16p), cout, B)
    return out


def splitmix64(x: int) -> int:
    return int(lib().orc_splitmix64(int(x) & 0xFFFFFFFFFFFFFFFF))


def substrate_f16(seed: int, pos: int, tok: int) -> int:
    return int(lib().orc_substrate_f16(seed, pos, tok))


def fill_substrate(seed: int, pos0: int, npos: int, tokens: int, stride: int) -> np.ndarray:
    out = np.zeros((npos, stride), dtype=np.uint16)
    lib().orc_fill_substrate(_p(out, _u16p), seed, pos0, npos, tokens, stride)
    return out


def fill_segments(seed: int, starts: np.ndarray, S: int, tokens: int, stride: int) -> np.ndarray:
    """Compact substrate: row i*S + s holds substrate position starts[i] + s."""
    st = np.ascontiguousarray(starts, dtype=np.uint64).ravel()
    out = np.zeros((st.size * S, stride), dtype=np.uint16)
    lib().orc_fill_segments(_p(out, _u16p), seed, _p(st, _u64p), st.size, S, tokens, stride)
    return out


ACT_IDS = {"none": 0, None: 0, "relu": 1, "sigmoid": 2, "silu": 3, "leaky_relu": 4, "gelu": 5}


def wave_f64(canvas: np.ndarray, seg: np.ndarray, w: np.ndarray, bias, cmap, K: int, S: int,
             cluster: int, step: int, tokens: int, out_stride: int, act, res_off=None,
             sel=None) -> np.ndarray:
    """fp64 oracle; returns [len(sel), tokens] float64 (pre-fp16-rounding) outputs."""
    canvas = np.ascontiguousarray(canvas).view(np.uint16)
    seg = np.ascontiguousarray(seg, dtype=np.uint64)
    w = np.ascontiguousarray(w).view(np.uint16)
    b = None if bias is None else np.ascontiguousarray(bias).view(np.uint16)
    cm = None if cmap is None else np.ascontiguousarray(cmap, dtype=np.uint16)
    cout = w.shape[0]
    sel = np.arange(cout, dtype=np.uint32) if sel is None else np.ascontiguousarray(sel, np.uint32)
    out = np.empty((sel.size, tokens), dtype=np.float64)
    lib().orc_wave_f64(_p(canvas, _u16p), _p(seg, _u64p), _p(w, _u16p), _p(b, _u16p),
                       _p(cm, _u16p), K, S, cluster, step, tokens, out_stride,
                       ACT_IDS.get(act, act) if not isinstance(act, int) else act,
                       0 if res_off is None else 1, 0 if res_off is None else res_off,
                       _p(sel, _u32p), sel.size, _p(out, _dp))
    return out


def wave_f32_omp(canvas: np.ndarray, seg, w, bias, cmap, K, S, cluster, step, tokens,
                 out_stride, act, y_off, res_off=None, threads=0) -> int:
    """OpenMP fp32 path writing fp16 outputs into `canvas` (uint16 array) in place."""
    assert canvas.dtype == np.uint16 and canvas.flags.c_contiguous
    seg = np.ascontiguousarray(seg, dtype=np.uint64)
    w = np.ascontiguousarray(w).view(np.uint16)
    b = None if bias is None else np.ascontiguousarray(bias).view(np.uint16)
    cm = None if cmap is None else np.ascontiguousarray(cmap, dtype=np.uint16)
    return int(lib().orc_wave_f32_omp(
        _p(canvas, _u16p), _p(seg, _u64p), _p(w, _u16p), _p(b, _u16p), _p(cm, _u16p),
        w.shape[0], K, S, cluster, step, tokens, out_stride,
        ACT_IDS.get(act, act) if not isinstance(act, int) else act,
        0 if res_off is None else 1, 0 if res_off is None else res_off, y_off, threads))


def rel_err(y: np.ndarray, ref: np.ndarray) -> float:
    """max |y - ref| / (|ref| + 1e-2): the north_star tolerance metric (bound 2e-3)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if y.size == 0:
        return 0.0
    return float(np.max(np.abs(y - ref) / (np.abs(ref) + 1e-2)))

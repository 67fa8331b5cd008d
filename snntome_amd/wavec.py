"""wavec.py — ctypes interface of libk44wavec.so, the MI355X (gfx950) wave executor.

Same Python API as the reference's wavec/wavec.py (ACT_MAP, get_lib, WavePlan, WaveGraph and
their methods, argument meaning, RuntimeError on a failed call), bound to this build's
library, plus the build extensions: sparse / dendritic-cluster waves, device-side input fill,
timed plan execution, raw canvas access and the per-wave execution report.

The library must exist next to this file (build it with ``python -m snntome_amd.build``);
loading fails loudly otherwise — there is no CPU fallback.
"""

import ctypes
import json
from pathlib import Path
from typing import List, Optional, Sequence, Tuple, Union

import numpy as np

ACT_MAP = {
    None: 0, "none": 0, "identity": 0, "linear": 0,
    "relu": 1, "sigmoid": 2, "silu": 3, "swish": 3, "leaky_relu": 4,
    "gelu": 5,
}

_c = ctypes
_vp, _cp, _i, _f = _c.c_void_p, _c.c_char_p, _c.c_int, _c.c_float
_pf = _c.POINTER(_c.c_float)
_pu16 = _c.POINTER(_c.c_uint16)
_pu32 = _c.POINTER(_c.c_uint32)
_pcp = _c.POINTER(_c.c_char_p)
_ull = _c.c_ulonglong
_u32 = _c.c_uint32

# name -> (restype, argtypes)
_SIGNATURES = {
    "wavec_create": (_vp, [_i, _i, _i, _i]),
    "wavec_destroy": (None, [_vp]),
    "wavec_gpu_release": (_i, [_vp]),
    "wavec_add_input": (_i, [_vp, _cp, _i, _i, _i, _i]),
    "wavec_add_flatten": (_i, [_vp, _cp, _cp, _cp]),
    "wavec_add_conv2d": (_i, [_vp, _cp, _cp, _cp, _i, _i, _i, _i, _i, _i, _i, _pf, _pf, _cp]),
    "wavec_add_conv2d_f16": (_i, [_vp, _cp, _cp, _cp, _i, _i, _i, _i, _i, _i, _i, _pu16, _pf, _cp]),
    "wavec_add_linear_f32": (_i, [_vp, _cp, _cp, _cp, _i, _i, _i, _pf, _pf, _cp]),
    "wavec_add_linear_f16": (_i, [_vp, _cp, _cp, _cp, _i, _i, _i, _pu16, _pf, _cp]),
    "wavec_add_linear_bf16": (_i, [_vp, _cp, _cp, _cp, _i, _i, _i, _pu16, _pf, _cp]),
    "wavec_add_upconv2x2": (_i, [_vp, _cp, _cp, _cp, _i, _i, _pf, _pf]),
    "wavec_add_maxpool": (_i, [_vp, _cp, _cp, _cp, _i, _i, _i]),
    "wavec_add_upsample2x": (_i, [_vp, _cp, _cp, _cp]),
    "wavec_add_rmsnorm": (_i, [_vp, _cp, _cp, _cp, _i, _f, _pf, _i]),
    "wavec_add_swiglu": (_i, [_vp, _cp, _cp, _cp, _cp]),
    "wavec_add_rope_gqa_attn": (_i, [_vp, _cp, _cp, _cp, _cp, _cp, _i, _i, _i, _f, _i]),
    "wavec_add_split": (_i, [_vp, _cp, _cp, _i, _pcp]),
    "wavec_add_slice": (_i, [_vp, _cp, _cp, _i, _pcp, _c.POINTER(_i)]),
    "wavec_add_concat": (_i, [_vp, _cp, _i, _pcp, _cp]),
    "wavec_set_output": (_i, [_vp, _cp]),
    "wavec_set_reuse_canvas": (_i, [_vp, _i]),
    "wavec_set_batch_size": (_i, [_vp, _i]),
    "wavec_set_target_preset": (_i, [_vp, _cp]),
    "wavec_compile": (_i, [_vp]),
    "wavec_get_summary_json": (_cp, [_vp]),
    "wavec_save_tcff": (_i, [_vp, _cp, _cp]),
    "wavec_save_tcff_ex": (_i, [_vp, _cp, _cp, _i, _i]),
    "wavec_load_tcff_weights": (_i, [_vp, _cp]),
    "wavec_gpu_init_plan": (_i, [_vp]),
    "wavec_gpu_infer_f32": (_i, [_vp, _pf, _i, _pf, _i, _pf]),
    # build extensions
    "wavec_last_error": (_cp, []),
    "wavec_add_sparse_wave": (_i, [_vp, _cp, _cp, _cp, _i, _i, _i, _pu32, _pu16, _pu16, _i, _cp]),
    "wavec_add_cluster_wave": (_i, [_vp, _cp, _cp, _cp, _i, _i, _i, _i, _pu32, _pu16, _pu16, _i, _cp]),
    "wavec_add_pruned_wave": (_i, [_vp, _cp, _cp, _cp, _i, _i, _i, _i, _pu32, _pu16, _pu16, _i, _cp]),
    "wavec_gpu_fill_input_uniform": (_i, [_vp, _ull]),
    "wavec_gpu_execute": (_i, [_vp, _i, _pf]),
    "wavec_gpu_sync": (_i, [_vp]),
    "wavec_gpu_execute_range": (_i, [_vp, _i, _i]),
    "wavec_gpu_read_canvas": (_i, [_vp, _ull, _ull, _pu16]),
    "wavec_gpu_write_canvas": (_i, [_vp, _ull, _ull, _pu16]),
    "wavec_add_token_shift": (_i, [_vp, _cp, _cp, _cp, _i, _i, _i, _pu16, _i]),
    "wavec_add_embedding": (_i, [_vp, _cp, _cp, _cp, _i, _i, _pu16]),
    "wavec_add_argmax": (_i, [_vp, _cp, _cp, _cp]),
    "wavec_gpu_set_ids": (_i, [_vp, _pu32, _i]),
    "wavec_gpu_get_ids": (_i, [_vp, _pu32, _i]),
    "wavec_gpu_set_history": (_i, [_vp, _i]),
    "wavec_gpu_get_history": (_i, [_vp, _pu32, _i]),
    "wavec_gpu_use_graph": (_i, [_vp, _i]),
    "wavec_gpu_copy_canvas": (_i, [_vp, _ull, _vp, _ull, _ull]),
    "wavec_gpu_copy_ids": (_i, [_vp, _i, _vp, _i, _i, _i]),
    "wavec_gpu_exec_report_json": (_cp, [_vp]),
    "wavec_dev_malloc": (_vp, [_ull]),
    "wavec_dev_free": (_i, [_vp]),
    "wavec_dev_upload": (_i, [_vp, _vp, _ull]),
    "wavec_dev_download": (_i, [_vp, _vp, _ull]),
    "wavec_dev_synchronize": (_i, []),
    "wavec_dev_fill_uniform": (_i, [_vp, _ull, _u32, _u32, _ull, _ull]),
    "wavec_dev_time_begin": (_i, []),
    "wavec_dev_time_end": (_i, [_pf]),
    "wavec_k44_f16_forward_token64": (_i, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp]),
    "wavec_interleave_weights_wmma": (_i, [_vp, _vp, _u32, _u32, _vp]),
}

REFERENCE_SYMBOLS = tuple(list(_SIGNATURES)[:30])
EXTENSION_SYMBOLS = tuple(list(_SIGNATURES)[30:])

LIB_PATH = Path(__file__).resolve().parent / "libk44wavec.so"


def _load_lib() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise FileNotFoundError(
            f"Shared library {LIB_PATH} not found. Run `python -m snntome_amd.build` first."
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_LIB: Optional[ctypes.CDLL] = None


def get_lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = _load_lib()
    return _LIB


def last_error() -> str:
    msg = get_lib().wavec_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed: {last_error()}")


def _ptr(a: Optional[np.ndarray], ctype):
    return None if a is None else a.ctypes.data_as(ctypes.POINTER(ctype))


def _f16_bits(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.float16:
        return np.ascontiguousarray(a).view(np.uint16)
    if a.dtype == np.uint16:
        return np.ascontiguousarray(a)
    return np.ascontiguousarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)


class WavePlan:
    """Compiled Wave Execution Plan with TCFF v1.0 serialization and GPU execution."""

    def __init__(self, handle: ctypes.c_void_p, lib: ctypes.CDLL, summary: dict, owner=None):
        self._handle = handle
        self._lib = lib
        self.summary = summary
        self._gpu_initialized = False
        self._owner = owner  # the WaveGraph that owns `handle`; kept alive with the plan

    @property
    def total_gflops(self) -> float:
        return float(self.summary.get("total_gflops", 0.0))

    @property
    def canvas_bytes(self) -> int:
        return int(self.summary.get("canvas_bytes", 0))

    @property
    def num_wave_dispatches(self) -> int:
        return int(self.summary.get("num_waves", self.summary.get("num_wave_dispatches", 0)))

    def save_tcff(self, tcff_path: Union[str, Path], model_prefix: str = "K44Model") -> int:
        n = self._lib.wavec_save_tcff(self._handle, str(tcff_path).encode("utf-8"),
                                      model_prefix.encode("utf-8"))
        if n < 0:
            raise RuntimeError(f"Failed to export TCFF v1.0 file: {tcff_path}")
        return self.num_wave_dispatches

    def load_tcff_weights(self, tcff_path: Union[str, Path]) -> None:
        rc = self._lib.wavec_load_tcff_weights(self._handle, str(tcff_path).encode("utf-8"))
        if rc != 0:
            raise RuntimeError(f"Failed to load TCFF weights from: {tcff_path}")
        self._gpu_initialized = False

    def init_gpu(self) -> None:
        if not self._gpu_initialized:
            rc = self._lib.wavec_gpu_init_plan(self._handle)
            if rc != 0:
                raise RuntimeError("Failed to initialize GPU execution state for WavePlan: "
                                   + last_error())
            self._gpu_initialized = True

    def infer_f32(self, x: np.ndarray) -> Tuple[np.ndarray, float]:
        self.init_gpu()
        x_f32 = np.ascontiguousarray(x, dtype=np.float32)
        c, h, w = tuple(self.summary["output_shape"])
        batch = int(self.summary.get("batch_size", 1))
        out_elems = batch * c * h * w if batch > 1 else c * h * w
        out_arr = np.empty((batch, c, h, w) if batch > 1 else (c, h, w), dtype=np.float32)
        gpu_ms = ctypes.c_float(0.0)
        rc = self._lib.wavec_gpu_infer_f32(self._handle, _ptr(x_f32, ctypes.c_float),
                                           int(x_f32.size), _ptr(out_arr, ctypes.c_float),
                                           int(out_elems), ctypes.byref(gpu_ms))
        if rc != 0:
            raise RuntimeError("GPU inference failed in wavec_gpu_infer_f32: " + last_error())
        return out_arr, float(gpu_ms.value)

    # ---------------------------------------------------------------- build extensions
    def fill_input_uniform(self, seed: int) -> None:
        """Device-side synthetic input (the substrate generator of include/k44wavec.h)."""
        self.init_gpu()
        _check(self._lib.wavec_gpu_fill_input_uniform(self._handle, int(seed)),
               "wavec_gpu_fill_input_uniform")

    def execute(self, iters: int = 1) -> float:
        """Runs the plan `iters` times back to back; returns average ms per run (HIP events)."""
        self.init_gpu()
        ms = ctypes.c_float(0.0)
        _check(self._lib.wavec_gpu_execute(self._handle, int(iters), ctypes.byref(ms)),
               "wavec_gpu_execute")
        return float(ms.value)

    def sync(self) -> None:
        _check(self._lib.wavec_gpu_sync(self._handle), "wavec_gpu_sync")

    def execute_range(self, first_cmd: int, n_cmds: int = 1) -> None:
        """Runs plan commands [first_cmd, first_cmd + n_cmds) and waits for them."""
        self.init_gpu()
        _check(self._lib.wavec_gpu_execute_range(self._handle, int(first_cmd), int(n_cmds)),
               "wavec_gpu_execute_range")

    def read_canvas(self, off: int, n: int) -> np.ndarray:
        out = np.empty(int(n), dtype=np.uint16)
        _check(self._lib.wavec_gpu_read_canvas(self._handle, int(off), int(n),
                                               _ptr(out, ctypes.c_uint16)),
               "wavec_gpu_read_canvas")
        return out

    def write_canvas(self, off: int, data: np.ndarray) -> None:
        d = _f16_bits(data).ravel()
        _check(self._lib.wavec_gpu_write_canvas(self._handle, int(off), int(d.size),
                                                _ptr(d, ctypes.c_uint16)),
               "wavec_gpu_write_canvas")

    def exec_report(self) -> dict:
        raw = self._lib.wavec_gpu_exec_report_json(self._handle)
        return json.loads(raw.decode("utf-8")) if raw else {}

    @property
    def cmds(self) -> List[dict]:
        return list(self.summary.get("cmds", []))

    def set_ids(self, ids) -> None:
        a = np.ascontiguousarray(ids, dtype=np.uint32)
        _check(self._lib.wavec_gpu_set_ids(self._handle, _ptr(a, ctypes.c_uint32), int(a.size)),
               "wavec_gpu_set_ids")

    def get_ids(self, n: int) -> np.ndarray:
        out = np.empty(int(n), dtype=np.uint32)
        _check(self._lib.wavec_gpu_get_ids(self._handle, _ptr(out, ctypes.c_uint32), int(n)),
               "wavec_gpu_get_ids")
        return out

    def set_history(self, steps: int) -> None:
        _check(self._lib.wavec_gpu_set_history(self._handle, int(steps)), "wavec_gpu_set_history")

    def get_history(self, steps: int, tokens: int) -> np.ndarray:
        out = np.zeros(int(steps) * int(tokens), dtype=np.uint32)
        n = self._lib.wavec_gpu_get_history(self._handle, _ptr(out, ctypes.c_uint32), out.size)
        if n < 0:
            raise RuntimeError("wavec_gpu_get_history failed: " + last_error())
        return out.reshape(int(steps), int(tokens))[:n]

    def use_graph(self, enable: bool = True) -> None:
        _check(self._lib.wavec_gpu_use_graph(self._handle, 1 if enable else 0),
               "wavec_gpu_use_graph")

    def copy_canvas_from(self, src: "WavePlan", dst_off: int, src_off: int, n: int) -> None:
        _check(self._lib.wavec_gpu_copy_canvas(self._handle, int(dst_off), src._handle,
                                               int(src_off), int(n)), "wavec_gpu_copy_canvas")

    def copy_ids_from(self, src: "WavePlan", dst_first: int, src_first: int, src_step: int,
                      n: int) -> None:
        _check(self._lib.wavec_gpu_copy_ids(self._handle, int(dst_first), src._handle,
                                            int(src_first), int(src_step), int(n)),
               "wavec_gpu_copy_ids")


class WaveGraph:
    """5-Pass Wave Graph Builder for Vision (2D Spatial) and LLM (1D Token) Connectomes."""

    def __init__(
        self,
        max_B_per_wave: int = 288,
        default_S: int = 0,
        kv_cache_max_seq: int = 2048,
        fold_rmsnorm_gamma: bool = True,
        reuse_canvas: bool = False,
        batch_size: int = 1,
        target: str = "auto",
    ):
        self._lib = get_lib()
        self._handle = self._lib.wavec_create(int(max_B_per_wave), int(default_S),
                                              int(kv_cache_max_seq),
                                              1 if fold_rmsnorm_gamma else 0)
        if not self._handle:
            raise RuntimeError("wavec_create failed")
        self._lib.wavec_set_reuse_canvas(self._handle, 1 if reuse_canvas else 0)
        self._lib.wavec_set_batch_size(self._handle, int(batch_size))
        self._lib.wavec_set_target_preset(self._handle, target.encode("utf-8"))
        self._keep: list = []

    def __del__(self):
        if getattr(self, "_handle", None):
            self._lib.wavec_destroy(self._handle)
            self._handle = None

    def add_input(self, name: str, c: int, h: int = 1, w: int = 1, is_1d: bool = False) -> str:
        _check(self._lib.wavec_add_input(self._handle, name.encode(), int(c), int(h), int(w),
                                         1 if is_1d else 0), "wavec_add_input")
        return name

    def add_conv2d(self, name: str, in_blob: str, out_blob: str, cin: int, cout: int, kh: int,
                   kw: int, weights: np.ndarray, bias: Optional[np.ndarray] = None,
                   stride: int = 1, pad: int = 0, act: Optional[str] = "silu",
                   res_blob: Optional[str] = None) -> str:
        w_f32 = np.ascontiguousarray(weights, dtype=np.float32)
        b_f32 = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
        _check(self._lib.wavec_add_conv2d(
            self._handle, name.encode(), in_blob.encode(), out_blob.encode(), int(cin), int(cout),
            int(kh), int(kw), int(stride), int(pad), ACT_MAP.get(act, 0),
            _ptr(w_f32, ctypes.c_float), _ptr(b_f32, ctypes.c_float),
            res_blob.encode() if res_blob else None), "wavec_add_conv2d")
        return out_blob

    def add_linear(self, name: str, in_blob: str, out_blob: str, cin: int, cout: int,
                   weights: np.ndarray, bias: Optional[np.ndarray] = None,
                   act: Optional[str] = None, res_blob: Optional[str] = None) -> str:
        b_f32 = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
        res_c = res_blob.encode() if res_blob else None
        if weights.dtype == np.float16 or weights.dtype == np.uint16:
            w_u16 = np.ascontiguousarray(weights.view(np.uint16), dtype=np.uint16)
            rc = self._lib.wavec_add_linear_f16(
                self._handle, name.encode(), in_blob.encode(), out_blob.encode(), int(cin),
                int(cout), ACT_MAP.get(act, 0), _ptr(w_u16, ctypes.c_uint16),
                _ptr(b_f32, ctypes.c_float), res_c)
        else:
            w_f32 = np.ascontiguousarray(weights, dtype=np.float32)
            rc = self._lib.wavec_add_linear_f32(
                self._handle, name.encode(), in_blob.encode(), out_blob.encode(), int(cin),
                int(cout), ACT_MAP.get(act, 0), _ptr(w_f32, ctypes.c_float),
                _ptr(b_f32, ctypes.c_float), res_c)
        _check(rc, "wavec_add_linear")
        return out_blob

    def add_rmsnorm(self, name: str, in_blob: str, out_blob: str, dim: int, gamma: np.ndarray,
                    eps: float = 1e-5, pre_folded: bool = False) -> str:
        g_f32 = np.ascontiguousarray(gamma, dtype=np.float32)
        _check(self._lib.wavec_add_rmsnorm(
            self._handle, name.encode(), in_blob.encode(), out_blob.encode(), int(dim),
            ctypes.c_float(eps), _ptr(g_f32, ctypes.c_float), 1 if pre_folded else 0),
            "wavec_add_rmsnorm")
        return out_blob

    def add_swiglu(self, name: str, gate_blob: str, up_blob: str, out_blob: str,
                   dim: int = 0) -> str:
        _check(self._lib.wavec_add_swiglu(self._handle, name.encode(), gate_blob.encode(),
                                          up_blob.encode(), out_blob.encode()),
               "wavec_add_swiglu")
        return out_blob

    def add_rope_gqa_attn(self, name: str, q_blob: str, k_blob: str, v_blob: str, out_blob: str,
                          h_q: int, h_kv: int, head_dim: int, rope_theta: float = 10000.0,
                          llama3_scaling: bool = False) -> str:
        _check(self._lib.wavec_add_rope_gqa_attn(
            self._handle, name.encode(), q_blob.encode(), k_blob.encode(), v_blob.encode(),
            out_blob.encode(), int(h_q), int(h_kv), int(head_dim), ctypes.c_float(rope_theta),
            1 if llama3_scaling else 0), "wavec_add_rope_gqa_attn")
        return out_blob

    def add_maxpool(self, name: str, in_blob: str, out_blob: str, kernel_size: int = 5,
                    stride: int = 1, pad: int = 2) -> str:
        _check(self._lib.wavec_add_maxpool(self._handle, name.encode(), in_blob.encode(),
                                           out_blob.encode(), int(kernel_size), int(stride),
                                           int(pad)), "wavec_add_maxpool")
        return out_blob

    def add_upconv2x2(self, name: str, in_blob: str, out_blob: str, cin: int, cout: int,
                      weights: np.ndarray, bias: Optional[np.ndarray] = None) -> str:
        """2x2 stride-2 transposed convolution; weights [cout][cin][2][2] (C ABI
        wavec_add_upconv2x2, which the reference binds but wraps in no method)."""
        w = np.ascontiguousarray(weights, dtype=np.float32)
        b = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
        _check(self._lib.wavec_add_upconv2x2(self._handle, name.encode(), in_blob.encode(),
                                             out_blob.encode(), int(cin), int(cout),
                                             _ptr(w, ctypes.c_float), _ptr(b, ctypes.c_float)),
               "wavec_add_upconv2x2")
        return out_blob

    def add_upsample2x(self, name: str, in_blob: str, out_blob: str) -> str:
        _check(self._lib.wavec_add_upsample2x(self._handle, name.encode(), in_blob.encode(),
                                              out_blob.encode()), "wavec_add_upsample2x")
        return out_blob

    def add_split(self, name: str, in_blob: str, out_blobs: Sequence[str]) -> List[str]:
        arr = (ctypes.c_char_p * len(out_blobs))(*[b.encode() for b in out_blobs])
        _check(self._lib.wavec_add_split(self._handle, name.encode(), in_blob.encode(),
                                         len(out_blobs), arr), "wavec_add_split")
        return list(out_blobs)

    def add_slice(self, name: str, in_blob: str, out_blobs: Sequence[str],
                  slice_sizes: Sequence[int]) -> List[str]:
        arr = (ctypes.c_char_p * len(out_blobs))(*[b.encode() for b in out_blobs])
        sz = (ctypes.c_int * len(slice_sizes))(*[int(s) for s in slice_sizes])
        _check(self._lib.wavec_add_slice(self._handle, name.encode(), in_blob.encode(),
                                         len(out_blobs), arr, sz), "wavec_add_slice")
        return list(out_blobs)

    def add_concat(self, name: str, in_blobs: Sequence[str], out_blob: str) -> str:
        arr = (ctypes.c_char_p * len(in_blobs))(*[b.encode() for b in in_blobs])
        _check(self._lib.wavec_add_concat(self._handle, name.encode(), len(in_blobs), arr,
                                          out_blob.encode()), "wavec_add_concat")
        return out_blob

    def set_output(self, out_blob: str) -> None:
        _check(self._lib.wavec_set_output(self._handle, out_blob.encode()), "wavec_set_output")

    def compile(self) -> WavePlan:
        rc = self._lib.wavec_compile(self._handle)
        if rc != 0:
            raise RuntimeError("WaveGraph 5-pass compilation failed: " + last_error())
        raw_json = self._lib.wavec_get_summary_json(self._handle)
        summary = json.loads(raw_json.decode("utf-8")) if raw_json else {}
        return WavePlan(self._handle, self._lib, summary, owner=self)

    # ---------------------------------------------------------------- build extensions
    def add_sparse_wave(self, name: str, in_blob: str, out_blob: str, rows: np.ndarray,
                        weights: np.ndarray, bias: Optional[np.ndarray] = None,
                        cluster: int = 1, act: Optional[str] = None,
                        res_blob: Optional[str] = None) -> str:
        """rows: [cout/cluster, fan_in] input channel of every synapse; weights [cout, fan_in]."""
        w = _f16_bits(weights)
        cout, fan_in = w.shape
        r = np.ascontiguousarray(rows, dtype=np.uint32)
        if r.shape != (cout // cluster, fan_in):
            raise ValueError(f"rows must have shape {(cout // cluster, fan_in)}, got {r.shape}")
        b = _f16_bits(bias) if bias is not None else None
        _check(self._lib.wavec_add_sparse_wave(
            self._handle, name.encode(), in_blob.encode(), out_blob.encode(), int(cout),
            int(fan_in), int(cluster), _ptr(r, ctypes.c_uint32), _ptr(w, ctypes.c_uint16),
            _ptr(b, ctypes.c_uint16), ACT_MAP.get(act, 0),
            res_blob.encode() if res_blob else None), "wavec_add_sparse_wave")
        return out_blob

    def add_cluster_wave(self, name: str, in_blob: str, out_blob: str, starts: np.ndarray,
                         seg_len: int, weights: np.ndarray, bias: Optional[np.ndarray] = None,
                         cluster: int = 1, act: Optional[str] = None,
                         res_blob: Optional[str] = None) -> str:
        """starts: [cout/cluster, K] first input channel of each dendritic cluster of seg_len
        consecutive channels; weights [cout, K*seg_len]."""
        w = _f16_bits(weights)
        cout = w.shape[0]
        st = np.ascontiguousarray(starts, dtype=np.uint32)
        K = st.shape[1]
        if st.shape[0] * cluster != cout or w.shape[1] != K * seg_len:
            raise ValueError("starts / weights shapes do not match cout, cluster, K, seg_len")
        b = _f16_bits(bias) if bias is not None else None
        _check(self._lib.wavec_add_cluster_wave(
            self._handle, name.encode(), in_blob.encode(), out_blob.encode(), int(cout), int(K),
            int(seg_len), int(cluster), _ptr(st, ctypes.c_uint32), _ptr(w, ctypes.c_uint16),
            _ptr(b, ctypes.c_uint16), ACT_MAP.get(act, 0),
            res_blob.encode() if res_blob else None), "wavec_add_cluster_wave")
        return out_blob

    def add_pruned_wave(self, name: str, in_blob: str, out_blob: str, starts: np.ndarray,
                        seg_len: int, weights: np.ndarray, bias: Optional[np.ndarray] = None,
                        tile: int = 64, act: Optional[str] = None,
                        res_blob: Optional[str] = None) -> str:
        """starts: [cout, K] first input channel of each cluster neuron j keeps; weights
        [cout, K*seg_len] in the same cluster order.  Compiled to pattern-sorted tiles."""
        w = _f16_bits(weights)
        st = np.ascontiguousarray(starts, dtype=np.uint32)
        cout, K = st.shape
        if w.shape != (cout, K * seg_len):
            raise ValueError("starts / weights shapes do not match cout, K, seg_len")
        b = _f16_bits(bias) if bias is not None else None
        _check(self._lib.wavec_add_pruned_wave(
            self._handle, name.encode(), in_blob.encode(), out_blob.encode(), int(cout), int(K),
            int(seg_len), int(tile), _ptr(st, ctypes.c_uint32), _ptr(w, ctypes.c_uint16),
            _ptr(b, ctypes.c_uint16), ACT_MAP.get(act, 0),
            res_blob.encode() if res_blob else None), "wavec_add_pruned_wave")
        return out_blob

    def add_token_shift(self, name: str, in_blob: str, out_blob: str, mu: np.ndarray,
                        seq_len: int, decode: bool = False) -> str:
        """Causal depth-wise mix over the last rf tokens of each request; mu: [dim, rf]."""
        m = _f16_bits(mu)
        dim, rf = m.shape
        _check(self._lib.wavec_add_token_shift(self._handle, name.encode(), in_blob.encode(),
                                               out_blob.encode(), int(dim), int(rf),
                                               int(seq_len), _ptr(m, ctypes.c_uint16),
                                               1 if decode else 0), "wavec_add_token_shift")
        return out_blob

    def add_embedding(self, name: str, tok_blob: str, out_blob: str, table: np.ndarray) -> str:
        """y[c][t] = table[id[t]][c]; table: [vocab, dim]."""
        t = _f16_bits(table)
        vocab, dim = t.shape
        _check(self._lib.wavec_add_embedding(self._handle, name.encode(), tok_blob.encode(),
                                             out_blob.encode(), int(vocab), int(dim),
                                             _ptr(t, ctypes.c_uint16)), "wavec_add_embedding")
        return out_blob

    def add_argmax(self, name: str, in_blob: str, out_blob: str) -> str:
        _check(self._lib.wavec_add_argmax(self._handle, name.encode(), in_blob.encode(),
                                          out_blob.encode()), "wavec_add_argmax")
        return out_blob

    def save_tcff(self, path: Union[str, Path], model_prefix: str = "K44Model",
                  include_geometry: bool = True) -> None:
        _check(self._lib.wavec_save_tcff_ex(self._handle, str(path).encode(),
                                            model_prefix.encode(), 1,
                                            1 if include_geometry else 0), "wavec_save_tcff_ex")


class DeviceBuffer:
    """Device memory owned through libk44wavec.so (hipMalloc / hipFree), for the stand-alone
    kernels; `.ptr` is the device address."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self._lib = get_lib()
        self.ptr = self._lib.wavec_dev_malloc(self.nbytes)
        if not self.ptr:
            raise RuntimeError(f"wavec_dev_malloc({self.nbytes}) failed: {last_error()}")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("array larger than the device buffer")
        _check(self._lib.wavec_dev_upload(self.ptr, a.ctypes.data, a.nbytes), "wavec_dev_upload")

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("requested more bytes than the device buffer holds")
        _check(self._lib.wavec_dev_download(out.ctypes.data, self.ptr, out.nbytes),
               "wavec_dev_download")
        return out

    def free(self) -> None:
        if self.ptr:
            self._lib.wavec_dev_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def device_synchronize() -> None:
    _check(get_lib().wavec_dev_synchronize(), "wavec_dev_synchronize")


def _dev_ptr(x) -> int:
    """Device address of a DeviceBuffer (.ptr), an object with data_ptr(), or an integer."""
    if x is None:
        return 0
    if isinstance(x, DeviceBuffer):
        return int(x.ptr)
    return int(x.data_ptr()) if hasattr(x, "data_ptr") else int(x)


def forward_token64_f16(Y, X, cluster_indices, cluster_weights_wmma, neuron_bias,
                        batch_size: int, Cin: int, Cout: int, B_vec16: int, cluster_size: int,
                        stream=None) -> None:
    """Stand-alone Token64 wave on caller-owned device memory (the whitepaper launcher
    launch_k44_f16_forward): X [ceil(batch/64)][Cin][64] fp16 -> Y [ceil(batch/64)][Cout][64]
    fp16, round toward zero.  Arguments are device tensors (anything with data_ptr()) or raw
    device addresses; `stream` a hipStream_t address or None.  Asynchronous."""
    lib = get_lib()
    _check(lib.wavec_k44_f16_forward_token64(
        _dev_ptr(Y), _dev_ptr(X), _dev_ptr(cluster_indices), _dev_ptr(cluster_weights_wmma),
        _dev_ptr(neuron_bias) or None, int(batch_size), int(Cin), int(Cout), int(B_vec16),
        int(cluster_size), _dev_ptr(stream) or None), "wavec_k44_f16_forward_token64")


def interleave_weights_wmma(dst_wmma, src_compact, num_output_neurons: int, B_vec8: int,
                            stream=None) -> None:
    """GPU weight interleave: row-major [neurons][8*B_vec8] fp16 -> RDNA4 WMMA vector order."""
    lib = get_lib()
    _check(lib.wavec_interleave_weights_wmma(_dev_ptr(dst_wmma), _dev_ptr(src_compact),
                                             int(num_output_neurons), int(B_vec8),
                                             _dev_ptr(stream) or None),
           "wavec_interleave_weights_wmma")

"""Python front end of libk44wavec.so, the gfx950 (MI355X) wave executor.

Callers of SNNtome's ``wavec`` module find the same surface here: ``ACT_MAP``, ``get_lib()``,
``WaveGraph`` and ``WavePlan`` with the method names, argument names, defaults and return values
of the reference binding (reference wavec/wavec.py:13-16, :135-141, :147-211, :214-344), and a
``RuntimeError`` whenever the library reports a failure.  The library text of the error
(``wavec_last_error``) is part of every message.

Beyond that surface this module binds the build's extensions: sparse, dendritic-cluster and
pruned waves, token ops (token shift, embedding, argmax), device-side input generation, timed
plan execution, command- and run-wise execution, raw canvas access, the per-wave execution
report, executor tuning switches, and device buffers for the stand-alone Token64 launcher.

The shared library must sit next to this file (``python -m snntome_amd.build`` makes it).  There
is no CPU fallback: importing works without it, the first call that needs it raises.
"""

import ctypes
import json
import os
from pathlib import Path
from typing import List, Optional, Sequence, Tuple, Union

import numpy as np

# Activation names -> the epilogue ids of K44ExecCmd.act.  Ids 0-4 are the reference's; 5 (GELU,
# erf form) is an extension.
ACT_MAP = {
    None: 0, "none": 0, "identity": 0, "linear": 0,
    "relu": 1, "sigmoid": 2, "silu": 3, "swish": 3, "leaky_relu": 4,
    "gelu": 5,
}

C = ctypes
_VOID, _STR, _INT, _FLT = C.c_void_p, C.c_char_p, C.c_int, C.c_float
_U32, _ULL = C.c_uint32, C.c_ulonglong
_P_FLT = C.POINTER(C.c_float)
_P_U16 = C.POINTER(C.c_uint16)
_P_U32 = C.POINTER(C.c_uint32)
_P_STR = C.POINTER(C.c_char_p)

# Every exported entry point: (name, result type, argument types).  The first 30 rows are the
# reference's C ABI (wavec/k44_wave_executor.cu:644-986), the rest this build's extensions.
_ABI = (
    ("wavec_create", _VOID, (_INT, _INT, _INT, _INT)),
    ("wavec_destroy", None, (_VOID,)),
    ("wavec_gpu_release", _INT, (_VOID,)),
    ("wavec_add_input", _INT, (_VOID, _STR, _INT, _INT, _INT, _INT)),
    ("wavec_add_flatten", _INT, (_VOID, _STR, _STR, _STR)),
    ("wavec_add_conv2d", _INT,
     (_VOID, _STR, _STR, _STR, _INT, _INT, _INT, _INT, _INT, _INT, _INT, _P_FLT, _P_FLT, _STR)),
    ("wavec_add_conv2d_f16", _INT,
     (_VOID, _STR, _STR, _STR, _INT, _INT, _INT, _INT, _INT, _INT, _INT, _P_U16, _P_FLT, _STR)),
    ("wavec_add_linear_f32", _INT, (_VOID, _STR, _STR, _STR, _INT, _INT, _INT, _P_FLT, _P_FLT, _STR)),
    ("wavec_add_linear_f16", _INT, (_VOID, _STR, _STR, _STR, _INT, _INT, _INT, _P_U16, _P_FLT, _STR)),
    ("wavec_add_linear_bf16", _INT, (_VOID, _STR, _STR, _STR, _INT, _INT, _INT, _P_U16, _P_FLT, _STR)),
    ("wavec_add_upconv2x2", _INT, (_VOID, _STR, _STR, _STR, _INT, _INT, _P_FLT, _P_FLT)),
    ("wavec_add_maxpool", _INT, (_VOID, _STR, _STR, _STR, _INT, _INT, _INT)),
    ("wavec_add_upsample2x", _INT, (_VOID, _STR, _STR, _STR)),
    ("wavec_add_rmsnorm", _INT, (_VOID, _STR, _STR, _STR, _INT, _FLT, _P_FLT, _INT)),
    ("wavec_add_swiglu", _INT, (_VOID, _STR, _STR, _STR, _STR)),
    ("wavec_add_rope_gqa_attn", _INT, (_VOID, _STR, _STR, _STR, _STR, _STR, _INT, _INT, _INT, _FLT, _INT)),
    ("wavec_add_split", _INT, (_VOID, _STR, _STR, _INT, _P_STR)),
    ("wavec_add_slice", _INT, (_VOID, _STR, _STR, _INT, _P_STR, C.POINTER(_INT))),
    ("wavec_add_concat", _INT, (_VOID, _STR, _INT, _P_STR, _STR)),
    ("wavec_set_output", _INT, (_VOID, _STR)),
    ("wavec_set_reuse_canvas", _INT, (_VOID, _INT)),
    ("wavec_set_batch_size", _INT, (_VOID, _INT)),
    ("wavec_set_target_preset", _INT, (_VOID, _STR)),
    ("wavec_compile", _INT, (_VOID,)),
    ("wavec_get_summary_json", _STR, (_VOID,)),
    ("wavec_save_tcff", _INT, (_VOID, _STR, _STR)),
    ("wavec_save_tcff_ex", _INT, (_VOID, _STR, _STR, _INT, _INT)),
    ("wavec_load_tcff_weights", _INT, (_VOID, _STR)),
    ("wavec_gpu_init_plan", _INT, (_VOID,)),
    ("wavec_gpu_infer_f32", _INT, (_VOID, _P_FLT, _INT, _P_FLT, _INT, _P_FLT)),
    # ---- extensions
    ("wavec_last_error", _STR, ()),
    ("wavec_add_sparse_wave", _INT,
     (_VOID, _STR, _STR, _STR, _INT, _INT, _INT, _P_U32, _P_U16, _P_U16, _INT, _STR)),
    ("wavec_add_cluster_wave", _INT,
     (_VOID, _STR, _STR, _STR, _INT, _INT, _INT, _INT, _P_U32, _P_U16, _P_U16, _INT, _STR)),
    ("wavec_add_pruned_wave", _INT,
     (_VOID, _STR, _STR, _STR, _INT, _INT, _INT, _INT, _P_U32, _P_U16, _P_U16, _INT, _STR)),
    ("wavec_gpu_fill_input_uniform", _INT, (_VOID, _ULL)),
    ("wavec_gpu_execute", _INT, (_VOID, _INT, _P_FLT)),
    ("wavec_gpu_sync", _INT, (_VOID,)),
    ("wavec_gpu_program_trace", _INT, (_VOID, C.POINTER(C.c_ulonglong), C.c_ulonglong)),
    ("wavec_gpu_execute_range", _INT, (_VOID, _INT, _INT)),
    ("wavec_gpu_read_canvas", _INT, (_VOID, _ULL, _ULL, _P_U16)),
    ("wavec_gpu_write_canvas", _INT, (_VOID, _ULL, _ULL, _P_U16)),
    ("wavec_add_token_shift", _INT, (_VOID, _STR, _STR, _STR, _INT, _INT, _INT, _P_U16, _INT)),
    ("wavec_add_embedding", _INT, (_VOID, _STR, _STR, _STR, _INT, _INT, _P_U16)),
    ("wavec_add_argmax", _INT, (_VOID, _STR, _STR, _STR)),
    ("wavec_gpu_set_ids", _INT, (_VOID, _P_U32, _INT)),
    ("wavec_gpu_get_ids", _INT, (_VOID, _P_U32, _INT)),
    ("wavec_gpu_set_history", _INT, (_VOID, _INT)),
    ("wavec_gpu_get_history", _INT, (_VOID, _P_U32, _INT)),
    ("wavec_gpu_use_graph", _INT, (_VOID, _INT)),
    ("wavec_gpu_copy_canvas", _INT, (_VOID, _ULL, _VOID, _ULL, _ULL)),
    ("wavec_gpu_copy_ids", _INT, (_VOID, _INT, _VOID, _INT, _INT, _INT)),
    ("wavec_gpu_exec_report_json", _STR, (_VOID,)),
    ("wavec_dev_malloc", _VOID, (_ULL,)),
    ("wavec_dev_free", _INT, (_VOID,)),
    ("wavec_dev_upload", _INT, (_VOID, _VOID, _ULL)),
    ("wavec_dev_download", _INT, (_VOID, _VOID, _ULL)),
    ("wavec_dev_synchronize", _INT, ()),
    ("wavec_dev_fill_uniform", _INT, (_VOID, _ULL, _U32, _U32, _ULL, _ULL)),
    ("wavec_dev_time_begin", _INT, ()),
    ("wavec_dev_time_end", _INT, (_P_FLT,)),
    ("wavec_k44_f16_forward_token64", _INT,
     (_VOID, _VOID, _VOID, _VOID, _VOID, _U32, _U32, _U32, _U32, _U32, _VOID)),
    ("wavec_interleave_weights_wmma", _INT, (_VOID, _VOID, _U32, _U32, _VOID)),
    ("wavec_argmax_f16", _INT, (_VOID, _VOID, _U32, _U32, _U32, _VOID)),
    ("wavec_argmax_f16_noalloc", _INT, (_VOID, _VOID, _U32, _U32, _U32, _VOID)),
    ("wavec_set_tuning", _INT, (_STR, _INT)),
    ("wavec_get_tuning", _INT, (_STR,)),
    ("wavec_reset_tuning", None, ()),
    ("wavec_gpu_execute_runs", _INT, (_VOID, _INT, _INT)),
    ("wavec_gpu_read_canvas_2d", _INT, (_VOID, _ULL, _ULL, _ULL, _ULL, _P_U16)),
)

REFERENCE_SYMBOLS = tuple(name for name, _, _ in _ABI[:30])
EXTENSION_SYMBOLS = tuple(name for name, _, _ in _ABI[30:])

LIB_PATH = Path(__file__).resolve().parent / "libk44wavec.so"

_LIB: Optional[ctypes.CDLL] = None


def _load_lib() -> ctypes.CDLL:
    """Opens libk44wavec.so beside this module and declares every entry point's types."""
    if not LIB_PATH.is_file():
        raise FileNotFoundError(
            f"{LIB_PATH.name} is missing from {LIB_PATH.parent}; build it with "
            "`python -m snntome_amd.build` (there is no CPU fallback)")
    lib = ctypes.CDLL(os.fspath(LIB_PATH))
    for name, restype, argtypes in _ABI:
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = restype, list(argtypes)
    return lib


def get_lib() -> ctypes.CDLL:
    """The process-wide handle of libk44wavec.so (loaded on first use)."""
    global _LIB
    if _LIB is None:
        _LIB = _load_lib()
    return _LIB


def last_error() -> str:
    """Message of the library's last failure on this thread ('' if none)."""
    raw = get_lib().wavec_last_error()
    return raw.decode("utf-8", "replace") if raw else ""


def _raise_on(rc: int, action: str) -> None:
    if rc != 0:
        detail = last_error() or f"return code {rc}"
        raise RuntimeError(f"{action}: {detail}")


def _cstr(s: Optional[str]) -> Optional[bytes]:
    return None if s is None else os.fspath(s).encode("utf-8")


def _pointer(a: Optional[np.ndarray], ctype):
    return None if a is None else a.ctypes.data_as(C.POINTER(ctype))


def _f32(a) -> Optional[np.ndarray]:
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _f16_bits(a) -> np.ndarray:
    """fp16 bit patterns (uint16) of an fp16 / uint16 array, or of a float array rounded RNE."""
    a = np.asarray(a)
    if a.dtype == np.uint16:
        return np.ascontiguousarray(a)
    if a.dtype != np.float16:
        a = np.asarray(a, dtype=np.float32).astype(np.float16)
    return np.ascontiguousarray(a).view(np.uint16)


def _opt_f16_bits(a) -> Optional[np.ndarray]:
    return None if a is None else _f16_bits(a)


def _name_array(names: Sequence[str]):
    return (C.c_char_p * len(names))(*[_cstr(n) for n in names])


def set_tuning(key: str, value: int) -> None:
    """Sets one of the executor's process-wide tuning switches (A/B tests and benchmarks; every
    switch defaults to -1, the executor's own choice).  Applies to plans initialised afterwards.
    Keys are listed with wavec_set_tuning in include/k44wavec.h."""
    _raise_on(get_lib().wavec_set_tuning(_cstr(key), int(value)), f"wavec_set_tuning({key!r})")


def get_tuning(key: str) -> int:
    v = get_lib().wavec_get_tuning(_cstr(key))
    if v < -1:
        raise RuntimeError(f"wavec_get_tuning({key!r}): {last_error()}")
    return int(v)


def reset_tuning() -> None:
    """Every tuning switch back to -1 (automatic)."""
    get_lib().wavec_reset_tuning()


class WavePlan:
    """Result of WaveGraph.compile(): the plan's commands, canvas layout and weights.  It can be
    written to a .tcff file, have its weights replaced from one, and run on the GPU.  The plan
    shares the compiler handle of its graph and keeps that graph alive."""

    def __init__(self, handle: ctypes.c_void_p, lib: ctypes.CDLL, summary: dict, owner=None):
        self._handle = handle
        self._lib = lib
        self.summary = summary
        self._owner = owner
        self._gpu_initialized = False

    # ------------------------------------------------------------------ summary values
    @property
    def total_gflops(self) -> float:
        return float(self.summary.get("total_gflops", 0.0))

    @property
    def canvas_bytes(self) -> int:
        return int(self.summary.get("canvas_bytes", 0))

    @property
    def num_wave_dispatches(self) -> int:
        for key in ("num_waves", "num_wave_dispatches"):
            if key in self.summary:
                return int(self.summary[key])
        return 0

    # ------------------------------------------------------------------ .tcff
    def save_tcff(self, tcff_path: Union[str, Path], model_prefix: str = "K44Model") -> int:
        """Writes the plan as .tcff v1.0; returns the number of wave commands written."""
        rc = self._lib.wavec_save_tcff(self._handle, _cstr(tcff_path), _cstr(model_prefix))
        if rc < 0:
            raise RuntimeError(f"could not write plan file {os.fspath(tcff_path)!r}: {last_error()}")
        return self.num_wave_dispatches

    def load_tcff_weights(self, tcff_path: Union[str, Path]) -> None:
        """Replaces weights, indices and biases with those of a .tcff file written for the same
        plan (every block hash-checked); the GPU state must be initialised again afterwards."""
        rc = self._lib.wavec_load_tcff_weights(self._handle, _cstr(tcff_path))
        if rc != 0:
            raise RuntimeError(f"plan file {os.fspath(tcff_path)!r} was rejected: {last_error()}")
        self._gpu_initialized = False

    # ------------------------------------------------------------------ GPU
    def init_gpu(self) -> None:
        """Uploads the plan (device schedules, weights, zeroed canvas); idempotent."""
        if self._gpu_initialized:
            return
        if self._lib.wavec_gpu_init_plan(self._handle) != 0:
            raise RuntimeError(f"the GPU executor refused this plan: {last_error()}")
        self._gpu_initialized = True

    def infer_f32(self, x: np.ndarray) -> Tuple[np.ndarray, float]:
        """Host fp32 input -> one plan run -> host fp32 output of shape output_shape (with a
        leading frame axis when the plan's batch_size > 1; the executor moves frame 0, as the
        reference's does).  Returns (output, GPU milliseconds of the run)."""
        self.init_gpu()
        c, h, w = (int(v) for v in self.summary["output_shape"])
        frames = int(self.summary.get("batch_size", 1))
        y = np.zeros((frames, c, h, w) if frames > 1 else (c, h, w), dtype=np.float32)
        xin = np.ascontiguousarray(x, dtype=np.float32)
        ms = C.c_float(0.0)
        rc = self._lib.wavec_gpu_infer_f32(self._handle, _pointer(xin, C.c_float), int(xin.size),
                                           _pointer(y, C.c_float), int(y.size), C.byref(ms))
        if rc != 0:
            raise RuntimeError(f"wavec_gpu_infer_f32 did not run the plan: {last_error()}")
        return y, float(ms.value)

    # ------------------------------------------------------------------ extensions
    def fill_input_uniform(self, seed: int) -> None:
        """Fills the plan input on the device with the synthetic substrate generator."""
        self.init_gpu()
        _raise_on(self._lib.wavec_gpu_fill_input_uniform(self._handle, int(seed)),
                  "wavec_gpu_fill_input_uniform")

    def execute(self, iters: int = 1) -> float:
        """`iters` back-to-back runs of the whole plan; average milliseconds per run."""
        self.init_gpu()
        ms = C.c_float(0.0)
        _raise_on(self._lib.wavec_gpu_execute(self._handle, int(iters), C.byref(ms)),
                  "wavec_gpu_execute")
        return float(ms.value)

    def sync(self) -> None:
        _raise_on(self._lib.wavec_gpu_sync(self._handle), "wavec_gpu_sync")

    def program_trace(self) -> np.ndarray:
        """[items][8] records of the last persistent launch (tuning prog_trace=1): item start, wait
        released, completion signalled (100 MHz device ticks), workgroup, inputs arrived and
        MFMAs done (projection items), stores performed."""
        rep = self.exec_report()["program"]
        n = int(rep.get("items", 0))
        out = np.zeros((n, 8), np.uint64)
        _raise_on(self._lib.wavec_gpu_program_trace(
            self._handle, out.ctypes.data_as(C.POINTER(C.c_ulonglong)), n * 8),
            "wavec_gpu_program_trace")
        return out

    def release_gpu(self) -> None:
        """Frees the plan's device state (canvas, schedules, graphs); init_gpu builds it again."""
        _raise_on(self._lib.wavec_gpu_release(self._handle), "wavec_gpu_release")
        self._gpu_initialized = False

    def execute_range(self, first_cmd: int, n_cmds: int = 1) -> None:
        """Commands [first_cmd, first_cmd + n_cmds), each as compiled and launched alone (no
        grouping, nothing folded); waits for them."""
        self.init_gpu()
        _raise_on(self._lib.wavec_gpu_execute_range(self._handle, int(first_cmd), int(n_cmds)),
                  "wavec_gpu_execute_range")

    def execute_runs(self, first_run: int, n_runs: int = 1) -> None:
        """Runs [first_run, first_run + n_runs) of the whole-plan schedule (exec_report()['runs']),
        launched exactly as wavec_gpu_execute launches them; waits for them."""
        self.init_gpu()
        _raise_on(self._lib.wavec_gpu_execute_runs(self._handle, int(first_run), int(n_runs)),
                  "wavec_gpu_execute_runs")

    def read_canvas(self, off: int, n: int) -> np.ndarray:
        buf = np.empty(int(n), dtype=np.uint16)
        _raise_on(self._lib.wavec_gpu_read_canvas(self._handle, int(off), int(n),
                                                  _pointer(buf, C.c_uint16)),
                  "wavec_gpu_read_canvas")
        return buf

    def read_canvas_2d(self, off: int, rows: int, row_stride: int, cols: int) -> np.ndarray:
        """[rows][cols] fp16 bits: `cols` elements from each of `rows` rows `row_stride` apart."""
        buf = np.empty((int(rows), int(cols)), dtype=np.uint16)
        _raise_on(self._lib.wavec_gpu_read_canvas_2d(self._handle, int(off), int(rows),
                                                     int(row_stride), int(cols),
                                                     _pointer(buf, C.c_uint16)),
                  "wavec_gpu_read_canvas_2d")
        return buf

    def write_canvas(self, off: int, data: np.ndarray) -> None:
        bits = _f16_bits(data).ravel()
        _raise_on(self._lib.wavec_gpu_write_canvas(self._handle, int(off), int(bits.size),
                                                   _pointer(bits, C.c_uint16)),
                  "wavec_gpu_write_canvas")

    def exec_report(self) -> dict:
        """Per-wave path choices, token ops, group launches and runs of the initialised plan."""
        raw = self._lib.wavec_gpu_exec_report_json(self._handle)
        return json.loads(raw) if raw else {}

    @property
    def cmds(self) -> List[dict]:
        return list(self.summary.get("cmds", []))

    def set_ids(self, ids) -> None:
        v = np.ascontiguousarray(ids, dtype=np.uint32)
        _raise_on(self._lib.wavec_gpu_set_ids(self._handle, _pointer(v, C.c_uint32), int(v.size)),
                  "wavec_gpu_set_ids")

    def get_ids(self, n: int) -> np.ndarray:
        v = np.empty(int(n), dtype=np.uint32)
        _raise_on(self._lib.wavec_gpu_get_ids(self._handle, _pointer(v, C.c_uint32), int(n)),
                  "wavec_gpu_get_ids")
        return v

    def set_history(self, steps: int) -> None:
        _raise_on(self._lib.wavec_gpu_set_history(self._handle, int(steps)),
                  "wavec_gpu_set_history")

    def get_history(self, steps: int, tokens: int) -> np.ndarray:
        v = np.zeros((int(steps), int(tokens)), dtype=np.uint32)
        got = self._lib.wavec_gpu_get_history(self._handle, _pointer(v, C.c_uint32), int(v.size))
        if got < 0:
            raise RuntimeError(f"wavec_gpu_get_history: {last_error()}")
        return v[:got]

    def use_graph(self, enable: bool = True) -> None:
        _raise_on(self._lib.wavec_gpu_use_graph(self._handle, int(bool(enable))),
                  "wavec_gpu_use_graph")

    def copy_canvas_from(self, src: "WavePlan", dst_off: int, src_off: int, n: int) -> None:
        _raise_on(self._lib.wavec_gpu_copy_canvas(self._handle, int(dst_off), src._handle,
                                                  int(src_off), int(n)),
                  "wavec_gpu_copy_canvas")

    def copy_ids_from(self, src: "WavePlan", dst_first: int, src_first: int, src_step: int,
                      n: int) -> None:
        _raise_on(self._lib.wavec_gpu_copy_ids(self._handle, int(dst_first), src._handle,
                                               int(src_first), int(src_step), int(n)),
                  "wavec_gpu_copy_ids")


class WaveGraph:
    """Graph builder in front of the 5-pass wave compiler: tensors are named blobs, every add_*
    appends one node (1-D token graphs for LLM-shaped networks, 2-D image graphs for CNNs) and
    returns its output blob name; compile() lowers the graph to a WavePlan."""

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
                                              int(kv_cache_max_seq), int(bool(fold_rmsnorm_gamma)))
        if not self._handle:
            raise RuntimeError("wavec_create returned no compiler handle")
        for fn, arg in ((self._lib.wavec_set_reuse_canvas, int(bool(reuse_canvas))),
                        (self._lib.wavec_set_batch_size, int(batch_size)),
                        (self._lib.wavec_set_target_preset, _cstr(target))):
            _raise_on(fn(self._handle, arg), fn.__name__)

    def __del__(self):
        handle, self._handle = getattr(self, "_handle", None), None
        if handle:
            self._lib.wavec_destroy(handle)

    def _node(self, fn_name: str, *args) -> None:
        """Calls wavec_<...>(handle, *args); a failure raises with the library's message."""
        _raise_on(getattr(self._lib, fn_name)(self._handle, *args), fn_name)

    # ------------------------------------------------------------------ reference API
    def add_input(self, name: str, c: int, h: int = 1, w: int = 1, is_1d: bool = False) -> str:
        self._node("wavec_add_input", _cstr(name), int(c), int(h), int(w), int(bool(is_1d)))
        return name

    def add_conv2d(self, name: str, in_blob: str, out_blob: str, cin: int, cout: int, kh: int,
                   kw: int, weights: np.ndarray, bias: Optional[np.ndarray] = None,
                   stride: int = 1, pad: int = 0, act: Optional[str] = "silu",
                   res_blob: Optional[str] = None) -> str:
        """weights: [cout][cin][kh][kw] (fp32 or anything convertible); bias: [cout] or None."""
        w, b = _f32(weights), _f32(bias)
        self._node("wavec_add_conv2d", _cstr(name), _cstr(in_blob), _cstr(out_blob), int(cin),
                   int(cout), int(kh), int(kw), int(stride), int(pad), ACT_MAP.get(act, 0),
                   _pointer(w, C.c_float), _pointer(b, C.c_float), _cstr(res_blob))
        return out_blob

    def add_linear(self, name: str, in_blob: str, out_blob: str, cin: int, cout: int,
                   weights: np.ndarray, bias: Optional[np.ndarray] = None,
                   act: Optional[str] = None, res_blob: Optional[str] = None) -> str:
        """weights [cout][cin]: fp16 / uint16 arrays go through the fp16 entry point unchanged,
        anything else is passed as fp32 (rounded to fp16 by the compiler)."""
        b = _f32(bias)
        if weights.dtype in (np.float16, np.uint16):
            fn, w = "wavec_add_linear_f16", _f16_bits(weights)
            wp = _pointer(w, C.c_uint16)
        else:
            fn, w = "wavec_add_linear_f32", _f32(weights)
            wp = _pointer(w, C.c_float)
        self._node(fn, _cstr(name), _cstr(in_blob), _cstr(out_blob), int(cin), int(cout),
                   ACT_MAP.get(act, 0), wp, _pointer(b, C.c_float), _cstr(res_blob))
        return out_blob

    def add_rmsnorm(self, name: str, in_blob: str, out_blob: str, dim: int, gamma: np.ndarray,
                    eps: float = 1e-5, pre_folded: bool = False) -> str:
        g = _f32(gamma)
        self._node("wavec_add_rmsnorm", _cstr(name), _cstr(in_blob), _cstr(out_blob), int(dim),
                   C.c_float(eps), _pointer(g, C.c_float), int(bool(pre_folded)))
        return out_blob

    def add_swiglu(self, name: str, gate_blob: str, up_blob: str, out_blob: str,
                   dim: int = 0) -> str:
        """Element-wise gate * up (the gate's SiLU is its projection's epilogue); `dim` is
        accepted for the reference signature and not used (the shapes come from the blobs)."""
        self._node("wavec_add_swiglu", _cstr(name), _cstr(gate_blob), _cstr(up_blob),
                   _cstr(out_blob))
        return out_blob

    def add_rope_gqa_attn(self, name: str, q_blob: str, k_blob: str, v_blob: str, out_blob: str,
                          h_q: int, h_kv: int, head_dim: int, rope_theta: float = 10000.0,
                          llama3_scaling: bool = False) -> str:
        self._node("wavec_add_rope_gqa_attn", _cstr(name), _cstr(q_blob), _cstr(k_blob),
                   _cstr(v_blob), _cstr(out_blob), int(h_q), int(h_kv), int(head_dim),
                   C.c_float(rope_theta), int(bool(llama3_scaling)))
        return out_blob

    def add_maxpool(self, name: str, in_blob: str, out_blob: str, kernel_size: int = 5,
                    stride: int = 1, pad: int = 2) -> str:
        self._node("wavec_add_maxpool", _cstr(name), _cstr(in_blob), _cstr(out_blob),
                   int(kernel_size), int(stride), int(pad))
        return out_blob

    def add_upsample2x(self, name: str, in_blob: str, out_blob: str) -> str:
        self._node("wavec_add_upsample2x", _cstr(name), _cstr(in_blob), _cstr(out_blob))
        return out_blob

    def add_split(self, name: str, in_blob: str, out_blobs: Sequence[str]) -> List[str]:
        names = list(out_blobs)
        self._node("wavec_add_split", _cstr(name), _cstr(in_blob), len(names), _name_array(names))
        return names

    def add_slice(self, name: str, in_blob: str, out_blobs: Sequence[str],
                  slice_sizes: Sequence[int]) -> List[str]:
        names, sizes = list(out_blobs), [int(s) for s in slice_sizes]
        self._node("wavec_add_slice", _cstr(name), _cstr(in_blob), len(names), _name_array(names),
                   (C.c_int * len(sizes))(*sizes))
        return names

    def add_concat(self, name: str, in_blobs: Sequence[str], out_blob: str) -> str:
        names = list(in_blobs)
        self._node("wavec_add_concat", _cstr(name), len(names), _name_array(names),
                   _cstr(out_blob))
        return out_blob

    def set_output(self, out_blob: str) -> None:
        self._node("wavec_set_output", _cstr(out_blob))

    def compile(self) -> WavePlan:
        """Runs the five compiler passes and returns the plan with its summary."""
        if self._lib.wavec_compile(self._handle) != 0:
            raise RuntimeError(f"the wave compiler rejected this graph: {last_error()}")
        raw = self._lib.wavec_get_summary_json(self._handle)
        return WavePlan(self._handle, self._lib, json.loads(raw) if raw else {}, owner=self)

    # ------------------------------------------------------------------ extensions
    def add_upconv2x2(self, name: str, in_blob: str, out_blob: str, cin: int, cout: int,
                      weights: np.ndarray, bias: Optional[np.ndarray] = None) -> str:
        """2x2 stride-2 transposed convolution, weights [cout][cin][2][2] (the reference exports
        wavec_add_upconv2x2 but its Python module has no method for it)."""
        w, b = _f32(weights), _f32(bias)
        self._node("wavec_add_upconv2x2", _cstr(name), _cstr(in_blob), _cstr(out_blob), int(cin),
                   int(cout), _pointer(w, C.c_float), _pointer(b, C.c_float))
        return out_blob

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
        b = _opt_f16_bits(bias)
        self._node("wavec_add_sparse_wave", _cstr(name), _cstr(in_blob), _cstr(out_blob),
                   int(cout), int(fan_in), int(cluster), _pointer(r, C.c_uint32),
                   _pointer(w, C.c_uint16), _pointer(b, C.c_uint16), ACT_MAP.get(act, 0),
                   _cstr(res_blob))
        return out_blob

    def add_cluster_wave(self, name: str, in_blob: str, out_blob: str, starts: np.ndarray,
                         seg_len: int, weights: np.ndarray, bias: Optional[np.ndarray] = None,
                         cluster: int = 1, act: Optional[str] = None,
                         res_blob: Optional[str] = None) -> str:
        """starts: [cout/cluster, K] first input channel of each dendritic cluster of seg_len
        consecutive channels; weights [cout, K*seg_len]."""
        w = _f16_bits(weights)
        st = np.ascontiguousarray(starts, dtype=np.uint32)
        cout, K = w.shape[0], st.shape[1]
        if st.shape[0] * cluster != cout or w.shape[1] != K * seg_len:
            raise ValueError("starts / weights shapes do not match cout, cluster, K, seg_len")
        b = _opt_f16_bits(bias)
        self._node("wavec_add_cluster_wave", _cstr(name), _cstr(in_blob), _cstr(out_blob),
                   int(cout), int(K), int(seg_len), int(cluster), _pointer(st, C.c_uint32),
                   _pointer(w, C.c_uint16), _pointer(b, C.c_uint16), ACT_MAP.get(act, 0),
                   _cstr(res_blob))
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
        b = _opt_f16_bits(bias)
        self._node("wavec_add_pruned_wave", _cstr(name), _cstr(in_blob), _cstr(out_blob),
                   int(cout), int(K), int(seg_len), int(tile), _pointer(st, C.c_uint32),
                   _pointer(w, C.c_uint16), _pointer(b, C.c_uint16), ACT_MAP.get(act, 0),
                   _cstr(res_blob))
        return out_blob

    def add_token_shift(self, name: str, in_blob: str, out_blob: str, mu: np.ndarray,
                        seq_len: int, decode: bool = False) -> str:
        """Causal depth-wise mix over the last rf tokens of each request; mu: [dim, rf]."""
        m = _f16_bits(mu)
        dim, rf = m.shape
        self._node("wavec_add_token_shift", _cstr(name), _cstr(in_blob), _cstr(out_blob),
                   int(dim), int(rf), int(seq_len), _pointer(m, C.c_uint16), int(bool(decode)))
        return out_blob

    def add_embedding(self, name: str, tok_blob: str, out_blob: str, table: np.ndarray) -> str:
        """y[c][t] = table[id[t]][c]; table: [vocab, dim]."""
        t = _f16_bits(table)
        vocab, dim = t.shape
        self._node("wavec_add_embedding", _cstr(name), _cstr(tok_blob), _cstr(out_blob),
                   int(vocab), int(dim), _pointer(t, C.c_uint16))
        return out_blob

    def add_argmax(self, name: str, in_blob: str, out_blob: str) -> str:
        self._node("wavec_add_argmax", _cstr(name), _cstr(in_blob), _cstr(out_blob))
        return out_blob

    def save_tcff(self, path: Union[str, Path], model_prefix: str = "K44Model",
                  include_geometry: bool = True) -> None:
        self._node("wavec_save_tcff_ex", _cstr(path), _cstr(model_prefix), 1,
                   int(bool(include_geometry)))


class DeviceBuffer:
    """Device memory allocated by libk44wavec.so (hipMalloc / hipFree) for the stand-alone
    kernels; `.ptr` is the device address."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self._lib = get_lib()
        self.ptr = self._lib.wavec_dev_malloc(self.nbytes)
        if not self.ptr:
            raise RuntimeError(f"wavec_dev_malloc({self.nbytes}): {last_error()}")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError(f"{a.nbytes} bytes do not fit a {self.nbytes}-byte device buffer")
        _raise_on(self._lib.wavec_dev_upload(self.ptr, a.ctypes.data, a.nbytes),
                  "wavec_dev_upload")

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError(f"{out.nbytes} bytes requested from a {self.nbytes}-byte buffer")
        _raise_on(self._lib.wavec_dev_download(out.ctypes.data, self.ptr, out.nbytes),
                  "wavec_dev_download")
        return out

    def free(self) -> None:
        ptr, self.ptr = self.ptr, None
        if ptr:
            self._lib.wavec_dev_free(ptr)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def device_synchronize() -> None:
    _raise_on(get_lib().wavec_dev_synchronize(), "wavec_dev_synchronize")


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
    _raise_on(get_lib().wavec_k44_f16_forward_token64(
        _dev_ptr(Y), _dev_ptr(X), _dev_ptr(cluster_indices), _dev_ptr(cluster_weights_wmma),
        _dev_ptr(neuron_bias) or None, int(batch_size), int(Cin), int(Cout), int(B_vec16),
        int(cluster_size), _dev_ptr(stream) or None), "wavec_k44_f16_forward_token64")


def interleave_weights_wmma(dst_wmma, src_compact, num_output_neurons: int, B_vec8: int,
                            stream=None) -> None:
    """GPU weight interleave: row-major [neurons][8*B_vec8] fp16 -> RDNA4 WMMA vector order."""
    _raise_on(get_lib().wavec_interleave_weights_wmma(
        _dev_ptr(dst_wmma), _dev_ptr(src_compact), int(num_output_neurons), int(B_vec8),
        _dev_ptr(stream) or None), "wavec_interleave_weights_wmma")


def argmax_f16(ids, logits, vocab: int, stride: int, tokens: int, stream=None) -> None:
    """ids[t] = argmax_c logits[c][t] (lowest channel on ties) on caller-owned device memory:
    logits [vocab][stride] fp16, ids [tokens] uint32.  Asynchronous on `stream`."""
    _raise_on(get_lib().wavec_argmax_f16(_dev_ptr(ids), _dev_ptr(logits), int(vocab), int(stride),
                                         int(tokens), _dev_ptr(stream) or None),
              "wavec_argmax_f16")


def argmax_f16_noalloc(ids, logits, vocab: int, stride: int, tokens: int, stream=None) -> None:
    """argmax_f16 without any allocation: the partials live in a fixed per-GPU array of the
    library (strides up to 524,288 tokens); calls that overlap on one GPU race."""
    _raise_on(get_lib().wavec_argmax_f16_noalloc(_dev_ptr(ids), _dev_ptr(logits), int(vocab),
                                                 int(stride), int(tokens),
                                                 _dev_ptr(stream) or None),
              "wavec_argmax_f16_noalloc")

"""The C-ABI boundary: libk44wavec.so loads, exports every entry point include/k44wavec.h
declares (the reference's 30 plus the build extensions), and behaves on error paths."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]

# The reference's extern "C" entry points (wavec/k44_wave_executor.cu:644-986).
REFERENCE_ABI = [
    "wavec_create", "wavec_destroy", "wavec_gpu_release", "wavec_add_input", "wavec_add_flatten",
    "wavec_add_conv2d", "wavec_add_conv2d_f16", "wavec_add_linear_f32", "wavec_add_linear_f16",
    "wavec_add_linear_bf16", "wavec_add_upconv2x2", "wavec_add_maxpool", "wavec_add_upsample2x",
    "wavec_add_rmsnorm", "wavec_add_swiglu", "wavec_add_rope_gqa_attn", "wavec_add_split",
    "wavec_add_slice", "wavec_add_concat", "wavec_set_output", "wavec_set_reuse_canvas",
    "wavec_set_batch_size", "wavec_set_target_preset", "wavec_compile", "wavec_get_summary_json",
    "wavec_save_tcff", "wavec_save_tcff_ex", "wavec_load_tcff_weights", "wavec_gpu_init_plan",
    "wavec_gpu_infer_f32",
]


def header_symbols():
    text = (ROOT / "include" / "k44wavec.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wavec_\w+)\s*\(", text)))


def test_header_declares_reference_abi_and_extensions(wavec):
    hdr = header_symbols()
    assert set(REFERENCE_ABI) <= set(hdr)
    assert len(REFERENCE_ABI) == 30
    assert set(hdr) == set(wavec.REFERENCE_SYMBOLS) | set(wavec.EXTENSION_SYMBOLS)
    assert list(wavec.REFERENCE_SYMBOLS) == REFERENCE_ABI


def test_library_exports_every_declared_symbol(wavec):
    lib = ctypes.CDLL(str(wavec.LIB_PATH))
    missing = [s for s in header_symbols() if not hasattr(lib, s)]
    assert not missing


def test_null_handle_returns_error(wavec):
    lib = wavec.get_lib()
    assert lib.wavec_compile(None) == -1
    assert lib.wavec_gpu_init_plan(None) == -1
    assert lib.wavec_gpu_release(None) == -1
    assert lib.wavec_add_input(None, b"x", 1, 1, 64, 1) == -1
    assert lib.wavec_save_tcff(None, b"/tmp/x.tcff", b"p") == -1
    assert lib.wavec_load_tcff_weights(None, b"/tmp/x.tcff") == -1
    assert lib.wavec_get_summary_json(None) == b"{}"
    assert lib.wavec_gpu_exec_report_json(None) == b"{}"
    lib.wavec_destroy(None)  # no-op


def test_gpu_entry_points_require_init(wavec):
    lib = wavec.get_lib()
    h = lib.wavec_create(0, 0, 0, 1)
    try:
        x = np.zeros(4, np.float32)
        out = np.zeros(4, np.float32)
        ms = ctypes.c_float()
        p = x.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        q = out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        assert lib.wavec_gpu_infer_f32(h, p, 4, q, 4, ctypes.byref(ms)) == -1
        assert "wavec_gpu_init_plan" in wavec.last_error()
        assert lib.wavec_gpu_execute(h, 1, ctypes.byref(ms)) == -1
    finally:
        lib.wavec_destroy(h)


def test_invalid_sparse_wave_is_rejected(wavec):
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", 100, 1, 64, is_1d=True)
    rows = np.zeros((3, 4), np.uint32)
    w = np.zeros((6, 4), np.uint16)
    rc = g._lib.wavec_add_sparse_wave(
        g._handle, b"s", b"x", b"y", 6, 4, 4,  # cluster 4 does not divide cout 6
        rows.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
        w.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), None, 1, None)
    assert rc == -1 and "cluster" in wavec.last_error()
    # a synapse position beyond the input's channel count fails at compile time
    g.add_sparse_wave("s2", "x", "y2", np.full((2, 4), 100, np.uint32), np.zeros((2, 4),
                                                                                 np.float16))
    with pytest.raises(RuntimeError, match="beyond the input"):
        g.compile()


def test_unsupported_plans_fail_init_with_message(wavec):
    """The executor refuses what it cannot run instead of silently skipping it."""
    g2 = wavec.WaveGraph(kv_cache_max_seq=0)
    g2.add_input("t", 128, 1, 64, is_1d=True)
    g2.add_rope_gqa_attn("a", "t", "t", "t", "o", 2, 2, 64)
    plan2 = g2.compile()
    with pytest.raises(RuntimeError, match="ROPE_GQA_ATTN_1D"):
        plan2.init_gpu()


# Host-side argument checks are tested with stand-in pointers (1, 2, ...) that no device could
# dereference: such a test runs only where no GPU is present (no /dev/kfd), so a check that
# ever stopped rejecting could not send them to a GPU.
host_only = pytest.mark.skipif(Path("/dev/kfd").exists(),
                               reason="stand-in device pointers: host-only test")


@host_only
def test_token64_and_interleave_validate_before_touching_the_gpu(wavec):
    """Argument checks of the stand-alone kernels run on the host (no device work on failure)."""
    lib = wavec.get_lib()
    assert lib.wavec_k44_f16_forward_token64(None, None, None, None, None, 64, 10, 64, 2, 64,
                                             None) == -1
    assert "required" in wavec.last_error()
    # cluster size 8 (not a multiple of 16) is refused
    assert lib.wavec_k44_f16_forward_token64(1, 1, 1, 1, None, 64, 10, 64, 2, 8, None) == -1
    assert "cluster_size" in wavec.last_error()
    assert lib.wavec_k44_f16_forward_token64(1, 1, 1, 1, None, 0, 10, 64, 2, 64, None) == -1
    assert lib.wavec_interleave_weights_wmma(1, 1, 20, 4, None) == -1  # 20 neurons
    assert lib.wavec_interleave_weights_wmma(1, 1, 32, 3, None) == -1  # odd B_vec8
    assert lib.wavec_interleave_weights_wmma(None, 1, 32, 4, None) == -1


def test_tuning_switches_set_get_reset(wavec):
    wavec.reset_tuning()
    for key in ("path", "dma", "fuse", "group", "t64_ring", "narrow_chunk"):
        assert wavec.get_tuning(key) == -1
    wavec.set_tuning("fuse", 0)
    wavec.set_tuning("narrow_chunk", 32)
    assert wavec.get_tuning("fuse") == 0 and wavec.get_tuning("narrow_chunk") == 32
    with pytest.raises(RuntimeError, match="unknown tuning key"):
        wavec.set_tuning("no_such_switch", 1)
    with pytest.raises(RuntimeError, match="-1"):
        wavec.set_tuning("fuse", -5)
    with pytest.raises(RuntimeError, match="unknown tuning key"):
        wavec.get_tuning("no_such_switch")
    # values a switch does not honour are refused (the old value stays)
    wavec.reset_tuning()
    for key, bad in (("dma_stages", 3), ("ksplit", 2), ("xcd_order", 7), ("path", 2),
                     ("narrow_chunk", 15), ("narrow_wgs", 0), ("narrow_reduce", 2),
                     ("t64_ring", 3), ("dma_prod", 2), ("narrow_pre", 2), ("narrow_local", 2),
                     ("embed_refresh", 2), ("narrow_byy", 2)):
        with pytest.raises(RuntimeError, match="not honoured"):
            wavec.set_tuning(key, bad)
        assert wavec.get_tuning(key) == -1
    for key, good in (("dma_stages", 4), ("ksplit", 4), ("xcd_order", 2), ("narrow_reduce", 0),
                      ("t64_ring", 2), ("dma_prod", 1), ("narrow_pre", 0), ("narrow_local", 0)):
        wavec.set_tuning(key, good)
        assert wavec.get_tuning(key) == good
    wavec.reset_tuning()
    assert wavec.get_tuning("fuse") == -1 and wavec.get_tuning("narrow_chunk") == -1


# The reference binding's public methods and their parameters (wavec/wavec.py:147-344): the
# drop-in contract of snntome_amd.wavec.
REFERENCE_PY_API = {
    "WavePlan": {
        "__init__": ["self", "handle", "lib", "summary"],
        "save_tcff": ["self", "tcff_path", "model_prefix"],
        "load_tcff_weights": ["self", "tcff_path"],
        "init_gpu": ["self"],
        "infer_f32": ["self", "x"],
    },
    "WaveGraph": {
        "__init__": ["self", "max_B_per_wave", "default_S", "kv_cache_max_seq",
                     "fold_rmsnorm_gamma", "reuse_canvas", "batch_size", "target"],
        "add_input": ["self", "name", "c", "h", "w", "is_1d"],
        "add_conv2d": ["self", "name", "in_blob", "out_blob", "cin", "cout", "kh", "kw",
                       "weights", "bias", "stride", "pad", "act", "res_blob"],
        "add_linear": ["self", "name", "in_blob", "out_blob", "cin", "cout", "weights", "bias",
                       "act", "res_blob"],
        "add_rmsnorm": ["self", "name", "in_blob", "out_blob", "dim", "gamma", "eps",
                        "pre_folded"],
        "add_swiglu": ["self", "name", "gate_blob", "up_blob", "out_blob", "dim"],
        "add_rope_gqa_attn": ["self", "name", "q_blob", "k_blob", "v_blob", "out_blob", "h_q",
                              "h_kv", "head_dim", "rope_theta", "llama3_scaling"],
        "add_maxpool": ["self", "name", "in_blob", "out_blob", "kernel_size", "stride", "pad"],
        "add_upsample2x": ["self", "name", "in_blob", "out_blob"],
        "add_split": ["self", "name", "in_blob", "out_blobs"],
        "add_slice": ["self", "name", "in_blob", "out_blobs", "slice_sizes"],
        "add_concat": ["self", "name", "in_blobs", "out_blob"],
        "set_output": ["self", "out_blob"],
        "compile": ["self"],
    },
}
REFERENCE_PY_DEFAULTS = {
    ("WaveGraph", "__init__"): (288, 0, 2048, True, False, 1, "auto"),
    ("WaveGraph", "add_conv2d"): (None, 1, 0, "silu", None),
    ("WaveGraph", "add_linear"): (None, None, None),
    ("WaveGraph", "add_rmsnorm"): (1e-5, False),
    ("WaveGraph", "add_maxpool"): (5, 1, 2),
    ("WaveGraph", "add_rope_gqa_attn"): (10000.0, False),
    ("WavePlan", "save_tcff"): ("K44Model",),
}


def test_python_api_keeps_reference_signatures(wavec):
    import inspect

    assert {k: v for k, v in wavec.ACT_MAP.items() if v <= 4} == {
        None: 0, "none": 0, "identity": 0, "linear": 0, "relu": 1, "sigmoid": 2, "silu": 3,
        "swish": 3, "leaky_relu": 4}
    for cls_name, methods in REFERENCE_PY_API.items():
        cls = getattr(wavec, cls_name)
        for m, params in methods.items():
            sig = inspect.signature(getattr(cls, m))
            got = list(sig.parameters)
            assert got[:len(params)] == params, (cls_name, m, got)
            extra = [p for p in list(sig.parameters.values())[len(params):]]
            assert all(p.default is not inspect.Parameter.empty for p in extra), (cls_name, m)
            want = REFERENCE_PY_DEFAULTS.get((cls_name, m))
            if want is not None:
                defs = tuple(p.default for p in sig.parameters.values()
                             if p.default is not inspect.Parameter.empty)
                assert defs[:len(want)] == want, (cls_name, m, defs)


@host_only
def test_standalone_argmax_validates_before_touching_the_gpu(wavec):
    lib = wavec.get_lib()
    # logits must be 8-byte aligned and ids 4-byte aligned (the kernels' load / store widths),
    # in both argmax entry points, refused before any launch
    for fn in ("wavec_argmax_f16", "wavec_argmax_f16_noalloc"):
        for logits in (2, 4, 6, 0x1002):
            assert getattr(lib, fn)(64, logits, 100, 64, 10, None) == -1
            assert "8-byte aligned" in wavec.last_error()
        assert getattr(lib, fn)(66, 64, 100, 64, 10, None) == -1
        assert "4-byte aligned" in wavec.last_error()
    assert lib.wavec_argmax_f16(None, 1, 100, 64, 10, None) == -1
    assert "required" in wavec.last_error()
    assert lib.wavec_argmax_f16(64, 64, 100, 100, 10, None) == -1  # stride not a multiple of 64
    assert lib.wavec_argmax_f16(64, 64, 100, 64, 65, None) == -1  # more tokens than the stride
    assert lib.wavec_argmax_f16(64, 64, 0, 64, 10, None) == -1

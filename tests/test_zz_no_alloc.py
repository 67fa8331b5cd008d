"""The allocation-free argmax (wavec_argmax_f16_noalloc) against the allocating entry point
(wavec_argmax_f16) through the C ABI: two calls in a row, the second with a smaller input (the
shared workspace keeps the first call's partials), ids bit for bit equal and equal to the
lowest-index rule; sizes beyond the fixed workspace are refused before any GPU work."""
import numpy as np
import pytest

from oracle import llm_oracle as lo

pytestmark = pytest.mark.gpu


def _case(rng, V, stride, tokens):
    x = (rng.standard_normal((V, stride)) * 3).astype(np.float16)
    for t in range(0, tokens, 7):  # planted ties: the lowest channel must win
        cs = np.sort(rng.choice(V, size=2, replace=False))
        x[cs, t] = np.float16(40.0)
    return x


def _argmax(wavec, fn, x, tokens):
    V, stride = x.shape
    X = wavec.DeviceBuffer.from_array(x)
    ids = wavec.DeviceBuffer(tokens * 4)
    rc = getattr(wavec.get_lib(), fn)(ids.ptr, X.ptr, V, stride, tokens, None)
    assert rc == 0, wavec.last_error()
    wavec.device_synchronize()
    return ids.download(np.uint32, tokens)


def test_noalloc_argmax_matches_allocating_entry_point(wavec):
    rng = np.random.default_rng(4)
    for V, stride, tokens in [(32000, 2048, 2000), (700, 128, 70)]:  # second call smaller
        x = _case(rng, V, stride, tokens)
        want = lo.argmax(x, tokens)
        a = _argmax(wavec, "wavec_argmax_f16", x, tokens)
        b = _argmax(wavec, "wavec_argmax_f16_noalloc", x, tokens)
        print(f"[noalloc argmax] V={V} stride={stride} tokens={tokens}", flush=True)
        assert np.array_equal(b, a)
        assert np.array_equal(b, want)


def test_noalloc_argmax_refuses_sizes_beyond_its_workspace(wavec):
    lib = wavec.get_lib()
    # V = 1, stride 2^20: 2 * 1 chunk * 2^20 partial floats > the 2^20 the array holds.  Real
    # buffers of that size: were the size check ever to let the call through, the kernels
    # would compute a valid argmax instead of touching unmapped memory.
    stride = 1 << 20
    X = wavec.DeviceBuffer.from_array(np.zeros((1, stride), np.float16))
    ids = wavec.DeviceBuffer(64 * 4)
    assert lib.wavec_argmax_f16_noalloc(ids.ptr, X.ptr, 1, stride, 64, None) == -1
    assert "workspace" in wavec.last_error()

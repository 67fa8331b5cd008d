"""GPU parity of the stand-alone Token64 wave (wavec_k44_f16_forward_token64, the whitepaper
launcher's semantics: X [tile][Cin][64], per-cluster index rows, WMMA-ordered weights, bias,
round toward zero) and of the GPU weight interleave, through the C ABI on device memory
allocated with wavec_dev_malloc."""
import numpy as np
import pytest

from snntome_amd import synth

from wave_cases import TOL

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("neurons,B", [(16, 16), (64, 96), (48, 512)])
def test_interleave_matches_host_order(wavec, orc, neurons, B):
    rng = np.random.default_rng(neurons + B)
    w = rng.integers(0, 1 << 16, size=(neurons, B), dtype=np.uint16)
    src = wavec.DeviceBuffer.from_array(w)
    dst = wavec.DeviceBuffer(w.nbytes)
    wavec.interleave_weights_wmma(dst, src, neurons, B // 8)
    wavec.device_synchronize()
    got = dst.download(np.uint16, w.size)
    assert np.array_equal(got, orc.raw_to_wmma(w).ravel())


_LAST_Y = [None]  # output bits of the last _token64_case call


def _token64_case(wavec, orc, *, Cin, Cout, cluster, B_vec16, batch, seed, bad_index=False):
    rng = np.random.default_rng(seed)
    B = 16 * B_vec16
    tiles = (batch + 63) // 64
    x = (rng.uniform(-1, 1, size=(tiles, Cin, 64))).astype(np.float16)
    idx = rng.integers(0, Cin, size=(Cout // cluster, B), dtype=np.int64).astype(np.uint32)
    if bad_index:
        idx[0, 3] = Cin + 5  # out of range: reads as a zero row
    w = (rng.standard_normal((Cout, B)) * 0.05).astype(np.float16)
    b = (rng.standard_normal(Cout) * 0.05).astype(np.float16)
    Xd = wavec.DeviceBuffer.from_array(x)
    Yd = wavec.DeviceBuffer.from_array(np.full((tiles, Cout, 64), 0xFFFF, np.uint16))
    Id = wavec.DeviceBuffer.from_array(idx)
    Wd = wavec.DeviceBuffer.from_array(orc.raw_to_wmma(w.view(np.uint16)))
    Bd = wavec.DeviceBuffer.from_array(b)
    wavec.forward_token64_f16(Yd, Xd, Id, Wd, Bd, batch, Cin, Cout, B_vec16, cluster)
    wavec.device_synchronize()
    y16 = Yd.download(np.float16, (tiles, Cout, 64))
    _LAST_Y[0] = y16.view(np.uint16).copy()
    y = y16.astype(np.float64)
    w_eff = w.copy()
    idx_eff = idx.astype(np.uint64)
    if bad_index:
        w_eff[:cluster, 3] = 0  # a zero row contributes nothing
        idx_eff[0, 3] = 0
    errs = []
    for t in range(tiles):
        canvas = x[t].reshape(-1)
        seg = (idx_eff * 64).ravel()
        ref = orc.wave_f64(canvas, seg, w_eff, b, None, B, 1, cluster, 64, 64, 64, "none")
        errs.append(orc.rel_err(y[t], ref))
        # round toward zero: never larger in magnitude than the exact sum beyond fp32 noise
        assert np.all(np.abs(y[t]) <= np.abs(ref) * (1 + 2 ** -12) + 1e-5)
    return max(errs)


@pytest.mark.parametrize("cluster", [16, 32, 48, 64, 128])
@pytest.mark.parametrize("B_vec16,batch", [(4, 64), (3, 100), (8, 300)])
def test_token64_matches_oracle(wavec, orc, cluster, B_vec16, batch):
    """Cluster sizes 16..128 (16/32/64-neuron waves), even and odd B_vec16 (a half-empty last
    k-step), ragged batches (2 and 5 tiles: workgroups with idle waves)."""
    err = _token64_case(wavec, orc, Cin=3000, Cout=cluster * max(2, 128 // cluster), cluster=cluster,
                        B_vec16=B_vec16, batch=batch, seed=cluster * 100 + B_vec16)
    _log(f"[token64 cluster={cluster} B_vec16={B_vec16} batch={batch}] rel err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("cluster,batch", [(64, 64), (64, 256), (128, 128)])
def test_token64_out_of_range_index_reads_zero(wavec, orc, cluster, batch):
    """Per-wave kernel (one tile), 64-neuron and 128-neuron ring kernels."""
    err = _token64_case(wavec, orc, Cin=500, Cout=cluster, cluster=cluster, B_vec16=2,
                        batch=batch, seed=7, bad_index=True)
    assert err <= TOL


@pytest.mark.parametrize("cluster,B_vec16,batch", [(64, 2, 256), (128, 8, 512), (192, 6, 256),
                                                   (64, 64, 256), (256, 4, 256), (512, 256, 256),
                                                   (128, 4, 128), (256, 2, 384)])
def test_token64_ring_matches_oracle_and_fallback(wavec, orc, tuning, cluster, B_vec16,
                                                  batch):
    """Shapes the LDS-ring kernels take (clusters of whole 64-neuron blocks, whole 4-tile
    groups for 64-neuron workgroups, whole 2-tile groups for 128-neuron workgroups, even
    B_vec16): within tolerance of the oracle, and bit-identical to the per-wave kernel (same
    k-step accumulation order from the bias).  Tuning switch t64_ring: -1 automatic, 1 the
    64-neuron ring only, 2 the 128-neuron ring only, 0 per-wave kernel."""
    Cout = cluster * 2
    ys = {}
    for ring in ("auto", "1", "2", "0"):
        tuning("t64_ring", -1 if ring == "auto" else int(ring))
        err = _token64_case(wavec, orc, Cin=5000, Cout=Cout, cluster=cluster, B_vec16=B_vec16,
                            batch=batch, seed=cluster + B_vec16)
        _log(f"[token64 ring={ring} cluster={cluster} B_vec16={B_vec16} batch={batch}] "
             f"rel err {err:.3e}")
        assert err <= TOL
        ys[ring] = _LAST_Y[0]
    for ring in ("auto", "1", "2"):
        assert np.array_equal(ys[ring], ys["0"]), ring


@pytest.mark.parametrize("batch", [64, 256])
def test_token64_64bit_substrate(wavec, orc, batch):
    """Cin = 40,000,000 positions (5.12 GB per 64-token tile, beyond 32-bit byte offsets),
    filled on the device with the synthetic generator; indices spread over the whole range,
    the last position included.  Batch 256 takes the LDS-ring kernel (tiles 1..3 at offsets
    past 5 GB)."""
    Cin, Cout, cluster, B_vec16, seed = 40_000_000, 64, 64, 4, 17
    tiles = batch // 64
    B = 16 * B_vec16
    rng = np.random.default_rng(11)
    idx = rng.integers(0, Cin, size=(1, B), dtype=np.int64)
    idx[0, :8] = [Cin - 1, (1 << 25) + 1, 1 << 25, 0, 33_554_431, 39_999_000, 12, Cin - 2]
    idx = idx.astype(np.uint32)
    _log("[token64 64-bit] filling a 5.12 GB substrate on the device")
    X = wavec.DeviceBuffer(tiles * Cin * 64 * 2)
    assert wavec.get_lib().wavec_dev_fill_uniform(X.ptr, tiles * Cin, 64, 64, 0, seed) == 0
    w = (rng.standard_normal((Cout, B)) * 0.05).astype(np.float16)
    b = (rng.standard_normal(Cout) * 0.05).astype(np.float16)
    Y = wavec.DeviceBuffer(tiles * Cout * 64 * 2)
    Id = wavec.DeviceBuffer.from_array(idx)
    Wd = wavec.DeviceBuffer.from_array(orc.raw_to_wmma(w.view(np.uint16)))
    Bd = wavec.DeviceBuffer.from_array(b)
    wavec.forward_token64_f16(Y, X, Id, Wd, Bd, batch, Cin, Cout, B_vec16, cluster)
    wavec.device_synchronize()
    X.free()
    y = Y.download(np.float16, (tiles, Cout, 64)).astype(np.float64)
    seg = np.arange(B, dtype=np.uint64) * 64
    for t in range(tiles):  # tile t's row p is generator position t * Cin + p
        rows = synth.substrate_rows(seed, idx[0].astype(np.uint64) + t * Cin, 64)
        ref = orc.wave_f64(rows.view(np.uint16).reshape(-1), seg, w, b, None, B, 1, cluster, 64,
                           64, 64, "none")
        err = orc.rel_err(y[t], ref)
        _log(f"[token64 64-bit batch={batch} tile {t}] rel err {err:.3e}")
        assert err <= TOL

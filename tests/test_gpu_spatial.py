"""2-D (spatial) plans on the GPU: waves over the padded-plane tile layout (3x3 taps shifted by
one element, masked tiles for widths that are not multiples of 64), the polyphase stride-2
convolution, pools, upsampling, the 2x2 transposed convolution, halo hygiene and batched frames,
against the CPU restatement in oracle/cnn_oracle.py."""
import numpy as np
import pytest

from oracle import cnn_oracle as co
from oracle import oracle as orc

from wave_cases import TOL

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _f16(rng, shape, s=1.0):
    return (rng.standard_normal(shape) * s).astype(np.float16)


def _conv_params(rng, cin, cout, k, s=0.2):
    return (_f16(rng, (cout, cin, k, k), s / np.sqrt(cin * k * k) * 3),
            _f16(rng, (cout,), 0.05))


def _run(plan, x):
    """infer_f32 of frame 0 -> fp16-valued float64 array [C][H][W]."""
    y, _ = plan.infer_f32(x[0].astype(np.float32))
    return y.astype(np.float64)


@pytest.mark.parametrize("H,W", [(8, 64), (7, 20), (5, 30), (3, 130), (6, 192)])
@pytest.mark.parametrize("act", ["relu", "gelu"])
def test_conv3x3_same(wavec, H, W, act):
    rng = np.random.default_rng(H * 1000 + W)
    cin, cout = 5, 24
    w, b = _conv_params(rng, cin, cout, 3)
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("img", cin, H, W)
    g.add_conv2d("c", "img", "y", cin, cout, 3, 3, w.astype(np.float32), b.astype(np.float32),
                 stride=1, pad=1, act=act)
    plan = g.compile()
    plan.init_gpu()
    assert plan.exec_report()["waves"][0]["path"] == "valu_gather_tile"
    x = _f16(rng, (1, cin, H, W))
    got = _run(plan, x)
    ref = co.conv2d_f64(x, w, b, 1, 1, act)[0]
    err = orc.rel_err(got, ref)
    _log(f"[conv3x3 {H}x{W} {act}] rel err {err:.3e}")
    assert err <= TOL


def test_conv_residual_1x1_and_stride2(wavec):
    rng = np.random.default_rng(7)
    H, W, c0 = 16, 64, 6
    w1, b1 = _conv_params(rng, c0, c0, 3)
    w2, b2 = _conv_params(rng, c0, 16, 1)
    w3, b3 = _conv_params(rng, 16, 12, 3)
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("img", c0, H, W)
    g.add_conv2d("c1", "img", "a", c0, c0, 3, 3, w1.astype(np.float32), b1.astype(np.float32),
                 stride=1, pad=1, act="silu", res_blob="img")
    g.add_conv2d("c2", "a", "b", c0, 16, 1, 1, w2.astype(np.float32), b2.astype(np.float32),
                 stride=1, pad=0, act="relu")
    g.add_conv2d("c3", "b", "y", 16, 12, 3, 3, w3.astype(np.float32), b3.astype(np.float32),
                 stride=2, pad=1, act="none")
    plan = g.compile()
    assert [c["type"] for c in plan.cmds] == ["K44_WAVE", "K44_WAVE", "S2D_2X2", "K44_WAVE"]
    plan.init_gpu()
    x = _f16(rng, (1, c0, H, W))
    got = _run(plan, x)
    a = co.conv2d_f64(x, w1, b1, 1, 1, "silu", x).astype(np.float16)
    bb = co.conv2d_f64(a, w2, b2, 1, 0, "relu").astype(np.float16)
    ref = co.conv2d_f64(bb, w3, b3, 2, 1)[0]
    scale = np.abs(ref).max()
    err = np.abs(got - ref).max() / scale
    _log(f"[residual/1x1/stride-2 chain] max|d|/max|ref| {err:.3e}")
    assert got.shape == (12, 8, 32)
    assert err <= 1e-2  # three layers, one fp16 rounding each (per-layer bound is TOL)


@pytest.mark.parametrize("H,W", [(8, 64), (6, 20), (10, 34)])
def test_pools_and_upsample_exact(wavec, H, W):
    """Max and nearest copies are exact in fp16: bit-identical to the restatement."""
    rng = np.random.default_rng(H + W)
    C = 7
    for op in ("maxpool2", "maxpool5", "upsample"):
        g = wavec.WaveGraph(kv_cache_max_seq=0)
        g.add_input("img", C, H, W)
        if op == "maxpool2":
            g.add_maxpool("p", "img", "y", kernel_size=2, stride=2)
        elif op == "maxpool5":
            g.add_maxpool("p", "img", "y", kernel_size=5, stride=1, pad=2)
        else:
            g.add_upsample2x("p", "img", "y")
        plan = g.compile()
        plan.init_gpu()
        x = _f16(rng, (1, C, H, W))
        got = _run(plan, x).astype(np.float16)
        ref = {"maxpool2": co.maxpool2, "maxpool5": co.maxpool5, "upsample": co.upsample2}[op](x)[0]
        _log(f"[{op} {H}x{W}] shape {got.shape}")
        assert got.shape == ref.shape
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("cout", [8, 16])
def test_upconv2x2(wavec, cout):
    rng = np.random.default_rng(cout)
    H, W, cin = 6, 32, 10
    w = _f16(rng, (cout, cin, 2, 2), 0.3)
    b = _f16(rng, (cout,), 0.05)
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("img", cin, H, W)
    g.add_upconv2x2("u", "img", "y", cin, cout, w.astype(np.float32), b.astype(np.float32))
    plan = g.compile()
    assert [c["type"] for c in plan.cmds] == ["K44_WAVE", "SCATTER_UP2X2"]
    plan.init_gpu()
    x = _f16(rng, (1, cin, H, W))
    got = _run(plan, x)
    ref = co.upconv2x2_f64(x, w, b)[0]
    err = orc.rel_err(got, ref)
    _log(f"[upconv cout={cout}] rel err {err:.3e}")
    assert got.shape == (cout, 2 * H, 2 * W)
    assert err <= TOL


def test_unet_block_end_to_end_and_halo_hygiene(wavec):
    """conv -> stride-2 conv -> maxpool -> upsample x2 -> concat with the skip -> conv: run
    twice, with a different input the second time, so stale canvas data from the first run sits
    where the second run's halos must read as zero padding."""
    rng = np.random.default_rng(11)
    H, W, c0 = 16, 40, 4
    w1, b1 = _conv_params(rng, c0, 8, 3)
    w2, b2 = _conv_params(rng, 8, 16, 3)
    w3, b3 = _conv_params(rng, 24, 8, 3)
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("img", c0, H, W)
    g.add_conv2d("c1", "img", "s", c0, 8, 3, 3, w1.astype(np.float32), b1.astype(np.float32),
                 stride=1, pad=1, act="relu")
    g.add_conv2d("c2", "s", "d", 8, 16, 3, 3, w2.astype(np.float32), b2.astype(np.float32),
                 stride=2, pad=1, act="relu")
    g.add_maxpool("mp", "d", "p", kernel_size=2, stride=2)
    g.add_upsample2x("u1", "p", "q")
    g.add_upsample2x("u2", "q", "r")
    g.add_concat("cat", ["s", "r"], "k")
    g.add_conv2d("c3", "k", "y", 24, 8, 3, 3, w3.astype(np.float32), b3.astype(np.float32),
                 stride=1, pad=1, act="none")
    plan = g.compile()
    plan.init_gpu()
    for run in range(2):
        x = _f16(rng, (1, c0, H, W), 1.0 + run)
        got = _run(plan, x)
        s = co.conv2d_f64(x, w1, b1, 1, 1, "relu").astype(np.float16)
        d = co.conv2d_f64(s, w2, b2, 2, 1, "relu").astype(np.float16)
        r = co.upsample2(co.upsample2(co.maxpool2(d)))
        k = np.concatenate([s, r], axis=1)
        ref = co.conv2d_f64(k, w3, b3, 1, 1)[0]
        err = np.abs(got - ref).max() / np.abs(ref).max()
        _log(f"[unet block run {run}] max|d|/max|ref| {err:.3e}")
        assert err <= 1e-2


def test_batched_frames_on_canvas(wavec):
    """Two frames per channel plane (batch_size 2): both frames written and read on the canvas
    through the restated layout."""
    rng = np.random.default_rng(5)
    H, W, cin, cout, F = 6, 24, 3, 16, 2
    w, b = _conv_params(rng, cin, cout, 3)
    g = wavec.WaveGraph(kv_cache_max_seq=0, batch_size=F)
    g.add_input("img", cin, H, W)
    g.add_conv2d("c", "img", "y", cin, cout, 3, 3, w.astype(np.float32), b.astype(np.float32),
                 stride=1, pad=1, act="relu")
    plan = g.compile()
    plan.init_gpu()
    lay = co.Layout2D(H, W, F)
    c = plan.cmds[0]
    x = _f16(rng, (F, cin, H, W))
    region = np.zeros(cin * lay.channel_stride, np.float16)
    region[lay.offsets(cin).ravel()] = x.ravel()
    plan.write_canvas(int(c["src_off"]), region)
    plan.execute(1)
    out = plan.read_canvas(int(c["y_off"]), cout * lay.channel_stride).view(np.float16)
    got = out[lay.offsets(cout)].astype(np.float64)
    ref = co.conv2d_f64(x, w, b, 1, 1, "relu")
    err = orc.rel_err(got, ref)
    _log(f"[frames={F}] rel err {err:.3e}")
    assert err <= TOL
    # halos of the output planes are zero padding
    halo = np.ones(cout * lay.channel_stride, bool)
    halo[lay.offsets(cout).ravel()] = False
    assert not out[halo].any()


def _t64_write(plan, off, lay, x):
    """x [F][C][H][W] fp16 -> the tensor region at `off` (halo elements zero)."""
    C = x.shape[1]
    buf = np.zeros(C * lay.channel_stride, np.float16)
    buf[lay.offsets(C).ravel()] = x.ravel()
    plan.write_canvas(int(off), buf)


def _t64_read(plan, off, lay, C):
    buf = plan.read_canvas(int(off), C * lay.channel_stride).view(np.float16)
    return buf[lay.offsets(C)]


@pytest.mark.parametrize("frames,reuse", [(64, False), (128, True)])
@pytest.mark.parametrize("H,W", [(6, 10), (8, 64), (5, 7)])
def test_token64_interleaved_image_plan(wavec, frames, reuse, H, W):
    """Plans of 64-frame interleaved images (batch 64, and batch 128 held as two 64-frame blocks
    with reuse_canvas): 3x3 and 1x1 convolutions (residual), 2x2 and 5x5 max pools, nearest
    upsampling, a stride-2 3x3 convolution gathering its input directly, and a 2x2 transposed
    convolution — every command against cnn_oracle on the tensors the device read (all frames);
    pools and copies bit for bit."""
    rng = np.random.default_rng(frames + 100 * H + W)
    cin, c1, c3, cu = 5, 16, 8, 16
    w1, b1 = _conv_params(rng, cin, c1, 3)
    w2, b2 = _conv_params(rng, c1, c1, 1)
    w3, b3 = _conv_params(rng, c1, c3, 3)
    wu, bu = _f16(rng, (cu, c3, 2, 2), 0.3), _f16(rng, (cu,), 0.05)
    f32 = lambda a: a.astype(np.float32)
    g = wavec.WaveGraph(kv_cache_max_seq=0, batch_size=frames, reuse_canvas=reuse)
    g.add_input("img", cin, H, W)
    g.add_conv2d("c1", "img", "a", cin, c1, 3, 3, f32(w1), f32(b1), stride=1, pad=1, act="relu")
    g.add_conv2d("c2", "a", "b", c1, c1, 1, 1, f32(w2), f32(b2), stride=1, pad=0, act="silu",
                 res_blob="a")
    g.add_maxpool("p", "b", "pb", kernel_size=2, stride=2)
    g.add_upsample2x("u", "pb", "ub")
    g.add_conv2d("c3", "ub", "d", c1, c3, 3, 3, f32(w3), f32(b3), stride=2, pad=1, act="none")
    g.add_maxpool("p5", "d", "e", kernel_size=5, stride=1, pad=2)
    g.add_upconv2x2("up", "e", "y", c3, cu, f32(wu), f32(bu))
    plan = g.compile()
    types = [c["type"] for c in plan.cmds]
    assert types == ["K44_WAVE", "K44_WAVE", "MAXPOOL_2X2", "UPSAMPLE_2X", "K44_WAVE",
                     "MAXPOOL_5X5", "K44_WAVE", "SCATTER_UP2X2"], types
    plan.init_gpu()
    assert {w["path"] for w in plan.exec_report()["waves"]} == {"valu_gather_tile"}
    F = frames
    lay = lambda h, w: co.Layout2D(h, w, F, tok64=True)
    x = _f16(rng, (F, cin, H, W))
    _t64_write(plan, plan.cmds[0]["src_off"], lay(H, W), x)
    Hp, Wp = H // 2, W // 2
    H3, W3 = (2 * Hp + 1) // 2, (2 * Wp + 1) // 2
    dev = {"img": x}
    steps = [  # (command, input tensors, output name, channels, H, W, reference, exact)
        ("img", "a", c1, H, W, lambda t: co.conv2d_f64(t["img"], w1, b1, 1, 1, "relu"), False),
        ("a", "b", c1, H, W, lambda t: co.conv2d_f64(t["a"], w2, b2, 1, 0, "silu", t["a"]), False),
        ("b", "pb", c1, Hp, Wp, lambda t: co.maxpool2(t["b"]), True),
        ("pb", "ub", c1, 2 * Hp, 2 * Wp, lambda t: co.upsample2(t["pb"]), True),
        ("ub", "d", c3, H3, W3, lambda t: co.conv2d_f64(t["ub"], w3, b3, 2, 1), False),
        ("d", "e", c3, H3, W3, lambda t: co.maxpool5(t["d"]), True),
        (None, None, 0, 0, 0, None, False),  # quadrant wave of the transposed convolution
        ("e", "y", cu, 2 * H3, 2 * W3, lambda t: co.upconv2x2_f64(t["e"], wu, bu), False),
    ]
    for i, (src, out, C, h, w, ref_fn, exact) in enumerate(steps):
        plan.execute_range(i, 1)
        if out is None:
            continue
        c = plan.cmds[i]
        assert (c["h_out"], c["w_out"]) == (h, w), (i, c["h_out"], c["w_out"])
        got = _t64_read(plan, c["y_off"], lay(h, w), C)
        dev[out] = got
        ref = ref_fn(dev)
        if exact:
            assert np.array_equal(got.view(np.uint16), ref.astype(np.float16).view(np.uint16)), out
        else:
            err = orc.rel_err(got.astype(np.float64), ref)
            _log(f"[token64 F={F} {H}x{W}] {out}: rel err {err:.3e}")
            assert err <= TOL, out


@pytest.mark.parametrize("frames,reuse", [(64, False), (128, True)])
@pytest.mark.parametrize("H,W", [(6, 10), (8, 16)])
def test_token64_dense_convs_on_mfma(wavec, tuning, frames, reuse, H, W):
    """Dense convolutions of 64-frame interleaved images take the MFMA kernels through per-pixel
    tile tables: a 3x3 convolution over 32 channels (phase-ordered into 9 segments of 32
    channels), a 1x1 over 64 channels with a residual, a stride-2 3x3 over 64 channels (register-
    staged and LDS-ring kernels, split-K) — each against cnn_oracle on the tensor the device
    read."""
    rng = np.random.default_rng(frames * 7 + H * W)
    c0, c1 = 32, 64
    w1, b1 = _conv_params(rng, c0, c1, 3)
    w2, b2 = _conv_params(rng, c1, c1, 1)
    w3, b3 = _conv_params(rng, c1, c0, 3)
    f32 = lambda a: a.astype(np.float32)
    g = wavec.WaveGraph(kv_cache_max_seq=0, batch_size=frames, reuse_canvas=reuse)
    g.add_input("img", c0, H, W)
    g.add_conv2d("c1", "img", "a", c0, c1, 3, 3, f32(w1), f32(b1), stride=1, pad=1, act="relu")
    g.add_conv2d("c2", "a", "b", c1, c1, 1, 1, f32(w2), f32(b2), stride=1, pad=0, act="silu",
                 res_blob="a")
    g.add_conv2d("c3", "b", "y", c1, c0, 3, 3, f32(w3), f32(b3), stride=2, pad=1, act="none")
    plan = g.compile()
    plan.init_gpu()
    rep = plan.exec_report()["waves"]
    _log(f"[token64 mfma F={frames} {H}x{W}] " + ", ".join(
        f"{w['path']} K={w['K']} S={w['S']} ksplit={w['ksplit']}" for w in rep))
    assert all(w["path"].startswith("mfma") for w in rep), rep
    lay = lambda h, w: co.Layout2D(h, w, frames, tok64=True)
    x = _f16(rng, (frames, c0, H, W))
    _t64_write(plan, plan.cmds[0]["src_off"], lay(H, W), x)
    dev = {"img": x}
    H3, W3 = (H + 1) // 2, (W + 1) // 2
    steps = [("a", c1, H, W, lambda t: co.conv2d_f64(t["img"], w1, b1, 1, 1, "relu")),
             ("b", c1, H, W, lambda t: co.conv2d_f64(t["a"], w2, b2, 1, 0, "silu", t["a"])),
             ("y", c0, H3, W3, lambda t: co.conv2d_f64(t["b"], w3, b3, 2, 1))]
    for i, (out, C, h, w, ref_fn) in enumerate(steps):
        plan.execute_range(i, 1)
        c = plan.cmds[i]
        got = _t64_read(plan, c["y_off"], lay(h, w), C)
        dev[out] = got
        err = orc.rel_err(got.astype(np.float64), ref_fn(dev))
        _log(f"[token64 mfma F={frames} {H}x{W}] {out}: rel err {err:.3e}")
        assert err <= TOL, out


@pytest.mark.parametrize("frames", [1, 3])
@pytest.mark.parametrize("H,W", [(8, 64), (7, 20), (5, 130)])
def test_single_frame_dense_convs_on_mfma(wavec, frames, H, W):
    """Dense convolutions of single-frame images (batch 1..63, the padded-plane layout: tiles
    and 3x3 tap shifts at any element offset, masked tiles spanning plane rows for widths that
    are not multiples of 64) take the MFMA tile kernel with rows shifted into place: a 3x3
    convolution over 64 channels (9 segments of 64) and a 1x1 with a residual; a stride-2 3x3
    follows.  Every command against cnn_oracle on the tensor the device read; the output halos
    stay zero padding."""
    rng = np.random.default_rng(frames * 11 + H * W)
    c0, c1 = 64, 64
    w1, b1 = _conv_params(rng, c0, c1, 3)
    w2, b2 = _conv_params(rng, c1, c1, 1)
    w3, b3 = _conv_params(rng, c1, 32, 3)
    f32 = lambda a: a.astype(np.float32)
    g = wavec.WaveGraph(kv_cache_max_seq=0, batch_size=frames)
    g.add_input("img", c0, H, W)
    g.add_conv2d("c1", "img", "a", c0, c1, 3, 3, f32(w1), f32(b1), stride=1, pad=1, act="relu")
    g.add_conv2d("c2", "a", "b", c1, c1, 1, 1, f32(w2), f32(b2), stride=1, pad=0, act="silu",
                 res_blob="a")
    g.add_conv2d("c3", "b", "y", c1, 32, 3, 3, f32(w3), f32(b3), stride=2, pad=1, act="none")
    plan = g.compile()
    plan.init_gpu()
    rep = plan.exec_report()["waves"]
    _log(f"[single-frame mfma F={frames} {H}x{W}] " + ", ".join(
        f"{w['path']} K={w['K']} S={w['S']} ksplit={w['ksplit']}" for w in rep))
    # the 3x3 and the 1x1 (dense index rows); the stride-2 convolution's index rows compile to
    # one-position segments (no dense tiling: the VALU tile kernel), checked all the same
    assert all(w["path"] == "mfma_tile" and "single-frame image" in w["why"] for w in rep[:2]), rep
    lay = lambda h, w: co.Layout2D(h, w, frames)
    x = _f16(rng, (frames, c0, H, W))
    region = np.zeros(c0 * lay(H, W).channel_stride, np.float16)
    region[lay(H, W).offsets(c0).ravel()] = x.ravel()
    plan.write_canvas(int(plan.cmds[0]["src_off"]), region)
    dev = {"img": x}
    # the stride-2 convolution (S2D polyphase planes, as the reference compiles it) produces
    # floor(H/2) x floor(W/2) pixels: the textbook output's first rows and columns
    checks = {"a": (c1, lambda t: co.conv2d_f64(t["img"], w1, b1, 1, 1, "relu")),
              "b": (c1, lambda t: co.conv2d_f64(t["a"], w2, b2, 1, 0, "silu", t["a"])),
              "y": (32, lambda t: co.conv2d_f64(t["b"], w3, b3, 2, 1))}
    order = iter(["a", "b", "y"])
    for i, c in enumerate(plan.cmds):
        plan.execute_range(i, 1)
        if c["type"] != "K44_WAVE":
            continue
        out = next(order)
        C, ref_fn = checks[out]
        h, w = int(c["h_out"]), int(c["w_out"])
        assert (h, w) == ((H, W) if out != "y" else (H // 2, W // 2)), (out, h, w)
        L = lay(h, w)
        buf = plan.read_canvas(int(c["y_off"]), C * L.channel_stride).view(np.float16)
        got = buf[L.offsets(C)]
        dev[out] = got
        err = orc.rel_err(got.astype(np.float64), ref_fn(dev)[:, :, :h, :w])
        _log(f"[single-frame mfma F={frames} {H}x{W}] {out}: rel err {err:.3e}")
        assert err <= TOL, out
        halo = np.ones(C * L.channel_stride, bool)
        halo[L.offsets(C).ravel()] = False
        assert not buf[halo].any(), f"{out}: halo written"

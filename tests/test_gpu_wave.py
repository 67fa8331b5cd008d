"""GPU parity of the wave kernels through the C ABI (libk44wavec.so) against the fp64 oracle.

Tolerance (north_star): max |y - ref| / (|ref| + 1e-2) <= 2e-3, y = fp16 output of the GPU,
ref = fp64 accumulation over the same fp16 operands (oracle/wave_oracle.c:orc_wave_f64).
"""
import numpy as np
import pytest

from snntome_amd import synth

from wave_cases import PATH_IDS, TOL, cluster_rows, random_rows, run_sparse_case, sampled_parity, stride_of

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def test_config1_full_wave(wavec, orc):
    """Config 1 (plumbing) at full size: 4,096 neurons x 8 clusters x S=64, batch 64."""
    wl = synth.config1(seed=1)
    w = wl.waves[0]
    _log(f"[c1] {wl.description}")
    y, ref, plan = run_sparse_case(wavec, orc, C=wl.substrate, tokens=wl.tokens,
                                   rows=cluster_rows(w.starts, w.S), weights=w.weights,
                                   bias=w.bias, act=w.act, seed=wl.seed)
    rep = plan.exec_report()["waves"][0]
    assert rep["path"] == "valu_gather_dot"
    assert (rep["K"], rep["S"]) == (8, 64)  # the upload recovered the dendritic segments
    err = orc.rel_err(y, ref)
    _log(f"[c1] rel err {err:.3e}")
    assert err <= TOL


def test_config2_full_wave_sampled(wavec, orc):
    """Config 2 at full size (40,000,000 x 256 substrate = 20.5 GB generated on the device,
    65,536 neurons x 4 clusters of S=16): the streaming kernel with non-temporal loads; 768
    neurons (first, middle and last workgroups) against the oracle, and a second execution
    bit-identical to the first (the kernel's result does not depend on cache state or timing)."""
    wl = synth.config2()
    _log(f"[c2] {wl.description}")
    plan = synth.build_graph(wl, wavec).compile()
    plan.init_gpu()
    rep = plan.exec_report()["waves"][0]
    _log(f"[c2] path={rep['path']} stream_kernel={rep['stream_kernel']} "
         f"stream_loads={rep['stream_loads']}")
    assert rep["path"] == "valu_gather_dot" and rep["stream_kernel"] and rep["stream_loads"]
    plan.fill_input_uniform(wl.seed)
    plan.execute(1)
    neurons = np.concatenate([np.arange(0, 256), np.arange(30000, 30256),
                              np.arange(65280, 65536)])
    y, ref = sampled_parity(orc, plan, wl, 0, neurons)
    err = orc.rel_err(y, ref)
    _log(f"[c2] rel err over {len(neurons)} neurons x 256 tokens: {err:.3e}")
    assert err <= TOL
    plan.execute(1)
    y2, _ = sampled_parity(orc, plan, wl, 0, neurons[:64])
    assert np.array_equal(y2, y[:64])


@pytest.mark.parametrize("lanes", [4, 8])
@pytest.mark.parametrize("tokens", [64, 128, 256, 320, 512, 100])
@pytest.mark.parametrize("act", ["none", "relu", "sigmoid", "silu", "leaky_relu", "gelu"])
def test_activation_and_slab_shapes(wavec, orc, tuning, tokens, act, lanes):
    """Every activation x every slab width (64/128/256 and ragged token counts) x both lane
    widths of the gather kernel (4 tokens / 8-byte loads, 8 tokens / 16-byte loads)."""
    tuning("lane8", 1 if lanes == 8 else 0)
    acts = ["none", "relu", "sigmoid", "silu", "leaky_relu", "gelu"]
    rng = np.random.default_rng(tokens * 16 + acts.index(act))
    C, cout, K, S = 3000, 48, 3, 24
    starts = rng.integers(0, C - S, size=(cout, K)).astype(np.uint32)
    w = synth.normal_f16(rng, (cout, K * S), 0.1)
    b = synth.normal_f16(rng, (cout,), 0.1)
    y, ref, plan = run_sparse_case(wavec, orc, C=C, tokens=tokens, rows=cluster_rows(starts, S),
                                   weights=w, bias=b, act=act, seed=5)
    rep = plan.exec_report()["waves"][0]
    assert rep["S"] == S and rep["tokens_per_lane"] == lanes
    assert orc.rel_err(y, ref) <= TOL


@pytest.mark.parametrize("fan", [1, 7, 33, 64])
def test_generic_gather_rows(wavec, orc, fan):
    """Arbitrary (non-contiguous) index rows: every synapse its own segment (S = 1)."""
    rng = np.random.default_rng(fan)
    C, cout, tokens = 5000, 40, 128
    rows = random_rows(rng, cout, fan, C)
    w = synth.normal_f16(rng, (cout, fan), 0.2)
    b = synth.normal_f16(rng, (cout,), 0.05)
    y, ref, plan = run_sparse_case(wavec, orc, C=C, tokens=tokens, rows=rows, weights=w, bias=b,
                                   act="relu", seed=9)
    assert orc.rel_err(y, ref) <= TOL


@pytest.mark.parametrize("cluster", [2, 16, 64])
def test_shared_rows_and_residual(wavec, orc, cluster):
    """Neurons sharing index rows (cluster > 1) with a residual add (y = act(v) + r)."""
    rng = np.random.default_rng(cluster)
    C, cout, K, S, tokens = 4096, 128, 4, 32, 256
    starts = rng.integers(0, C - S, size=(cout // cluster, K)).astype(np.uint32)
    w = synth.normal_f16(rng, (cout, K * S), 0.05)
    b = synth.normal_f16(rng, (cout,), 0.05)
    y, ref, plan = run_sparse_case(wavec, orc, C=C, tokens=tokens,
                                   rows=cluster_rows(starts, S), weights=w, bias=b,
                                   cluster=cluster, act="silu", residual=True, seed=3)
    assert orc.rel_err(y, ref) <= TOL


def test_infer_f32_host_roundtrip(wavec, orc):
    """The reference entry point wavec_gpu_infer_f32: host fp32 input -> fp32 output."""
    rng = np.random.default_rng(0)
    C, cout, K, S, tokens = 1024, 64, 2, 16, 96
    starts = rng.integers(0, C - S, size=(cout, K)).astype(np.uint32)
    w = synth.normal_f16(rng, (cout, K * S), 0.1)
    b = synth.normal_f16(rng, (cout,), 0.1)
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", C, 1, tokens, is_1d=True)
    g.add_cluster_wave("w0", "x", "y", starts, S, w, b, act="relu")
    plan = g.compile()
    x = rng.uniform(-1, 1, size=(C, 1, tokens)).astype(np.float32)
    out, ms = plan.infer_f32(x)
    assert out.shape == (cout, 1, tokens)
    st = stride_of(tokens)
    xs = np.zeros((C, st), np.float16)
    xs[:, :tokens] = x[:, 0, :].astype(np.float16)
    seg = (starts.astype(np.uint64) * st).reshape(-1)
    ref = orc.wave_f64(xs.view(np.uint16).ravel(), seg, w, b, None, K, S, 1, st, st, st, "relu")
    assert orc.rel_err(out[:, 0, :], ref[:, :tokens]) <= TOL


def test_tcff_roundtrip_on_gpu(wavec, orc, tmp_path):
    """Save a plan, load its weights into a freshly compiled plan, run both: identical bits."""
    rng = np.random.default_rng(1)
    C, cout, K, S, tokens = 2048, 96, 4, 16, 128
    starts = rng.integers(0, C - S, size=(cout, K)).astype(np.uint32)
    w = synth.normal_f16(rng, (cout, K * S), 0.1)
    b = synth.normal_f16(rng, (cout,), 0.1)

    def make(weights):
        g = wavec.WaveGraph(kv_cache_max_seq=0)
        g.add_input("x", C, 1, tokens, is_1d=True)
        g.add_cluster_wave("w0", "x", "y", starts, S, weights, b, act="gelu")
        return g, g.compile()

    g1, p1 = make(w)
    path = tmp_path / "plan.tcff"
    p1.save_tcff(path)
    g2, p2 = make(np.zeros_like(w))
    p2.load_tcff_weights(path)
    outs = []
    for p in (p1, p2):
        p.init_gpu()
        p.fill_input_uniform(21)
        p.execute(1)
        cmd = p.cmds[0]
        outs.append(p.read_canvas(int(cmd["y_off"]), cout * stride_of(tokens)))
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("lanes", [4, 8])
@pytest.mark.parametrize("tokens,S", [(256, 32), (256, 24), (100, 16), (512, 40)])
def test_streaming_loads_bit_identical(wavec, orc, tuning, lanes, tokens, S):
    """The non-temporal load policy (chosen for substrates far beyond the caches, forced here
    with tuning switch nt=1) changes the cache policy only: outputs equal the default policy's bit
    for bit, over whole and partial 16-row batches, both lane widths, residual and bias."""
    tuning("lane8", 1 if lanes == 8 else 0)
    rng = np.random.default_rng(tokens + S)
    C, cout, K = 4000, 64, 3
    starts = (rng.integers(0, (C - S) // 8, size=(cout, K)) * 8).astype(np.uint32)
    w = synth.normal_f16(rng, (cout, K * S), 0.1)
    b = synth.normal_f16(rng, (cout,), 0.1)
    ys = {}
    for nt in ("0", "1"):
        tuning("nt", int(nt))
        y, ref, plan = run_sparse_case(wavec, orc, C=C, tokens=tokens,
                                       rows=cluster_rows(starts, S), weights=w, bias=b,
                                       act="relu", residual=True, seed=11)
        rep = plan.exec_report()["waves"][0]
        assert rep["path"] == "valu_gather_dot" and rep["stream_loads"] == (nt == "1"), rep
        assert rep["tokens_per_lane"] == lanes
        assert orc.rel_err(y, ref) <= TOL
        ys[nt] = y
    assert np.array_equal(ys["0"], ys["1"])


@pytest.mark.parametrize("cout,K,S,tokens,act,cluster", [
    (300, 3, 24, 256, "gelu", 1),    # two workgroups, the second short; partial 16-row batches
    (512, 4, 16, 512, "relu", 1),    # two 256-token slabs
    (256, 1, 40, 256, "silu", 2),    # one segment per neuron, shared index rows
    (40, 2, 16, 256, "none", 1),     # fewer neurons than waves in the workgroup
])
def test_stream_kernel_bit_identical(wavec, orc, tuning, cout, K, S, tokens, act, cluster):
    """The streaming gather kernel (output rows staged in LDS, written after the last gather;
    forced with tuning switch stream_kernel=1) accumulates each neuron in the order of the one-neuron-per-
    wave kernel (ksplit=1): bit-identical outputs, both within tolerance of the oracle."""
    tuning("nt", 1)
    tuning("lane8", 0)
    rng = np.random.default_rng(cout + K * 10 + S)
    C = 5000
    starts = (rng.integers(0, (C - S) // 8, size=(cout // cluster, K)) * 8).astype(np.uint32)
    w = synth.normal_f16(rng, (cout, K * S), 0.08)
    b = synth.normal_f16(rng, (cout,), 0.1)
    ys = {}
    for mode in ("stream", "plain"):
        tuning("stream_kernel", 1 if mode == "stream" else 0)
        tuning("ksplit", 1)
        y, ref, plan = run_sparse_case(wavec, orc, C=C, tokens=tokens,
                                       rows=cluster_rows(starts, S), weights=w, bias=b,
                                       cluster=cluster, act=act, seed=13)
        rep = plan.exec_report()["waves"][0]
        assert rep["stream_kernel"] == (mode == "stream"), rep
        err = orc.rel_err(y, ref)
        _log(f"[stream-kernel cout={cout} K={K} S={S} tok={tokens} {mode}] rel err {err:.3e}")
        assert err <= TOL
        ys[mode] = y
    assert np.array_equal(ys["stream"], ys["plain"])


def test_stream_kernel_cout_map(wavec, orc, tuning):
    """Streaming kernel on a pruned projection (VALU path): cout_map stores and empty slots of
    the pattern-sorted tiles, against the per-neuron fp64 oracle."""
    tuning("path", 0)
    tuning("nt", 1)
    tuning("lane8", 0)
    tuning("stream_kernel", 1)
    rng = np.random.default_rng(77)
    n_cl, K, S, cout, tokens = 6, 3, 32, 333, 256
    C = n_cl * S
    pick = np.argsort(rng.random((cout, n_cl)), axis=1)[:, :K]
    starts = (pick * S).astype(np.uint32)
    w = synth.normal_f16(rng, (cout, K * S), 0.05)
    b = synth.normal_f16(rng, (cout,), 0.05)
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", C, 1, tokens, is_1d=True)
    g.add_pruned_wave("p", "x", "y", starts, S, w, b, tile=32, act="gelu")
    plan = g.compile()
    plan.init_gpu()
    rep = plan.exec_report()["waves"]
    assert all(r["stream_kernel"] and r["mapped"] for r in rep), rep
    plan.fill_input_uniform(5)
    plan.execute(1)
    st = stride_of(tokens)
    canvas = plan.read_canvas(0, int(plan.summary["canvas_elems"]))
    x0 = int(plan.cmds[0]["src_off"])
    seg = (x0 + starts.astype(np.uint64) * st).ravel()
    ref = orc.wave_f64(canvas, seg, w, b, None, K, S, 1, st, st, st, "gelu")
    y0 = int(plan.cmds[0]["y_off"])
    y = canvas[y0:y0 + cout * st].view(np.float16).reshape(cout, st).astype(np.float64)
    err = orc.rel_err(y, ref)
    _log(f"[stream-kernel cout_map] rel err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("path,cluster", [("valu", 1), ("mfma", 16)])
def test_neuron_65535_without_cout_map(wavec, orc, tuning, path, cluster):
    """Waves of more than 65,536 neurons: channel 65535 equals the 16-bit empty-slot marker of
    cout_map, which must only mean "no output" when the wave has a cout_map (regression: the
    last neuron of config 2 was dropped)."""
    tuning("path", PATH_IDS[path])
    rng = np.random.default_rng(65535)
    C, cout, K, S, tokens = 4096, 65536 + 32, 1, 32, 64
    starts = (rng.integers(0, (C - S) // 16, size=(cout // cluster, K)) * 16).astype(np.uint32)
    w = synth.normal_f16(rng, (cout, K * S), 0.1)
    b = synth.normal_f16(rng, (cout,), 0.1)
    y, ref, plan = run_sparse_case(wavec, orc, C=C, tokens=tokens,
                                   rows=cluster_rows(starts, S), weights=w, bias=b,
                                   cluster=cluster, act="none", seed=21)
    assert plan.exec_report()["waves"][0]["path"].startswith(path)
    tail = slice(65536 - 64, cout)
    err = orc.rel_err(y[tail], ref[tail])
    _log(f"[65535 {path}] rel err over neurons 65472..{cout - 1}: {err:.3e}")
    assert err <= TOL
    assert np.any(y[65535] != 0.0)


@pytest.mark.parametrize("tokens,K,S", [(128, 16, 128), (64, 8, 64), (256, 3, 40), (100, 12, 24)])
def test_weights_staged_in_lds_bit_identical(wavec, orc, tuning, tokens, K, S):
    """The 8-token-per-lane gather kernel stages each neuron's weights in LDS before its gathers
    (tuning switch wlds=0 reads them from memory per batch): same values, same FMA order, so the
    outputs are bit-identical; one neuron per wave (K > 8) and four waves per neuron (K <= 8)."""
    tuning("lane8", 1)
    rng = np.random.default_rng(tokens + K * 3 + S)
    C, cout = 5000, 96
    starts = (rng.integers(0, (C - S) // 8, size=(cout, K)) * 8).astype(np.uint32)
    w = synth.normal_f16(rng, (cout, K * S), 0.05)
    b = synth.normal_f16(rng, (cout,), 0.1)
    ys = {}
    for mode in ("lds", "memory"):
        tuning("wlds", 1 if mode == "lds" else 0)
        y, ref, plan = run_sparse_case(wavec, orc, C=C, tokens=tokens,
                                       rows=cluster_rows(starts, S), weights=w, bias=b,
                                       act="silu", residual=True, seed=23)
        assert plan.exec_report()["waves"][0]["tokens_per_lane"] == 8
        assert orc.rel_err(y, ref) <= TOL
        ys[mode] = y
    assert np.array_equal(ys["lds"], ys["memory"])

"""GPU parity of the MFMA dense-cluster path (k44_mfma_tile_kernel) against the fp64 oracle,
and agreement with the VALU path on the same plans.  Tolerance as in test_gpu_wave.py."""

import numpy as np
import pytest

from snntome_amd import synth

from wave_cases import PATH_IDS, TOL, cluster_rows, run_sparse_case, sampled_parity, stride_of

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def test_config3_full_wave_every_tile(wavec, orc):
    """Config 3 at full size (1,048,576 x 512 substrate, 16,384 neurons, 64-neuron tiles of
    16 x S=512 clusters, GELU) on the MFMA path: every neuron of all 256 tiles x 512 tokens
    against the oracle (32 tiles at a time, each from a compact host copy of the rows it reads)."""
    wl = synth.config3()
    _log(f"[c3] {wl.description}")
    plan = synth.build_graph(wl, wavec).compile()
    plan.init_gpu()
    rep = plan.exec_report()["waves"][0]
    _log(f"[c3] path={rep['path']} K={rep['K']} S={rep['S']} tile={rep['cluster']}")
    assert rep["path"] == "mfma_dma" and (rep["K"], rep["S"]) == (16, 512)
    plan.fill_input_uniform(wl.seed)
    plan.execute(1)
    w = wl.waves[0]
    st = stride_of(wl.tokens)
    y0 = int(plan.cmds[0]["y_off"])
    y_all = plan.read_canvas(y0, w.cout * st).view(np.float16).reshape(w.cout, st)
    worst = 0.0
    for t0 in range(0, w.cout // 64, 32):
        neurons = np.arange(t0 * 64, (t0 + 32) * 64)
        _, ref = sampled_parity(orc, plan, wl, 0, neurons, read_out=False)
        worst = max(worst, orc.rel_err(y_all[neurons].astype(np.float64), ref))
    _log(f"[c3] rel err over all {w.cout} neurons x {wl.tokens} tokens: {worst:.3e}")
    assert worst <= TOL


def test_config3_mfma_matches_valu(wavec, orc, tuning):
    """Same reduced config-3 plan on both paths: each within tolerance of the oracle."""
    wl = synth.config3(neurons=512, substrate=65536, tokens=256)
    outs = {}
    for path in ("mfma", "valu"):
        tuning("path", PATH_IDS[path])
        plan = synth.build_graph(wl, wavec).compile()
        plan.init_gpu()
        tuning("path", -1)
        assert plan.exec_report()["waves"][0]["path"].startswith(path)
        plan.fill_input_uniform(wl.seed)
        plan.execute(1)
        neurons = np.arange(512)
        y, ref = sampled_parity(orc, plan, wl, 0, neurons)
        assert orc.rel_err(y, ref) <= TOL
        outs[path] = y
    # both paths round the same fp32-ish sums to fp16: they agree to a few fp16 ulps
    assert orc.rel_err(outs["mfma"], outs["valu"]) <= TOL


@pytest.mark.parametrize("nt", [16, 32, 64, 128])
@pytest.mark.parametrize("tokens", [64, 128, 256, 512, 192, 640])
def test_mfma_tile_shapes(wavec, orc, nt, tokens):
    """Every tile size x token tiling (incl. ragged 192/640 -> 64/128-token workgroups)."""
    rng = np.random.default_rng(nt * 1000 + tokens)
    C, tiles, K, S = 4096, 3, 2, 64
    cout = tiles * nt
    starts = (rng.integers(0, (C - S) // 8, size=(tiles, K)) * 8).astype(np.uint32)
    w = synth.normal_f16(rng, (cout, K * S), 0.05)
    b = synth.normal_f16(rng, (cout,), 0.05)
    y, ref, plan = run_sparse_case(wavec, orc, C=C, tokens=tokens, rows=cluster_rows(starts, S),
                                   weights=w, bias=b, cluster=nt, act="gelu", seed=13)
    assert orc.rel_err(y, ref) <= TOL
    rep = plan.exec_report()["waves"][0]
    dma = tokens % 512 == 0 and nt in (32, 64, 128)
    assert rep["path"] == ("mfma_dma" if dma else "mfma_tile")


@pytest.mark.parametrize("S", [32, 96, 128, 160])
def test_mfma_segment_lengths_and_residual(wavec, orc, S):
    """Segments of 32..160 positions (32- and 64-row stages) with a residual add."""
    rng = np.random.default_rng(S)
    C, nt, tiles, K, tokens = 8192, 64, 2, 3, 256
    starts = (rng.integers(0, (C - S) // 8, size=(tiles, K)) * 8).astype(np.uint32)
    w = synth.normal_f16(rng, (tiles * nt, K * S), 0.05)
    b = synth.normal_f16(rng, (tiles * nt,), 0.05)
    y, ref, plan = run_sparse_case(wavec, orc, C=C, tokens=tokens, rows=cluster_rows(starts, S),
                                   weights=w, bias=b, cluster=nt, act="relu", residual=True,
                                   seed=17)
    assert plan.exec_report()["waves"][0]["path"] == "mfma_tile"
    assert orc.rel_err(y, ref) <= TOL


def test_dense_linear_layer_takes_mfma(wavec, orc):
    """A reference-style dense 1x1 linear layer (every index row = all input channels, one
    contiguous segment) is tiled onto MFMA and matches the oracle."""
    rng = np.random.default_rng(2)
    din, dout, tokens = 512, 256, 128
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", din, 1, tokens, is_1d=True)
    wt = (rng.standard_normal((dout, din)) * 0.05).astype(np.float32)
    bs = (rng.standard_normal(dout) * 0.05).astype(np.float32)
    g.add_linear("fc", "x", "y", din, dout, wt, bs, act="silu")
    plan = g.compile()
    plan.init_gpu()
    rep = plan.exec_report()["waves"][0]
    assert rep["path"] == "mfma_tile" and rep["K"] == 1 and rep["S"] == din
    plan.fill_input_uniform(5)
    plan.execute(1)
    st = stride_of(tokens)
    canvas = plan.read_canvas(0, int(plan.summary["canvas_elems"]))
    cmd = plan.cmds[0]
    x0 = int(cmd["src_off"])
    rows = (x0 + np.arange(din, dtype=np.uint64) * st)
    seg = np.tile(rows[:1], dout // int(rep["cluster"]))
    w16 = wt.astype(np.float16)
    b16 = bs.astype(np.float16)
    ref = orc.wave_f64(canvas, seg, w16, b16, None, 1, din, int(rep["cluster"]), st, st, st,
                       "silu")
    y0 = int(cmd["y_off"])
    y = canvas[y0:y0 + dout * st].view(np.float16).reshape(dout, st).astype(np.float64)
    assert orc.rel_err(y, ref) <= TOL


@pytest.mark.parametrize("tokens", [1, 5, 16])
@pytest.mark.parametrize("nt", [16, 32, 64, 128])
def test_narrow_mfma_decode_sizes(wavec, orc, tuning, tokens, nt):
    """Waves over at most 16 tokens take the narrow MFMA kernel (16-token tiles, contraction
    chunks in LDS, split-K partials); valid columns match the oracle and the wide kernel."""
    rng = np.random.default_rng(tokens * 1000 + nt)
    S, K, tiles = 512, 4, 3
    C = 16384
    starts = (rng.integers(0, C // S, size=(tiles, K)) * S).astype(np.uint32)
    cout = tiles * nt
    w = synth.normal_f16(rng, (cout, K * S), 0.02)
    b = synth.normal_f16(rng, (cout,), 0.05)
    ys = {}
    for mode in ("narrow", "wide"):
        if mode == "wide":
            tuning("narrow", 0)
        g = wavec.WaveGraph(kv_cache_max_seq=0)
        g.add_input("x", C, 1, tokens, is_1d=True)
        g.add_cluster_wave("w", "x", "y", starts, S, w, b, cluster=nt, act="gelu", res_blob="x")
        plan = g.compile()
        plan.init_gpu()
        rep = plan.exec_report()["waves"][0]
        assert rep["path"] == ("mfma_tile" if mode == "wide" else "mfma_narrow"), rep
        plan.fill_input_uniform(9)
        plan.execute(1)
        st = stride_of(tokens)
        canvas = plan.read_canvas(0, int(plan.summary["canvas_elems"]))
        x0 = int(plan.cmds[0]["src_off"])
        y0 = int(plan.cmds[0]["y_off"])
        y = canvas[y0:y0 + cout * st].view(np.float16).reshape(cout, st)[:, :tokens]
        seg = (x0 + starts.astype(np.uint64) * st).ravel()
        ref = orc.wave_f64(canvas, seg, w, b, None, K, S, nt, st, st, st, "gelu", res_off=x0)
        err = orc.rel_err(y.astype(np.float64), ref[:, :tokens])
        print(f"[narrow {tokens} tok nt={nt} {mode}] ksplit {rep['ksplit']} rel err {err:.3e}",
              flush=True)
        assert err <= TOL
        for _ in range(3):  # repeated launches (split-K scratch reused): identical results
            plan.execute(1)
            again = plan.read_canvas(y0, cout * st).view(np.float16).reshape(cout, st)
            assert np.array_equal(again[:, :tokens].view(np.uint16), y.view(np.uint16))
        ys[mode] = y.astype(np.float64)
    assert orc.rel_err(ys["narrow"], ys["wide"]) <= TOL


@pytest.mark.parametrize("nt,S,K,tiles,tokens,res", [
    (64, 32, 1, 2, 512, False),    # one 32-position stage per tile
    (64, 64, 1, 1, 512, True),     # two stages
    (32, 96, 1, 1, 512, False),    # three stages (drain only)
    (32, 160, 3, 2, 1024, True),   # 15 stages, two token tiles
    (64, 512, 4, 5, 512, False),   # 64 stages
])
@pytest.mark.parametrize("nbuf", ["2", "4", "4p"])
def test_dma_ring_matches_register_staged(wavec, orc, tuning, nt, S, K, tiles, tokens, res,
                                          nbuf):
    """512-token workgroups take the LDS-ring kernel (direct loads, 2- or 4-stage ring, explicit
    waits; "4p": 4 stages with producer waves issuing every load).  Without split-K it
    accumulates in the same k-step order as the register-staged kernel, so the outputs are
    bit-identical; with split-K (partial boundaries differ) both are within tolerance of the
    oracle.  Stage counts 1..3 exercise the drain-only path."""
    prod = nbuf.endswith("p")
    nbuf = nbuf.rstrip("p")
    tuning("dma_stages", int(nbuf))
    tuning("dma_prod", 1 if prod else 0)
    rng = np.random.default_rng(S * 7 + K)
    C = 16384
    starts = (rng.integers(0, (C - S) // 8, size=(tiles, K)) * 8).astype(np.uint32)
    cout = tiles * nt
    w = synth.normal_f16(rng, (cout, K * S), 0.05)
    b = synth.normal_f16(rng, (cout,), 0.05)
    out = {}
    for split in ("1", "0"):
        tuning("splitk", -1 if split == "1" else 0)
        for dma in ("1", "0"):
            tuning("dma", int(dma))
            y, ref, plan = run_sparse_case(wavec, orc, C=C, tokens=tokens,
                                           rows=cluster_rows(starts, S), weights=w, bias=b,
                                           cluster=nt, act="gelu", residual=res, seed=21)
            rep = plan.exec_report()["waves"][0]
            assert rep["path"] == ("mfma_dma" if dma == "1" else "mfma_tile"), rep
            assert rep["ring_stages"] == (int(nbuf) if dma == "1" else 0), rep
            want_prod = (2 if nt == 32 else 4) if (prod and dma == "1") else 0
            assert rep["ring_producers"] == want_prod, rep
            err = orc.rel_err(y, ref)
            _log(f"[dma nt={nt} S={S} K={K} tiles={tiles} tokens={tokens} split={split} "
                 f"dma={dma} ring={nbuf} producers={want_prod}] ksplit {rep['ksplit']} "
                 f"rel err {err:.3e}")
            assert err <= TOL
            out[(split, dma)] = y
    assert np.array_equal(out[("0", "1")], out[("0", "0")])


@pytest.mark.parametrize("K,tokens", [(3, 16), (7, 16), (7, 9), (2, 1)])
def test_narrow_long_chunks_many_tiles(wavec, orc, tuning, K, tokens):
    """Waves of >= 128 64-neuron tiles over <= 16 tokens: contraction chunks of several 16-k-step
    sub-chunks through two LDS buffers, fused epilogue when one chunk covers the contraction
    (K = 2: 32 k-steps), split-K partials reduced by each tile's last workgroup otherwise
    (K = 3, 7: 48 / 112 k-steps in chunks of at most 32); within tolerance of the oracle and of
    the wide kernel."""
    rng = np.random.default_rng(K * 100 + tokens)
    S, nt, tiles, C = 512, 64, 130, 16384  # residual rows: cout <= C
    starts = (rng.integers(0, C // S, size=(tiles, K)) * S).astype(np.uint32)
    cout = tiles * nt
    w = synth.normal_f16(rng, (cout, K * S), 0.02)
    b = synth.normal_f16(rng, (cout,), 0.05)
    ys = {}
    for mode in ("narrow", "wide"):
        if mode == "wide":
            tuning("narrow", 0)
        g = wavec.WaveGraph(kv_cache_max_seq=0)
        g.add_input("x", C, 1, tokens, is_1d=True)
        g.add_cluster_wave("w", "x", "y", starts, S, w, b, cluster=nt, act="silu", res_blob="x")
        plan = g.compile()
        plan.init_gpu()
        rep = plan.exec_report()["waves"][0]
        assert rep["path"] == ("mfma_tile" if mode == "wide" else "mfma_narrow"), rep
        if mode == "narrow":
            assert (rep["ksplit"] > 1) == (K * S // 32 > 32), rep
        plan.fill_input_uniform(4)
        plan.execute(1)
        st = stride_of(tokens)
        canvas = plan.read_canvas(0, int(plan.summary["canvas_elems"]))
        x0 = int(plan.cmds[0]["src_off"])
        y0 = int(plan.cmds[0]["y_off"])
        y = canvas[y0:y0 + cout * st].view(np.float16).reshape(cout, st)[:, :tokens]
        seg = (x0 + starts.astype(np.uint64) * st).ravel()
        ref = orc.wave_f64(canvas, seg, w, b, None, K, S, nt, st, st, st, "silu", res_off=x0)
        err = orc.rel_err(y.astype(np.float64), ref[:, :tokens])
        _log(f"[narrow-long K={K} tok={tokens} {mode}] ksplit {rep['ksplit']} rel err {err:.3e}")
        assert err <= TOL
        ys[mode] = y.astype(np.float64)
    assert orc.rel_err(ys["narrow"], ys["wide"]) <= TOL


@pytest.mark.parametrize("S,K,tiles,tokens,res", [
    (32, 1, 2, 512, False),     # one stage per tile
    (64, 1, 1, 512, True),      # two stages (drain only)
    (160, 3, 2, 1024, True),    # 15 stages, two token tiles
    (512, 4, 3, 512, False),    # 64 stages
])
def test_dma_ring_nt128_matches_register_staged(wavec, orc, tuning, S, K, tiles, tokens, res):
    """128-neuron tiles over 512-token workgroups take the LDS-ring kernel with a 3-stage ring
    (one workgroup per CU); without split-K bit-identical to the register-staged 128-neuron
    kernel (same k-step order), both within tolerance of the oracle."""
    rng = np.random.default_rng(S * 11 + K)
    C = 16384
    starts = (rng.integers(0, (C - S) // 8, size=(tiles, K)) * 8).astype(np.uint32)
    cout = tiles * 128
    w = synth.normal_f16(rng, (cout, K * S), 0.05)
    b = synth.normal_f16(rng, (cout,), 0.05)
    out = {}
    tuning("splitk", 0)
    for dma in (1, 0):
        tuning("dma", dma)
        y, ref, plan = run_sparse_case(wavec, orc, C=C, tokens=tokens, rows=cluster_rows(starts, S),
                                       weights=w, bias=b, cluster=128, act="silu", residual=res,
                                       seed=23)
        rep = plan.exec_report()["waves"][0]
        assert rep["path"] == ("mfma_dma" if dma else "mfma_tile"), rep
        assert rep["ring_stages"] == (3 if dma else 0), rep
        err = orc.rel_err(y, ref)
        _log(f"[dma nt=128 S={S} K={K} tiles={tiles} tokens={tokens} dma={dma}] rel err {err:.3e}")
        assert err <= TOL
        out[dma] = y
    assert np.array_equal(out[1], out[0])


@pytest.mark.parametrize("nt,tokens,tiles", [(64, 512, 13), (32, 1024, 7), (64, 192, 5),
                                             (128, 512, 3), (16, 256, 9)])
def test_xcd_item_order_bit_identical(wavec, orc, tuning, nt, tokens, tiles):
    """Work items taken as per-wave shares of the XCDs (xcd_order 2, the default), contiguous
    ranges per XCD (1) or in plain workgroup order (0) are the same items: bit-identical outputs,
    within tolerance of the oracle; item counts that are not multiples of 8 included (LDS-ring
    and register-staged kernels)."""
    rng = np.random.default_rng(nt * 31 + tiles)
    C, K, S = 8192, 2, 64
    starts = (rng.integers(0, (C - S) // 8, size=(tiles, K)) * 8).astype(np.uint32)
    w = synth.normal_f16(rng, (tiles * nt, K * S), 0.05)
    b = synth.normal_f16(rng, (tiles * nt,), 0.05)
    out = {}
    for order in (2, 1, 0):
        tuning("xcd_order", order)
        y, ref, plan = run_sparse_case(wavec, orc, C=C, tokens=tokens,
                                       rows=cluster_rows(starts, S), weights=w, bias=b,
                                       cluster=nt, act="silu", seed=29)
        assert plan.exec_report()["waves"][0]["path"] in ("mfma_dma", "mfma_tile")
        assert orc.rel_err(y, ref) <= TOL
        out[order] = y
    assert np.array_equal(out[0], out[1])
    assert np.array_equal(out[0], out[2])


@pytest.mark.parametrize("n_cl,K,cout,tokens", [(4, 2, 1000, 1024), (7, 3, 700, 512),
                                                (5, 2, 333, 1536)])
def test_group_item_orders_pruned_bit_identical(wavec, orc, tuning, n_cl, K, cout, tokens):
    """A pruned projection compiles to sub-waves of different stage counts (full-pattern tiles,
    union tiles) launched as one group; per-wave XCD shares with the longest waves first
    (xcd_order 2), contiguous ranges (1) and plain order (0) run the same items: bit-identical,
    and the per-neuron fp64 oracle agrees."""
    rng = np.random.default_rng(n_cl * 13 + cout)
    S = 256
    C = n_cl * S
    pick = np.argsort(rng.random((cout, n_cl)), axis=1)[:, :K]
    starts = (pick * S).astype(np.uint32)
    w = synth.normal_f16(rng, (cout, K * S), 0.05)
    b = synth.normal_f16(rng, (cout,), 0.05)
    out = {}
    for order in (2, 1, 0):
        tuning("xcd_order", order)
        g = wavec.WaveGraph(kv_cache_max_seq=0)
        g.add_input("x", C, 1, tokens, is_1d=True)
        g.add_pruned_wave("p", "x", "y", starts, S, w, b, tile=64, act="silu")
        plan = g.compile()
        plan.init_gpu()
        rep = plan.exec_report()
        parts = rep["waves"]
        assert {r["path"] for r in parts} <= {"mfma_dma", "mfma_tile"}
        assert len({r["K"] for r in parts}) >= 2, "expected sub-waves of several lengths"
        assert len(rep["groups"]) == 1 and len(rep["groups"][0]) == len(parts)
        plan.fill_input_uniform(11)
        plan.execute(1)
        st = stride_of(tokens)
        canvas = plan.read_canvas(0, int(plan.summary["canvas_elems"]))
        y0 = int(plan.cmds[0]["y_off"])
        y = canvas[y0:y0 + cout * st].view(np.float16).reshape(cout, st)
        if order == 2:
            x0 = int(plan.cmds[0]["src_off"])
            seg = (x0 + starts.astype(np.uint64) * st).ravel()
            ref = orc.wave_f64(canvas, seg, w, b, None, K, S, 1, st, st, st, "silu")
            err = orc.rel_err(y.astype(np.float64), ref)
            _log(f"[pruned orders {n_cl}/{K} cout={cout} tokens={tokens}] parts "
                 f"{[(r['path'], r['cout'], r['K']) for r in parts]} rel err {err:.3e}")
            assert err <= TOL
        out[order] = y.copy()
        plan.release_gpu()
    assert np.array_equal(out[2], out[1])
    assert np.array_equal(out[2], out[0])

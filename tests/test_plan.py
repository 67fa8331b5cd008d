"""Plan compilation and the .tcff format, checked bit-exactly against an independent Python
restatement of the reference's compiler and writer (oracle/plan_oracle.py), plus format
invariants, tamper rejection and the 64-bit extension tag.  Host only (no GPU)."""
import json
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import plan_oracle as po
from snntome_amd import synth

GOLDEN = Path(__file__).resolve().parent / "golden"


def _f16(a):
    return np.asarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)


def _pair(wavec, build):
    """Build the same graph with the library and with the Python restatement."""
    g = wavec.WaveGraph(kv_cache_max_seq=0, fold_rmsnorm_gamma=False)
    pg = po.Graph()
    build(g, pg)
    return g, g.compile(), po.compile_plan(pg)


def _linear(g, pg, name, i, o, din, dout, rng, act=None, res=None):
    w = (rng.standard_normal((dout, din)) * 0.1).astype(np.float32)
    b = (rng.standard_normal(dout) * 0.1).astype(np.float32)
    g.add_linear(name, i, o, din, dout, w, b, act=act, res_blob=res)
    pg.linear(name, i, o, din, dout, _f16(w).reshape(dout, din), _f16(b),
              act=po.ACT_NAMES.index((act or "none").upper()) if act else 0,
              residual=res or "")


def _sparse(g, pg, name, i, o, rows, cout, cluster, rng, act="relu", res=None, seg_len=0):
    fan = rows.shape[1]
    w = synth.normal_f16(rng, (cout, fan), 0.05)
    b = synth.normal_f16(rng, (cout,), 0.05)
    if seg_len:
        K = fan // seg_len
        g.add_cluster_wave(name, i, o, rows[:, ::seg_len], seg_len, w, b, cluster=cluster,
                           act=act, res_blob=res)
    else:
        g.add_sparse_wave(name, i, o, rows, w, b, cluster=cluster, act=act, res_blob=res)
    pg.sparse(name, i, o, rows, w.view(np.uint16), b.view(np.uint16), cluster=cluster,
              act=po.ACT_NAMES.index(act.upper()), residual=res or "", seg_len=seg_len)


def _assert_same_tcff(plan, pplan, tmp_path, prefix="K44Model"):
    path = tmp_path / "p.tcff"
    plan.save_tcff(path, prefix)
    got = path.read_bytes()
    want = po.tcff_bytes(pplan, prefix)
    if got != want:
        n = min(len(got), len(want))
        first = next((i for i in range(n) if got[i] != want[i]), n)
        pytest.fail(f".tcff differs: sizes {len(got)} vs {len(want)}, first diff at {first}")
    return got


def _assert_same_plan(plan, pplan):
    s = plan.summary
    assert s["canvas_elems"] == pplan["canvas_elems"]
    waves = [c for c in s["cmds"] if c["type"] == "K44_WAVE"]
    pw = [c for c in pplan["cmds"] if c["type"] == 0]
    assert len(waves) == len(pw)
    for c, p in zip(waves, pw):
        for k_lib, k_or in (("Cout", "Cout"), ("logical_Cout", "logical_Cout"), ("B", "B"),
                            ("B_raw", "B_raw"), ("S", "cluster"), ("src_off", "src_off"),
                            ("y_off", "y_off"), ("Cin", "Cin")):
            assert c[k_lib] == p[k_or], (c["name"], k_lib, c[k_lib], p[k_or])
    assert list(s["output_shape"]) == list(pplan["output"])


def test_linear_chain_with_views(wavec, tmp_path):
    rng = np.random.default_rng(0)

    def build(g, pg):
        for G in (g, pg):
            (G.add_input if G is g else G.input)("x", 96, 1, 100, True)
        _linear(g, pg, "fc1", "x", "h1", 96, 200, rng, act="relu")
        g.add_split("sp", "h1", ["a", "b"])
        pg.split("sp", "h1", ["a", "b"])
        g.add_slice("sl", "a", ["a0", "a1"], [72, 128])
        pg.slice("sl", "a", ["a0", "a1"], [72, 128])
        _linear(g, pg, "fc2", "a1", "h2", 128, 48, rng, act="silu")
        g.add_concat("cat", ["a0", "h2"], "h3")
        pg.concat("cat", ["a0", "h2"], "h3")
        _linear(g, pg, "fc3", "h3", "h4", 120, 72, rng, act="sigmoid", res="a0")
        _linear(g, pg, "fc4", "h4", "out", 72, 33, rng)
        g.set_output("out")
        pg.output = "out"

    g, plan, pplan = _pair(wavec, build)
    _assert_same_plan(plan, pplan)
    _assert_same_tcff(plan, pplan, tmp_path)


def test_sparse_waves_over_concat(wavec, tmp_path):
    """A small config-4-style plan: sparse waves over concatenations of earlier outputs."""
    wl = synth.config4(waves=3, width=2048, neurons=128, K=4, S=32, tokens=64)

    def build(g, pg):
        g.add_input("x", wl.substrate, 1, wl.tokens, is_1d=True)
        pg.input("x", wl.substrate, 1, wl.tokens, True)
        for i, w in enumerate(wl.waves):
            src = w.sources[0] if len(w.sources) == 1 else f"cat{i}"
            if len(w.sources) > 1:
                g.add_concat(f"cat{i}", w.sources, src)
                pg.concat(f"cat{i}", w.sources, src)
            rows = (w.starts[:, :, None].astype(np.int64) + np.arange(w.S)).reshape(
                w.cout, -1).astype(np.uint32)
            g.add_cluster_wave(w.name, src, f"y{i}", w.starts, w.S, w.weights, w.bias,
                               act=w.act)
            pg.sparse(w.name, src, f"y{i}", rows, w.weights.view(np.uint16),
                      w.bias.view(np.uint16), act=1, seg_len=w.S)
        g.set_output("y2")
        pg.output = "y2"

    g, plan, pplan = _pair(wavec, build)
    _assert_same_plan(plan, pplan)
    _assert_same_tcff(plan, pplan, tmp_path)


@pytest.mark.parametrize("cluster", [1, 16, 64])
def test_sparse_wave_clusters_and_residual(wavec, tmp_path, cluster):
    rng = np.random.default_rng(cluster)
    C, cout, fan = 1500, 128, 48
    rows = rng.integers(0, C, size=(cout // cluster, fan)).astype(np.uint32)

    def build(g, pg):
        g.add_input("x", C, 1, 192, is_1d=True)
        pg.input("x", C, 1, 192, True)
        _sparse(g, pg, "s", "x", "y", rows, cout, cluster, rng, act="gelu", res="x")

    g, plan, pplan = _pair(wavec, build)
    _assert_same_plan(plan, pplan)
    _assert_same_tcff(plan, pplan, tmp_path)


def test_summary_json_keys(wavec):
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", 64, 1, 64, is_1d=True)
    g.add_linear("fc", "x", "y", 64, 32, np.ones((32, 64), np.float32))
    plan = g.compile()
    for key in ("batch_size", "num_waves", "num_cmds", "canvas_elems", "canvas_bytes",
                "kv_cache_elems", "total_w_bytes", "total_idx_bytes", "single_frame_gflops",
                "total_gflops", "single_frame_gsyn", "total_gsyn", "input_shape",
                "output_shape", "max_B_per_wave", "target_profile", "target_num_cus",
                "persistent_neurons", "reuse_canvas", "cmds"):
        assert key in plan.summary
    assert plan.canvas_bytes == 2 * plan.summary["canvas_elems"]
    assert plan.num_wave_dispatches == 1
    assert plan.total_gflops == pytest.approx(2 * 64 * 32 * 64 / 1e9, rel=1e-5)


def _tcff_ifds(data: bytes):
    """Minimal TIFF walk: list of {tag: (type, count, value)} per IFD."""
    out = []
    off = struct.unpack_from("<I", data, 4)[0]
    while off:
        n = struct.unpack_from("<H", data, off)[0]
        tags = {}
        for i in range(n):
            t, ty, cnt, val = struct.unpack_from("<HHII", data, off + 2 + 12 * i)
            tags[t] = (ty, cnt, val)
        out.append(tags)
        off = struct.unpack_from("<I", data, off + 2 + 12 * n)[0]
    return out


def test_tcff_header_layout_by_hand(wavec, tmp_path):
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", 64, 1, 64, is_1d=True)
    g.add_linear("fc", "x", "y", 64, 32, np.ones((32, 64), np.float32))
    plan = g.compile()
    p = tmp_path / "h.tcff"
    plan.save_tcff(p, "Hand")
    d = p.read_bytes()
    assert d[:4] == b"II*\x00"
    assert d[8:16] == b"TCFFv1.0"
    align, waves, canvas_bytes, flags = struct.unpack_from("<IIII", d, 16)
    assert (align, waves, flags) == (256, 1, 1)
    assert canvas_bytes == plan.canvas_bytes
    assert struct.unpack_from("<Q", d, 32)[0] == po.fnv1a64(d[8:32])
    assert struct.unpack_from("<I", d, 4)[0] % 256 == 0 and len(d) % 256 == 0
    (ifd,) = _tcff_ifds(d)
    assert ifd[0x8440] == (4, 1, 0x45564157)
    assert ifd[256][2] == 64 and ifd[257][2] == 32  # B, Cout
    aux = struct.unpack_from("<11I", d, ifd[0x8442][2])
    w_off, w_bytes, i_off, i_bytes, b_off, b_bytes = aux[:6]
    assert w_bytes == 32 * 64 * 2 and i_bytes == (32 // 32) * 64 * 4 and b_bytes == 64
    h = struct.unpack_from("<II", d, ifd[0x8443][2])
    assert (h[1] << 32 | h[0]) == po.fnv1a64(d[aux[8]:aux[9]])
    assert 0x8445 not in ifd  # no extension tag for a plain 32-bit plan


def test_tcff_roundtrip_and_tamper_rejection(wavec, tmp_path):
    rng = np.random.default_rng(4)
    starts = rng.integers(0, 900, size=(64, 2)).astype(np.uint32)
    w = synth.normal_f16(rng, (64, 32), 0.1)
    b = synth.normal_f16(rng, (64,), 0.1)

    def make(weights):
        g = wavec.WaveGraph(kv_cache_max_seq=0)
        g.add_input("x", 1000, 1, 64, is_1d=True)
        g.add_cluster_wave("w", "x", "y", starts, 16, weights, b, act="relu")
        return g, g.compile()

    g1, p1 = make(w)
    path = tmp_path / "a.tcff"
    p1.save_tcff(path)
    good = path.read_bytes()
    g2, p2 = make(np.zeros_like(w))
    p2.load_tcff_weights(path)
    # loaded plan re-saves to the identical file
    path2 = tmp_path / "b.tcff"
    p2.save_tcff(path2)
    assert path2.read_bytes() == good
    ifd = _tcff_ifds(good)[0]
    aux = struct.unpack_from("<11I", good, ifd[0x8442][2])
    for where in (9, 20, 33, aux[0] + 5, aux[2] + 1, aux[4]):  # header, hash, payloads
        bad = bytearray(good)
        bad[where] ^= 0x40
        p = tmp_path / f"bad{where}.tcff"
        p.write_bytes(bytes(bad))
        with pytest.raises(RuntimeError):
            p2.load_tcff_weights(p)
    trunc = tmp_path / "trunc.tcff"
    trunc.write_bytes(good[: len(good) // 2])
    with pytest.raises(RuntimeError):
        p2.load_tcff_weights(trunc)


def test_index_rebase_above_0x70000000(wavec, tmp_path):
    """Indices >= 0x70000000 fp16 elements are re-based on min & ~63 (x_base_off) and the
    padded synapses zeroed (reference pack_wave_buffers).  30M channels x 64 tokens."""
    C = 30_000_000
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", C, 1, 64, is_1d=True)
    rows = np.full((16, 3), 29_500_000, np.uint32)  # 16 neurons: no padded (all-zero) rows
    rows[0] = [29_999_000, 29_999_001, 5]
    rows[1] = [29_000_000, 29_000_007, 29_999_999]
    g.add_sparse_wave("s", "x", "y", rows, np.ones((16, 3), np.float16))
    plan = g.compile()
    p = tmp_path / "r.tcff"
    plan.save_tcff(p)
    d = p.read_bytes()
    ifd = _tcff_ifds(d)[0]
    aux = struct.unpack_from("<11I", d, ifd[0x8442][2])
    idx = np.frombuffer(d, dtype="<u4", count=aux[3] // 4, offset=aux[2]).reshape(-1, 64)
    base = (5 * 64) & ~63
    assert idx[0, 0] == 29_999_000 * 64 - base and idx[0, 2] == 5 * 64 - base
    assert idx[1, 2] == 29_999_999 * 64 - base
    assert idx[2, 0] == 29_500_000 * 64 - base
    assert not idx[:, 3:].any()


def test_row_index_mode_beyond_4g_elements(wavec, tmp_path):
    """A 70M-position x 64-token input is 4.48 G fp16 elements: the sparse wave is emitted in
    row-index mode and the 0x8445 tag records the 64-bit offsets."""
    C = 70_000_000
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", C, 1, 64, is_1d=True)
    rows = np.array([[69_999_990 + i for i in range(8)]] * 16, np.uint32)
    g.add_sparse_wave("s", "x", "y", rows, np.ones((16, 8), np.float16))
    plan = g.compile()
    cmd = plan.cmds[0]
    assert cmd["idx_mode"] == 1 and cmd["y_off"] == C * 64
    p = tmp_path / "big.tcff"
    plan.save_tcff(p)
    d = p.read_bytes()
    ifd = _tcff_ifds(d)[0]
    ext = struct.unpack_from("<12I", d, ifd[0x8445][2])
    assert ext[0] == 1 and ext[1] == 64 and ext[2] == 0  # mode, idx_stride
    assert (ext[8] << 32 | ext[7]) == C * 64  # y_off (64-bit)
    aux = struct.unpack_from("<11I", d, ifd[0x8442][2])
    idx = np.frombuffer(d, dtype="<u4", count=aux[3] // 4, offset=aux[2]).reshape(-1, 64)
    assert idx[0, 0] == 69_999_990 and idx[0, 7] == 69_999_997


def test_golden_fixture(wavec, tmp_path):
    """Regression pin: the committed golden plan file (tests/golden/make_golden.py) is
    reproduced byte for byte, and equals the Python restatement's bytes."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    data = mg.build_tcff(wavec, tmp_path / "g.tcff")
    assert data == (GOLDEN / "small_plan.tcff").read_bytes()
    assert po.tcff_bytes(po.compile_plan(mg.oracle_graph(po)), "Golden") == data
    meta = json.loads((GOLDEN / "small_plan.json").read_text())
    assert mg.summary_fields(wavec) == meta


def _pruned_case(rng, n_cl, K, S, cout):
    pick = np.argsort(rng.random((cout, n_cl)), axis=1)[:, :K]
    starts = (pick * S).astype(np.uint32)
    w = synth.normal_f16(rng, (cout, K * S), 0.05)
    b = synth.normal_f16(rng, (cout,), 0.05)
    return starts, w, b


@pytest.mark.parametrize("n_cl,K,tile,cout", [(4, 2, 64, 448), (11, 6, 16, 200), (6, 3, 32, 97)])
def test_pruned_wave_plan_bit_exact(wavec, tmp_path, n_cl, K, tile, cout):
    """Pattern-sorted tile schedule, index rows, zero-filled weights and biases of pruned waves
    are identical to the Python restatement, byte for byte in the .tcff."""
    rng = np.random.default_rng(n_cl * 100 + K)
    S = 32
    starts, w, b = _pruned_case(rng, n_cl, K, S, cout)

    def build(g, pg):
        g.add_input("x", n_cl * S, 1, 80, is_1d=True)
        pg.input("x", n_cl * S, 1, 80, True)
        g.add_pruned_wave("p", "x", "y", starts, S, w, b, tile=tile, act="silu", res_blob=None)
        pg.pruned("p", "x", "y", starts, S, w.view(np.uint16), b.view(np.uint16), tile=tile,
                  act=po.ACT_NAMES.index("SILU"))
        g.add_pruned_wave("q", "y", "z", starts[:, :1] % (cout // S * S or S), S,
                          w[:, :S], b, tile=tile, res_blob="y")
        pg.pruned("q", "y", "z", starts[:, :1] % (cout // S * S or S), S,
                  w[:, :S].view(np.uint16), b.view(np.uint16), tile=tile, residual="y")
        g.set_output("z")
        pg.output = "z"

    g, plan, pplan = _pair(wavec, build)
    _assert_same_plan(plan, pplan)
    _assert_same_tcff(plan, pplan, tmp_path)
    s = plan.summary
    assert s["total_idx_bytes"] == sum(c["idx"].size * 4 + c["Cout"] * 4
                                       for c in pplan["cmds"] if c["type"] == 0)
    # effective FLOPs count real synapses only (2 nnz tokens), not the zero-filled unions
    eff = sum(c["gflops"] for c in s["cmds"] if c["name"].split("/")[0] == "p")
    assert eff == pytest.approx(2 * cout * K * S * 80 / 1e9, rel=1e-6)


def test_pruned_tiles_bound_unions(wavec):
    """Config 5's pruned projections compile to the fewest tiles with bounded unions: the down
    projection (2,048 neurons, 6 of 11 clusters each, all patterns distinct) to 32 tiles of at
    most 9 clusters (pattern-sorted cutting gave up to 11), the d-input projections (2 of 4) to
    tiles of at most 3 (it gave 4)."""
    spec = synth.LLMSpec(layers=1)
    wts = synth.llm_weights(spec)
    for name, fan, bound in (("dn", spec.ffn, 9), ("o", spec.d, 3), ("g", spec.d, 3)):
        p = wts.proj[0][name]
        g = wavec.WaveGraph(kv_cache_max_seq=0)
        g.add_input("x", fan, 1, 64, is_1d=True)
        g.add_pruned_wave(name, "x", "y", p.starts, spec.S, p.weights, p.bias, tile=64)
        g.set_output("y")
        plan = g.compile()
        subs = [(c["Cout"], c["B"] // c["seg_len"]) for c in plan.cmds]
        tiles = sum(n // 64 for n, _ in subs)
        assert tiles == -(-p.weights.shape[0] // 64), subs
        assert max(u for _, u in subs) <= bound, subs


def test_pack_union_tiles_against_exhaustive_optimum():
    """On 200 small random cases (8 or 9 neurons of 2 or 3 clusters out of 4 or 5, tiles of 3
    or 4) the tiles a pruned wave compiles to never have a larger largest union than
    pattern-sorted cutting, and reach the exhaustive optimum over every partition into equal
    tiles in at least 190 cases (the packer is a heuristic; cutting alone reaches it in about
    60 %)."""
    import itertools
    rng = np.random.default_rng(3)
    hits = cut_hits = 0
    for trial in range(200):
        nu, k = (4, 2) if trial % 2 == 0 else (5, 3)
        n, T = (8, 4) if trial % 3 else (9, 3)
        starts = np.stack([np.sort(rng.choice(nu, k, replace=False)) for _ in range(n)])
        pm = [int(sum(1 << int(c) for c in row)) for row in starts]
        w = np.zeros((n, k), np.uint16)
        parts = po.pruned_parts(starts.astype(np.uint32), 1, w, np.zeros(n, np.uint16), T)
        got = max(r.shape[1] for r, _, _, _ in parts)

        def best(rest):  # smallest achievable largest union over partitions of `rest`
            if not rest:
                return 0
            first, others = rest[0], rest[1:]
            out = nu
            for comb in itertools.combinations(others, T - 1):
                u = bin(int(np.bitwise_or.reduce([pm[j] for j in (first,) + comb]))).count("1")
                if u < out:
                    out = min(out, max(u, best([j for j in others if j not in comb])))
            return out

        def cut():  # largest union of pattern-sorted cutting
            groups = {}
            for j in range(n):
                groups.setdefault(tuple(starts[j]), []).append(j)
            ts, rest = [], []
            for key in sorted(groups):
                g = groups[key]
                f = len(g) // T
                ts += [g[i * T:(i + 1) * T] for i in range(f)]
                rest += g[f * T:]
            ts += [rest[b:b + T] for b in range(0, len(rest), T)]
            return max(bin(int(np.bitwise_or.reduce([pm[j] for j in t]))).count("1") for t in ts)

        opt, c = best(list(range(n))), cut()
        assert opt <= got <= c
        hits += got == opt
        cut_hits += c == opt
    assert hits >= 190 and cut_hits < hits, (hits, cut_hits)


def test_pruned_parts_semantics():
    """The decomposition reproduces every neuron's dot product (float64, any input) and places
    each neuron in exactly one slot; full tiles of a single pattern keep the minimal union."""
    rng = np.random.default_rng(7)
    n_cl, K, S, cout, tile = 11, 6, 8, 300, 16
    starts, w, b = _pruned_case(rng, n_cl, K, S, cout)
    parts = po.pruned_parts(starts, S, w.view(np.uint16), b.view(np.uint16), tile)
    x = rng.standard_normal((n_cl * S, 5))
    want = np.stack([sum(w[j, k * S:(k + 1) * S].astype(np.float64) @ x[starts[j, k]:starts[j, k] + S]
                         for k in range(K)) for j in range(cout)])
    got = np.full((cout, 5), np.nan)
    seen = []
    prev_u = 0
    for rows, wp, bp, cm in parts:
        U = rows.shape[1]
        assert U > prev_u and U >= K  # one part per union size, ascending
        prev_u = U
        assert np.all(np.diff(rows.astype(np.int64), axis=1) > 0)
        wf = wp.view(np.float16).astype(np.float64)
        for r in range(wp.shape[0]):
            if cm[r] == 0xFFFF:
                assert not wp[r].any() and bp[r] == 0
                continue
            j = int(cm[r])
            seen.append(j)
            assert set(starts[j].tolist()) <= set(rows[r // tile].tolist())
            assert bp[r] == b.view(np.uint16)[j]
            xs = np.concatenate([x[u:u + S] for u in rows[r // tile]])
            got[j] = wf[r] @ xs
    assert sorted(seen) == list(range(cout))
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
    # a projection whose neurons all share one pattern compiles to full tiles of width K
    same = np.tile(np.array([[0, 2 * S]], np.uint32), (64, 1))
    (rows, wp, _, cm), = po.pruned_parts(same, S, np.zeros((64, 2 * S), np.uint16),
                                          np.zeros(64, np.uint16), 32)
    assert rows.shape == (2, 2) and (cm != 0xFFFF).all()


def test_pruned_wave_rejects_overlap(wavec):
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", 256, 1, 64, is_1d=True)
    st = np.array([[0, 16]] * 16, np.uint32)  # clusters of 32 channels overlap
    with pytest.raises(RuntimeError, match="overlap"):
        g.add_pruned_wave("p", "x", "y", st, 32, np.zeros((16, 64), np.float16), tile=16)


@pytest.mark.parametrize("H,W,batch", [(8, 64, 1), (5, 30, 1), (7, 20, 2), (4, 128, 3)])
def test_2d_layout_matches_restatement(wavec, tmp_path, H, W, batch):
    """The padded-plane layout the compiler writes into each 2-D wave's .tcff geometry tag
    (W_pad, channel stride) equals the independent restatement oracle.cnn_oracle.Layout2D."""
    from oracle import cnn_oracle as co

    rng = np.random.default_rng(H * W)
    g = wavec.WaveGraph(kv_cache_max_seq=0, batch_size=batch)
    g.add_input("img", 3, H, W)
    w = (rng.standard_normal((8, 3, 3, 3)) * 0.1).astype(np.float32)
    g.add_conv2d("c", "img", "y", 3, 8, 3, 3, w, None, stride=1, pad=1, act="relu")
    plan = g.compile()
    p = tmp_path / "c.tcff"
    plan.save_tcff(p, "L")
    d = p.read_bytes()
    (ifd,) = _tcff_ifds(d)
    geo = struct.unpack_from("<10I", d, ifd[0x8444][2])
    lay = co.Layout2D(H, W, min(batch, 8))
    assert geo[:5] == (3, 1, 8, H, W)
    assert geo[6] == lay.channel_stride and geo[7] == lay.W_pad and geo[9] == lay.W_pad + 4
    assert geo[5] == plan.cmds[0]["Cout"] * lay.channel_stride


# ---- 2-D image plans: the padded-plane layouts, tap offsets, stride-2 polyphase (S2D) waves,
# ---- pooling / upsampling / transposed-convolution scratch, checked the same way.

def _conv(g, pg, name, i, o, cin, cout, k, rng, stride=1, act="silu", res=None):
    w = (rng.standard_normal((cout, cin, k, k)) * 0.1).astype(np.float32)
    b = (rng.standard_normal(cout) * 0.1).astype(np.float32)
    g.add_conv2d(name, i, o, cin, cout, k, k, w, b, stride=stride, pad=k // 2, act=act,
                 res_blob=res)
    pg.conv2d(name, i, o, cin, cout, k, k, stride, _f16(w).reshape(cout, cin * k * k), _f16(b),
              act=po.ACT_NAMES.index(act.upper()) if act else 0, residual=res or "")


def _upconv(g, pg, name, i, o, cin, cout, rng):
    w = (rng.standard_normal((cout, cin, 2, 2)) * 0.1).astype(np.float32)
    b = (rng.standard_normal(cout) * 0.1).astype(np.float32)
    g.add_upconv2x2(name, i, o, cin, cout, w, b)
    pg.upconv2x2(name, i, o, cin, cout, _f16(w).reshape(cout, cin, 4), _f16(b))


def _pair2d(wavec, build, batch):
    g = wavec.WaveGraph(kv_cache_max_seq=0, batch_size=batch)
    pg = po.Graph(batch_size=batch)
    build(g, pg)
    return g, g.compile(), po.compile_plan(pg)


@pytest.mark.parametrize("batch", [1, 3])
def test_2d_yolo_like_plan(wavec, tmp_path, batch):
    """Aligned width (W % 64 == 0): 3x3 stride 1 and 2 (S2D scratch), 5x5 max-pool, 1x1 with a
    residual, upsample, concat, 2x2 max-pool; 1 and 3 frames per wave."""
    rng = np.random.default_rng(batch)

    def build(g, pg):
        g.add_input("img", 3, 64, 64)
        pg.input("img", 3, 64, 64, False)
        _conv(g, pg, "c1", "img", "a", 3, 16, 3, rng)
        _conv(g, pg, "c2", "a", "b", 16, 32, 3, rng, stride=2)
        for G in (g, pg):
            (G.add_maxpool if G is g else G.maxpool)("sppf", "b", "p", 5, 1, *([2] if G is g else []))
        _conv(g, pg, "c3", "p", "r", 32, 32, 1, rng, act="relu", res="b")
        g.add_upsample2x("up", "r", "u")
        pg.upsample2x("up", "r", "u")
        g.add_concat("cat", ["u", "a"], "m")
        pg.concat("cat", ["u", "a"], "m")
        _conv(g, pg, "c4", "m", "q", 48, 24, 3, rng, act="gelu")
        g.add_maxpool("mp", "q", "out", 2, 2, 0)
        pg.maxpool("mp", "q", "out", 2, 2)
        g.set_output("out")
        pg.output = "out"

    g, plan, pplan = _pair2d(wavec, build, batch)
    _assert_same_plan(plan, pplan)
    _assert_same_tcff(plan, pplan, tmp_path)


def test_2d_unet_like_masked_plan(wavec, tmp_path):
    """Masked width (W % 64 != 0): pooling down, 2x2 transposed convolution up (quadrant wave
    into its scratch), skip concatenation, split / slice views of a 2-D tensor."""
    rng = np.random.default_rng(7)

    def build(g, pg):
        g.add_input("img", 4, 20, 20)
        pg.input("img", 4, 20, 20, False)
        _conv(g, pg, "e1", "img", "s", 4, 16, 3, rng, act="relu")
        g.add_maxpool("down", "s", "d", 2, 2, 0)
        pg.maxpool("down", "s", "d", 2, 2)
        _conv(g, pg, "e2", "d", "e", 16, 32, 3, rng, act="relu")
        _upconv(g, pg, "up", "e", "u", 32, 16, rng)
        g.add_concat("cat", ["u", "s"], "m")
        pg.concat("cat", ["u", "s"], "m")
        g.add_slice("sl", "m", ["m0", "m1"], [8, 24])
        pg.slice("sl", "m", ["m0", "m1"], [8, 24])
        _conv(g, pg, "d1", "m1", "h", 24, 12, 3, rng, act="silu")
        _conv(g, pg, "head", "h", "out", 12, 5, 1, rng, act=None)
        g.set_output("out")
        pg.output = "out"

    g, plan, pplan = _pair2d(wavec, build, 2)
    _assert_same_plan(plan, pplan)
    _assert_same_tcff(plan, pplan, tmp_path)


def test_2d_rectangular_and_stride2_masked(wavec, tmp_path):
    """H != W layout keys ((h << 14) ^ w) and a stride-2 convolution on a masked width."""
    rng = np.random.default_rng(9)

    def build(g, pg):
        g.add_input("img", 6, 16, 128)
        pg.input("img", 6, 16, 128, False)
        _conv(g, pg, "a", "img", "x", 6, 20, 3, rng, stride=2)   # 8 x 64 (aligned)
        _conv(g, pg, "b", "x", "y", 20, 40, 3, rng, stride=2)    # 4 x 32 (masked)
        _conv(g, pg, "c", "y", "out", 40, 64, 1, rng, act="leaky_relu")
        g.set_output("out")
        pg.output = "out"

    g, plan, pplan = _pair2d(wavec, build, 1)
    _assert_same_plan(plan, pplan)
    _assert_same_tcff(plan, pplan, tmp_path)


def test_2d_tap_offsets_by_hand():
    """One 3x3 tap row of the oracle against hand-computed offsets (aligned 64-wide layout):
    W_pad = 72, channel c of a tensor at base B starts at B + c * 66 * 72; tap (dy, dx) adds
    (1 + dy) * 72 + (1 + dx)."""
    pg = po.Graph()
    pg.input("img", 2, 64, 64, False)
    w = np.zeros((16, 2 * 9), np.uint16)
    pg.conv2d("c", "img", "out", 2, 16, 3, 3, 1, w, np.zeros(16, np.uint16))
    pg.output = "out"
    p = po.compile_plan(pg)
    wave = [c for c in p["cmds"] if c["type"] == 0][0]
    cs = 66 * 72
    base = p["input_off"]
    want = [base + c * cs + (1 + dy) * 72 + (1 + dx) for c in range(2) for dy in (-1, 0, 1)
            for dx in (-1, 0, 1)]
    assert list(wave["idx"][0, :18]) == want
    assert wave["geom"] == [3, 1, 16, 64, 64, 16 * cs, cs, 72, 1, 76]


@pytest.mark.parametrize("mistake", ["dy_sign", "kernel_transposed", "quad_order"])
def test_2d_planted_mistakes_are_caught(wavec, tmp_path, monkeypatch, mistake):
    """The 2-D comparison is sensitive: a flipped tap sign, a transposed 3x3 kernel on the
    stride-2 polyphase path or a wrong transposed-convolution quadrant order in the oracle each
    change the .tcff bytes."""
    rng = np.random.default_rng(3)
    if mistake == "dy_sign":
        monkeypatch.setattr(po, "tap_2d", lambda L, b, dy, dx: b + (1 - dy) * L.W_pad + (1 + dx))

    def build(g, pg):
        g.add_input("img", 4, 20, 20)
        pg.input("img", 4, 20, 20, False)
        if mistake == "quad_order":
            w = (rng.standard_normal((8, 4, 2, 2)) * 0.1).astype(np.float32)
            b = np.zeros(8, np.float32)
            g.add_upconv2x2("up", "img", "out", 4, 8, w, b)
            wq = _f16(w).reshape(8, 4, 4)[:, :, ::-1].copy()  # planted: quadrants reversed
            pg.upconv2x2("up", "img", "out", 4, 8, wq, _f16(b))
        else:
            w = (rng.standard_normal((16, 4, 3, 3)) * 0.1).astype(np.float32)
            b = np.zeros(16, np.float32)
            g.add_conv2d("c", "img", "out", 4, 16, 3, 3, w, b, stride=2, pad=1, act="relu")
            wr = _f16(w).reshape(16, 4, 3, 3)
            if mistake == "kernel_transposed":  # planted: ky <-> kx
                wr = wr.transpose(0, 1, 3, 2).copy()
            pg.conv2d("c", "img", "out", 4, 16, 3, 3, 2, wr.reshape(16, 36), _f16(b), act=1)
        g.set_output("out")
        pg.output = "out"

    g, plan, pplan = _pair2d(wavec, build, 1)
    path = tmp_path / "p.tcff"
    plan.save_tcff(path, "K44Model")
    assert path.read_bytes() != po.tcff_bytes(pplan, "K44Model")


@pytest.mark.parametrize("seed", range(6))
def test_canvas_allocator_invariants_on_random_graphs(wavec, seed):
    """The compiler's canvas allocator (reference wavec/k44_wave_compiler.hpp:388-593, restated in
    pass4) checked by invariants that do not depend on its tie-breaks, on random 1-D graphs of
    sparse waves, residual waves, RMSNorms and element-wise products reading random earlier
    tensors.  Liveness is computed here from the graph as built (a tensor lives from the node
    that writes it through its last reader; the plan input and output to the end):
      * every tensor starts on a 64-element boundary;
      * two tensors alive at the same node never share a canvas element (a node's output and
        its own inputs are alive together);
      * the canvas is exactly the highest reserved element, rounded up to 128."""
    rng = np.random.default_rng(1000 + seed)
    T = int(rng.choice([64, 100, 256]))
    stride = (T + 63) // 64 * 64
    g = wavec.WaveGraph(kv_cache_max_seq=0, fold_rmsnorm_gamma=False)
    C0 = int(rng.integers(40, 200))
    g.add_input("x", C0, 1, T, is_1d=True)
    chans = {"x": C0}
    order = ["x"]
    reads = {"x": []}  # tensor -> node indices that read it
    srcs = []  # first input of every node
    for k in range(int(rng.integers(8, 20))):
        name = f"t{k}"
        kind = rng.choice(["wave", "wave", "res", "norm", "mul"])
        src = order[int(rng.integers(max(0, len(order) - 4), len(order)))]
        if kind == "norm":
            g.add_rmsnorm(f"n{k}", src, name, chans[src], np.ones(chans[src], np.float32))
            chans[name] = chans[src]
            ins = [src]
        elif kind == "mul":
            same = [t for t in order if chans[t] == chans[src] and t != src]
            if not same:
                continue
            other = same[int(rng.integers(0, len(same)))]
            g.add_swiglu(f"m{k}", src, other, name)
            chans[name] = chans[src]
            ins = [src, other]
        else:
            cout = int(rng.integers(16, 160))
            res = None
            if kind == "res":
                cands = [t for t in order if chans[t] == cout]
                if not cands:
                    cout = chans[src]
                    cands = [src]
                res = cands[int(rng.integers(0, len(cands)))]
            fan = int(rng.integers(1, 5)) * 8
            rows = rng.integers(0, chans[src], size=(cout, fan)).astype(np.uint32)
            _w = synth.normal_f16(rng, (cout, fan), 0.05)
            g.add_sparse_wave(f"w{k}", src, name, rows, _w, None, act="relu", res_blob=res)
            chans[name] = cout
            ins = [src] + ([res] if res else [])
        node = len(order) - 1  # index of this node's command (the input has none)
        srcs.append(ins[0])
        for t in ins:
            reads[t].append(node)
        reads[name] = []
        order.append(name)
    g.set_output(order[-1])
    plan = g.compile()
    s = plan.summary
    cmds = s["cmds"]
    assert len(cmds) == len(order) - 1
    end = len(cmds)
    span = {}  # tensor -> (canvas lo, hi, def node, last node)
    span["x"] = None
    for i, (name, c) in enumerate(zip(order[1:], cmds)):
        reserve = -(-int(c["Cout"]) * stride // 64) * 64
        lo = int(c["y_off"])
        last = end if name == order[-1] else max(reads[name], default=i)
        span[name] = (lo, lo + reserve, i, last)
    # the plan input is allocated first, at offset 0, and lives to the end
    span["x"] = (0, -(-C0 * stride // 64) * 64, -1, end)
    assert _alloc_violations(span, int(s["canvas_elems"])) == []
    for i in reads["x"]:  # the plan input sits at offset 0
        if srcs[i] == "x":
            assert int(cmds[i]["src_off"]) == 0
    # The check is not vacuous: moving one tensor onto another that is alive at the same time
    # (what an allocator freeing a tensor too early would do) is reported.
    pairs = [(a, b) for a in span for b in span if a != b and a != "x" and
             not (span[a][3] < span[b][2] or span[b][3] < span[a][2])]
    a, b = pairs[int(rng.integers(0, len(pairs)))]
    bad = dict(span)
    lo_a, hi_a, d_a, e_a = span[a]
    bad[a] = (span[b][0], span[b][0] + hi_a - lo_a, d_a, e_a)
    assert _alloc_violations(bad, int(s["canvas_elems"]))


def _alloc_violations(span, canvas_elems):
    """Violated allocator invariants of {tensor: (lo, hi, first node, last node)}."""
    out = []
    items = list(span.items())
    for name, (lo, hi, d, l) in items:
        if lo % 64:
            out.append(f"{name} not 64-aligned")
    for a in range(len(items)):
        na, (la, ha, da, ea) = items[a]
        for b in range(a + 1, len(items)):
            nb, (lb, hb, db, eb) = items[b]
            if not (ea < db or eb < da) and not (ha <= lb or hb <= la):
                out.append(f"{na} and {nb} alive together share elements")
    top = max(hi for _, (lo, hi, d, l) in items)
    if canvas_elems != -(-top // 128) * 128:
        out.append(f"canvas {canvas_elems} != highest element {top} rounded to 128")
    return out


def test_conv1d_tap_before_the_canvas_is_refused(wavec):
    """A 1-D convolution applied directly to the plan input (canvas offset 0) would gather its
    first channel's dx = -1 tap from offset -1; the reference wraps it to 0xFFFFFFFF
    (k44_plan_types.hpp:593-595), this compiler refuses the plan."""
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", 32, 1, 64, is_1d=True)
    g.add_conv2d("c", "x", "y", 32, 16, 1, 3, np.zeros((16, 32, 1, 3), np.float32), pad=1)
    with pytest.raises(RuntimeError, match="32-bit index range"):
        g.compile()

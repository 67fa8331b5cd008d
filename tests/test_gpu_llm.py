"""LLM-shaped plans on the GPU (the decoder of config 5 at a tiny size): every command checked
against the CPU restatement on the inputs the device itself read, the whole prefill against the
oracle run end to end, prefill -> decode hand-over, decode steps, and HIP-graph replay with the
device-side id history."""
import dataclasses
import numpy as np
import pytest

from oracle import llm_oracle as lo
from snntome_amd import synth

from wave_cases import PATH_IDS, TOL, stride_of

pytestmark = pytest.mark.gpu

TINY = synth.LLMSpec(layers=2, d=256, ffn=384, vocab=640, S=64, requests=2, prompt=64,
                     decode_steps=4, seed=9)
# End-to-end tolerance, relative to the largest logit: the device and the oracle round every
# stored tensor to fp16 and may round a value differently by one ulp (each command alone stays
# within TOL); through 2 layers of residual streams, RMSNorms and gates these differences add up
# to a few fp16 ulps of the logits' scale (one ulp at the largest logit is ~1e-3 of it).  The
# per-element metric of TOL does not apply end to end: its 1e-2 floor makes a 1-ulp difference
# on a logit near zero look like a 10 % error.
E2E_TOL = 1e-2
ACTS = {"q": "sigmoid", "k": "silu", "g": "silu"}


def _log(msg):
    print(msg, flush=True)


def _read(plan, off, c, t):
    return plan.read_canvas(int(off), int(c) * t).view(np.float16).reshape(int(c), t)


def _projections(spec, wts):
    out = {"head": (wts.head, None)}
    for l in range(spec.layers):
        for k, p in wts.proj[l].items():
            out[f"l{l}.{k}"] = (p, ACTS.get(k))
    return out


def _groups(cmds):
    """Consecutive commands of one graph node (the sub-waves "name/0", "name/1", ... of a pruned
    projection) -> [(node name, first index, count, first cmd)]."""
    out = []
    for i, c in enumerate(cmds):
        base = c["name"].split("/")[0]
        if out and out[-1][0] == base:
            out[-1][2] += 1
        else:
            out.append([base, i, 1, c])
    return out


def _check_commands(plan, spec, wts, ids, decode, tag):
    """Runs the plan node by node; each node's output (token columns < the plan's token count)
    is compared with the CPU restatement of that node applied to the canvas contents it read."""
    valid = len(ids)
    T = stride_of(valid)
    projs = _projections(spec, wts)
    mixes = {f"l{l}.shift": wts.mix[l] for l in range(spec.layers)}
    plan.set_ids(ids)
    worst = {}
    for name, first, count, c in _groups(plan.cmds):
        typ = c["type"]
        cout = c["logical_Cout"]
        if typ == "K44_WAVE":
            x = _read(plan, c["src_off"], c["Cin"], T)
            res = _read(plan, c["res_off"], cout, T) if c["has_residual"] else None
        elif typ in ("RMSNORM_1D", "TOKEN_SHIFT_1D", "ARGMAX_1D"):
            x = _read(plan, c["src_off"], c["Cin"], T)
        elif typ == "SWIGLU_MUL_1D":
            a = _read(plan, c["src_off"], cout, T)
            b = _read(plan, c["src2_off"], cout, T)
        if typ == "TOKEN_SHIFT_1D" and decode:
            st_in = _read(plan, c["state_off"], spec.d * (spec.rf - 1), 64).reshape(
                spec.d, spec.rf - 1, 64)
        plan.execute_range(first, count)
        if typ == "ARGMAX_1D":
            got = plan.get_ids(valid)
            assert np.array_equal(got, lo.argmax(x, valid)), f"{tag} {name}"
            continue
        y = _read(plan, c["y_off"], cout, T)
        if typ == "EMBED_1D":
            assert np.array_equal(y.view(np.uint16), lo.embed(wts.embed, ids, T).view(np.uint16))
            continue
        if typ == "SWIGLU_MUL_1D":  # a product of two fp16 is exact in fp32: one rounding
            assert np.array_equal(y[:, :valid].view(np.uint16),
                                  lo.mul(a, b)[:, :valid].view(np.uint16)), name
            continue
        if typ == "K44_WAVE":
            p, act = projs[name]
            ref = lo.project(x, p.starts, spec.S, 1, p.weights, p.bias, act, res, f64=True)
        elif typ == "RMSNORM_1D":
            ref = lo.rmsnorm_f64(x)
        else:  # TOKEN_SHIFT_1D
            st = _read(plan, c["state_off"], spec.d * (spec.rf - 1), 64).reshape(
                spec.d, spec.rf - 1, 64)
            if decode:
                ref, st_ref = lo.token_shift_decode(x, mixes[name], st_in, valid, f64=True)
            else:
                ref, st_ref = lo.token_shift(x, mixes[name], spec.prompt, valid, f64=True)
            assert np.array_equal(st.view(np.uint16), st_ref.view(np.uint16)), f"{name} state"
        # token columns past the plan's token count are unspecified (narrow kernels skip them)
        err = lo.orc.rel_err(y[:, :valid].astype(np.float64), ref[:, :valid])
        worst[typ] = max(worst.get(typ, 0.0), err)
        assert err <= TOL, f"{tag} {name}: rel err {err:.3e}"
    _log(f"[{tag}] per-node worst rel err: "
         + ", ".join(f"{k} {v:.2e}" for k, v in sorted(worst.items())))


@pytest.mark.parametrize("path", ["auto", "valu"])
def test_llm_prefill_commandwise_and_end_to_end(wavec, tuning, path):
    if path != "auto":
        tuning("path", PATH_IDS[path])
    wts = synth.llm_weights(TINY)
    plan = synth.build_llm_graph(TINY, wts, decode=False, wavec_mod=wavec).compile()
    plan.init_gpu()
    paths = {w["path"] for w in plan.exec_report()["waves"]}
    _log(f"[llm prefill {path}] wave paths {sorted(paths)}")
    if path == "auto":
        assert paths and paths <= {"mfma_tile", "mfma_dma"}
    else:
        assert paths == {"valu_gather_dot"}
    rng = np.random.default_rng(1)
    ids = rng.integers(0, TINY.vocab, TINY.requests * TINY.prompt).astype(np.uint32)
    _check_commands(plan, TINY, wts, ids, False, f"llm prefill {path}")
    # the whole prefill once more in one call, against the oracle run end to end
    plan.set_ids(ids)
    plan.execute(1)
    valid = ids.size
    T = stride_of(valid)
    head = next(c for c in plan.cmds if c["name"].split("/")[0] == "head")
    logits = _read(plan, head["y_off"], head["logical_Cout"], T)[:, :valid].astype(np.float64)
    ref = lo.llm_forward(TINY, wts, ids, decode=False)
    want = ref.tensors["logits"][:, :valid].astype(np.float64)
    scale = np.abs(want).max()
    err = np.abs(logits - want).max() / scale
    _log(f"[llm prefill {path}] end-to-end max|d| / max|logit| = {err:.3e} (max|logit| "
         f"{scale:.2f}, per-element metric {lo.orc.rel_err(logits, want):.2e})")
    assert err <= E2E_TOL
    got = plan.get_ids(valid)
    srt = np.sort(ref.tensors["logits"][:, :valid].astype(np.float64), axis=0)
    clear = (srt[-1] - srt[-2]) > 0.05  # ids whose top-2 margin dwarfs the logit error
    assert clear.mean() > 0.5
    assert np.array_equal(got[clear], ref.ids[clear])


def test_llm_decode_handoff_and_steps(wavec):
    wts = synth.llm_weights(TINY)
    pre = synth.build_llm_graph(TINY, wts, decode=False, wavec_mod=wavec).compile()
    dec = synth.build_llm_graph(TINY, wts, decode=True, wavec_mod=wavec).compile()
    pre.init_gpu()
    dec.init_gpu()
    R, P = TINY.requests, TINY.prompt
    rng = np.random.default_rng(2)
    ids = rng.integers(0, TINY.vocab, R * P).astype(np.uint32)
    pre.set_ids(ids)
    pre.execute(1)
    synth.llm_handoff(TINY, pre, dec)
    assert np.array_equal(dec.get_ids(R), pre.get_ids(R * P)[P - 1::P])
    shifts_pre = {c["name"]: c for c in pre.cmds if c["type"] == "TOKEN_SHIFT_1D"}
    n_st = TINY.d * (TINY.rf - 1)
    for c in dec.cmds:
        if c["type"] == "TOKEN_SHIFT_1D":
            a = dec.read_canvas(int(c["state_off"]), n_st * 64)
            b = pre.read_canvas(int(shifts_pre[c["name"]]["state_off"]), n_st * 64)
            assert np.array_equal(a, b)
    for step in range(TINY.decode_steps):
        _check_commands(dec, TINY, wts, dec.get_ids(R), True, f"llm decode step {step}")


def test_llm_decode_graph_replay_matches_eager(wavec):
    """Two decode plans start from the same hand-over; one runs kernel by kernel, the other as
    replays of one captured HIP graph with the device-side id history; every step agrees bit for
    bit (ids and the logits canvas)."""
    spec = TINY
    steps = 6
    wts = synth.llm_weights(spec)
    pre = synth.build_llm_graph(spec, wts, decode=False, wavec_mod=wavec).compile()
    eager = synth.build_llm_graph(spec, wts, decode=True, wavec_mod=wavec).compile()
    graph = synth.build_llm_graph(spec, wts, decode=True, wavec_mod=wavec).compile()
    for p in (pre, eager, graph):
        p.init_gpu()
    R = spec.requests
    pre.set_ids(np.random.default_rng(3).integers(0, spec.vocab, R * spec.prompt))
    pre.execute(1)
    synth.llm_handoff(spec, pre, eager)
    synth.llm_handoff(spec, pre, graph)
    graph.use_graph(True)
    graph.set_history(steps)
    head = next(c for c in eager.cmds if c["name"].split("/")[0] == "head")
    want_ids, want_logits = [], []
    for _ in range(steps):
        eager.execute(1)
        want_ids.append(eager.get_ids(R))
        want_logits.append(eager.read_canvas(int(head["y_off"]), spec.vocab * 64))
    # replays 1 and 2 one at a time with host reads between them, then the rest in one call
    for s in range(2):
        graph.execute(1)
        assert np.array_equal(graph.get_ids(R), want_ids[s])
        assert np.array_equal(graph.read_canvas(int(head["y_off"]), spec.vocab * 64),
                              want_logits[s])
    graph.execute(steps - 2)
    assert np.array_equal(graph.read_canvas(int(head["y_off"]), spec.vocab * 64),
                          want_logits[-1])
    hist = graph.get_history(steps, R)
    assert hist.shape == (steps, R)
    assert np.array_equal(hist, np.stack(want_ids))
    _log(f"[llm graph] {steps} decode steps, ids {hist.tolist()}")


def test_token_shift_long_rf_and_many_requests(wavec):
    """Token shift alone at rf = 9 (the kernel's maximum) with 64 requests of 3 tokens (the
    maximum number of requests) and a non-multiple-of-64 token count."""
    D, rf, seq, req = 80, 9, 3, 64
    valid = seq * req  # 192 tokens
    rng = np.random.default_rng(4)
    mu = (rng.standard_normal((D, rf)) * 0.5).astype(np.float16)
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", D, 1, valid, is_1d=True)
    g.add_token_shift("ts", "x", "y", mu, seq)
    plan = g.compile()
    plan.init_gpu()
    T = stride_of(valid)
    x = (rng.standard_normal((D, T)) * 2).astype(np.float16)
    x[:, valid:] = 0
    c = plan.cmds[0]
    plan.write_canvas(int(c["src_off"]), x)
    plan.execute(1)
    y = _read(plan, c["y_off"], D, T)
    ref, st = lo.token_shift(x, mu, seq, valid, f64=True)
    assert lo.orc.rel_err(y.astype(np.float64), ref) <= TOL
    assert not y[:, valid:].any()
    got_st = _read(plan, c["state_off"], D * (rf - 1), 64).reshape(D, rf - 1, 64)
    # requests shorter than rf - 1 leave the older state slots untouched (zero)
    assert np.array_equal(got_st.view(np.uint16), st.view(np.uint16))


@pytest.mark.parametrize("rf", [1, 2, 5, 9])
def test_token_shift_decode_every_rf(wavec, rf):
    """Decode token shift (one token per request, state shifted in place) for receptive fields
    1..9 (one kernel instance per rf) over two steps, against the oracle: outputs within
    tolerance, state bit-exact."""
    D, req = 96, 13
    rng = np.random.default_rng(rf)
    mu = (rng.standard_normal((D, rf)) * 0.5).astype(np.float16)
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", D, 1, req, is_1d=True)
    g.add_token_shift("ts", "x", "y", mu, 1, decode=True)
    plan = g.compile()
    plan.init_gpu()
    c = plan.cmds[0]
    state = np.zeros((D, max(rf - 1, 0), 64), np.float16)
    if rf > 1:
        state = (rng.standard_normal(state.shape)).astype(np.float16)
        plan.write_canvas(int(c["state_off"]), state.reshape(D * (rf - 1), 64))
    for step in range(2):
        x = np.zeros((D, 64), np.float16)
        x[:, :req] = rng.standard_normal((D, req)).astype(np.float16)
        plan.write_canvas(int(c["src_off"]), x)
        plan.execute(1)
        y = _read(plan, c["y_off"], D, 64)
        ref, state = lo.token_shift_decode(x, mu, state, req, f64=True)
        assert lo.orc.rel_err(y.astype(np.float64), ref) <= TOL
        assert not y[:, req:].any()
        if rf > 1:
            got = _read(plan, c["state_off"], D * (rf - 1), 64).reshape(D, rf - 1, 64)
            assert np.array_equal(got[:, :, :req].view(np.uint16),
                                  state[:, :, :req].view(np.uint16)), step


@pytest.mark.parametrize("V,tokens", [(1000, 100), (32000, 64), (300, 1000)])
def test_argmax_chunks_and_ties(wavec, V, tokens):
    """Two-pass argmax (per-chunk partials, merge in chunk order) against the lowest-index rule,
    with planted ties inside one chunk and across chunk boundaries."""
    rng = np.random.default_rng(V)
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", V, 1, tokens, is_1d=True)
    g.add_argmax("am", "x", "ids")
    plan = g.compile()
    plan.init_gpu()
    T = stride_of(tokens)
    x = (rng.standard_normal((V, T)) * 3).astype(np.float16)
    x[:, tokens:] = 0
    top = np.float16(20.0)
    for t in range(0, tokens, 3):  # ties: two or three equal maxima at random channels
        cs = np.sort(rng.choice(V, size=2 + t % 2, replace=False))
        x[cs, t] = top
    x[:, 1] = np.float16(-np.inf)  # all -inf: channel 0
    plan.write_canvas(int(plan.cmds[0]["src_off"]), x)
    plan.execute(1)
    got = plan.get_ids(tokens)
    want = lo.argmax(x, tokens)
    assert want[1] == 0
    assert np.array_equal(got, want)


@pytest.mark.parametrize("D,tokens", [(100, 70), (2048, 64), (300, 1000)])
def test_rmsnorm_and_embed_shapes(wavec, D, tokens):
    rng = np.random.default_rng(D)
    V = 97
    table = (rng.standard_normal((V, D)) * 2).astype(np.float16)
    g = wavec.WaveGraph(kv_cache_max_seq=0, fold_rmsnorm_gamma=False)
    g.add_input("tok", 1, 1, tokens, is_1d=True)
    g.add_embedding("emb", "tok", "e", table)
    gamma = rng.uniform(0.5, 1.5, D).astype(np.float32)
    g.add_rmsnorm("n", "e", "y", D, gamma)
    plan = g.compile()
    plan.init_gpu()
    ids = rng.integers(0, V + 5, tokens).astype(np.uint32)  # some ids >= vocab -> zero rows
    plan.set_ids(ids)
    plan.execute(1)
    T = stride_of(tokens)
    ce, cn = plan.cmds[0], plan.cmds[1]
    e = _read(plan, ce["y_off"], D, T)
    assert np.array_equal(e.view(np.uint16), lo.embed(table, ids, T).view(np.uint16))
    y = _read(plan, cn["y_off"], D, T)[:, :tokens]  # columns past the token count: unspecified
    ref = lo.rmsnorm_f64(e, gamma.astype(np.float16))[:, :tokens]
    assert lo.orc.rel_err(y.astype(np.float64), ref) <= TOL


@pytest.mark.parametrize("tokens,tiles", [(64, 2), (64, 40), (512, 1), (300, 3)])
def test_mfma_split_k_matches_oracle_and_unsplit(wavec, orc, tuning, tokens, tiles):
    """Small tile x token-tile grids run split-K (partials + ordered reduction); the result is
    within tolerance of the oracle and of the single-pass kernel, and identical across runs."""
    rng = np.random.default_rng(tokens + tiles)
    S, K, nt = 64, 6, 64
    C = 4096
    starts = (rng.integers(0, C // S, size=(tiles, K)) * S).astype(np.uint32)
    cout = tiles * nt
    w = synth.normal_f16(rng, (cout, K * S), 0.05)
    b = synth.normal_f16(rng, (cout,), 0.05)
    outs = {}
    for mode in ("split", "single"):
        if mode == "single":
            tuning("splitk", 0)
        g = wavec.WaveGraph(kv_cache_max_seq=0)
        g.add_input("x", C, 1, tokens, is_1d=True)
        g.add_cluster_wave("w", "x", "y", starts, S, w, b, cluster=nt, act="gelu", res_blob="x")
        plan = g.compile()
        plan.init_gpu()
        rep = plan.exec_report()["waves"][0]
        assert rep["path"] in ("mfma_tile", "mfma_dma")
        assert (rep["ksplit"] > 1) == (mode == "split"), rep
        plan.fill_input_uniform(3)
        plan.execute(1)
        st = stride_of(tokens)
        canvas = plan.read_canvas(0, int(plan.summary["canvas_elems"]))
        x0 = int(plan.cmds[0]["src_off"])
        y0 = int(plan.cmds[0]["y_off"])
        y = canvas[y0:y0 + cout * st].view(np.float16).reshape(cout, st).astype(np.float64)
        seg = (x0 + starts.astype(np.uint64) * st).ravel()
        ref = orc.wave_f64(canvas, seg, w, b, None, K, S, nt, st, st, st, "gelu", res_off=x0)
        err = orc.rel_err(y, ref)
        _log(f"[split-k {tokens}x{tiles} {mode}] ksplit {rep['ksplit']} rel err {err:.3e}")
        assert err <= TOL
        plan.execute(1)
        again = plan.read_canvas(y0, cout * st)
        assert np.array_equal(again, canvas[y0:y0 + cout * st])  # deterministic reduction
        outs[mode] = y
    assert orc.rel_err(outs["split"], outs["single"]) <= TOL


@pytest.mark.parametrize("decode", [False, True])
def test_grouped_launches_match_per_wave(wavec, tuning, decode):
    """Independent MFMA waves (sub-waves of a pruned projection, projections of one input) run
    as one grouped launch; the logits are bit-identical to launching every wave alone."""
    wts = synth.llm_weights(TINY)
    R = TINY.requests
    n = R if decode else R * TINY.prompt
    ids = np.random.default_rng(8).integers(0, TINY.vocab, n).astype(np.uint32)
    out = {}
    for mode in ("grouped", "alone"):
        if mode == "alone":
            tuning("group", 0)
        plan = synth.build_llm_graph(TINY, wts, decode=decode, wavec_mod=wavec).compile()
        plan.init_gpu()
        rep = plan.exec_report()
        sizes = [len(g) for g in rep["groups"]]
        _log(f"[groups {mode} decode={decode}] {len(sizes)} groups, largest {max(sizes)}, "
             f"{rep['launches_per_run']} launches per run")
        assert (max(sizes) > 1) == (mode == "grouped")
        plan.set_ids(ids)
        plan.execute(1)
        head = next(c for c in plan.cmds if c["name"].split("/")[0] == "head")
        out[mode] = plan.read_canvas(int(head["y_off"]), TINY.vocab * stride_of(n))
        out[mode + "_ids"] = plan.get_ids(n)
    assert np.array_equal(out["grouped"], out["alone"])
    assert np.array_equal(out["grouped_ids"], out["alone_ids"])


@pytest.mark.parametrize("rf,requests", [(4, 2), (3, 9), (2, 16)])
def test_folded_multiplies_match_unfolded(wavec, tuning, rf, requests):
    """Decode plans fold the element-wise multiplies (k*v, q*(k*v), g*u) into the gathers of the
    narrow MFMA waves that read the products, and the RMSNorms after projections into their
    producers (exact sums of squares per tile) and readers (normalising gathers; for the norms
    that run the decode token shift, normalising and shifting gathers whose shifted state is
    copied back by the next launch); ids, logits and token-shift states of several decode steps
    are bit-identical to the plan that launches every multiply and norm (tuning switch
    fuse=0).  Receptive fields 2-4 (state rows 1-3) and batches of 2, 9 and 16 requests."""
    spec = dataclasses.replace(TINY, rf=rf, requests=requests)
    steps = 4
    wts = synth.llm_weights(spec)
    pre = synth.build_llm_graph(spec, wts, decode=False, wavec_mod=wavec).compile()
    pre.init_gpu()
    plans = {}
    tuning("program", 0)  # both plans launch kernel by kernel (the folds are what is compared)
    for mode in ("folded", "launched"):
        if mode == "launched":
            tuning("fuse", 0)
        else:
            tuning("fuse", -1)
        p = synth.build_llm_graph(spec, wts, decode=True, wavec_mod=wavec).compile()
        p.init_gpu()
        plans[mode] = p
    rep = plans["folded"].exec_report()
    fused = [a for a in rep["aux"] if a["fused"] and a["type"] == "SWIGLU_MUL_1D"]
    shifts = [a for a in rep["aux"] if a["fused"] and a["type"] == "TOKEN_SHIFT_1D"]
    norms = [a for a in rep["aux"] if a["type"] == "RMSNORM_1D"]
    norm_folded = [a for a in norms if a["fused"]]
    norm_shifted = [a for a in norm_folded if "token shift" in a["fuse_note"]]
    norm_scaled = [a for a in norms if not a["fused"] and "sums of squares stored" in a["fuse_note"]]
    prods = sorted({w["xprod"] for w in rep["waves"]})
    _log(f"[fold] {len(fused)} multiplies folded, {len(shifts)} token shifts run by their "
         f"RMSNorm, {len(norm_folded)} RMSNorms folded into their readers "
         f"({len(norm_shifted)} with their token shift), "
         f"{len(norm_scaled)} run with their producers' scales, xprod kinds {prods}, "
         f"{rep['launches_per_run']} vs {plans['launched'].exec_report()['launches_per_run']} "
         "launches per run")
    assert len(fused) == 3 * spec.layers and prods == [2, 3, 4, 5] and len(shifts) == spec.layers
    # every norm folds: the first of every layer with its token shift (layer 0's after the
    # embedding, which stores the sums of squares and refreshes that shift's compact state
    # copy), the second of every layer and the final one
    assert len(norm_folded) == 2 * spec.layers + 1 and len(norm_shifted) == spec.layers
    assert len(norm_scaled) == 0
    embeds = [a for a in rep["aux"] if a["type"] == "EMBED_1D"]
    assert len(embeds) == 1 and embeds[0]["refreshes_state_of"] >= 0
    assert not any(a["fused"] for a in plans["launched"].exec_report()["aux"])
    R = spec.requests
    pre.set_ids(np.random.default_rng(5).integers(0, spec.vocab, R * spec.prompt))
    pre.execute(1)
    head = next(c for c in pre.cmds if c["name"].split("/")[0] == "head")
    out = {}
    for mode, p in plans.items():
        synth.llm_handoff(spec, pre, p)
        hd = next(c for c in p.cmds if c["name"].split("/")[0] == "head")
        ids, logits, states = [], [], []
        shifts_of = [c for c in p.cmds if c["type"] == "TOKEN_SHIFT_1D"]
        for _ in range(steps):
            p.execute(1)
            ids.append(p.get_ids(R))
            # token columns past the plan's token count are unspecified (the narrow kernels
            # compute 16 columns; a folded norm scales all 16, the norm kernel whole octets)
            logits.append(p.read_canvas(int(hd["y_off"]), spec.vocab * 64).reshape(-1, 64)[:, :R])
            states.append(np.stack([
                p.read_canvas(int(c["state_off"]), spec.d * (spec.rf - 1) * 64).reshape(-1, 64)
                for c in shifts_of]))
        out[mode] = (np.stack(ids), np.stack(logits), np.stack(states))
    assert head is not None
    assert np.array_equal(out["folded"][0], out["launched"][0])
    assert np.array_equal(out["folded"][1], out["launched"][1])
    # the whole state rows (columns past R are carried unchanged by both)
    assert np.array_equal(out["folded"][2], out["launched"][2])


def test_decode_inkernel_splitk_matches_epilogue_kernel(wavec, tuning):
    """Split narrow waves of 64-neuron tiles reduce their chunk partials in the last workgroup
    of each tile (per-tile arrival counters; device-coherent partial stores and loads, or, by
    default, plain ones through the L2 of the one XCD every chunk of a tile runs on; with the
    waves' weight addresses and geometry preloaded as kernel arguments or not); ids and
    logits of several decode steps, eager and HIP-graph replays, are bit-identical to the plan
    whose partials are reduced by the split-K epilogue kernel (narrow_reduce=0), and every
    counter is back at zero between launches (a later launch sums the right chunks; the
    executor checks the XCD-local counters after every run)."""
    # contractions of 32 k-steps (d-input: 4 of 8 clusters of 256) and 40 (FFN input: 5 of 10):
    # 2 and 3 chunks of <= 16 k-steps, the last one ragged
    spec = synth.LLMSpec(layers=2, d=2048, ffn=2560, vocab=1024, S=256, requests=4, prompt=64,
                         decode_steps=5, seed=13)
    steps = 5
    wts = synth.llm_weights(spec)
    pre = synth.build_llm_graph(spec, wts, decode=False, wavec_mod=wavec).compile()
    pre.init_gpu()
    R = spec.requests
    pre.set_ids(np.random.default_rng(31).integers(0, spec.vocab, R * spec.prompt))
    pre.execute(1)
    out = {}
    tuning("program", 0)  # split narrow waves exist only in kernel-by-kernel launches
    for mode in ("kernel", "in_launch", "xcd_local", "no_preload"):
        tuning("narrow_reduce", 0 if mode == "kernel" else 1)
        tuning("narrow_local", 1 if mode in ("xcd_local", "no_preload") else 0)
        # no_preload: every wave reads its weights' address and geometry from its descriptor
        tuning("narrow_pre", 0 if mode == "no_preload" else 1)
        tuning("narrow_wgs", 512)  # many chunks per tile: every narrow wave splits
        p = synth.build_llm_graph(spec, wts, decode=True, wavec_mod=wavec).compile()
        p.init_gpu()
        rep = p.exec_report()
        split = [w for w in rep["waves"] if w["path"] == "mfma_narrow" and w["ksplit"] > 1]
        inl = [w for w in split if w["reduce_in_kernel"]]
        loc = [w for w in split if w["reduce_xcd_local"]]
        _log(f"[narrow reduce {mode}] {len(split)} split narrow waves, {len(inl)} reduced in "
             f"their launch ({len(loc)} XCD-locally), chunks "
             f"{sorted({w['ksplit'] for w in split})}, {rep['launches_per_run']} launches per run")
        assert split and len(inl) == (0 if mode == "kernel" else len(split))
        # (XCD-local only where set-up found workgroups 8 apart sharing an XCD)
        want_loc = mode in ("xcd_local", "no_preload") and rep["xcd_local_ok"]
        assert len(loc) == (len(split) if want_loc else 0)
        synth.llm_handoff(spec, pre, p)
        hd = next(c for c in p.cmds if c["name"].split("/")[0] == "head")
        ids, logits = [], []
        for s in range(steps):
            if s == 2:
                p.use_graph(True)  # steps 2.. as replays of one captured graph
            p.execute(1)
            ids.append(p.get_ids(R))
            # the plan's token columns (the others are unspecified)
            logits.append(p.read_canvas(int(hd["y_off"]), spec.vocab * 64).reshape(-1, 64)[:, :R])
        out[mode] = (np.stack(ids), np.stack(logits))
        p.release_gpu()
    for mode in ("in_launch", "xcd_local", "no_preload"):
        assert np.array_equal(out["kernel"][0], out[mode][0])
        assert np.array_equal(out["kernel"][1], out[mode][1])


def test_prefill_multiply_chain_matches_launched(wavec, tuning):
    """Prefill plans run m = q*(k*v) as one 3-operand multiply (the inner product k*v is not
    launched); logits and next ids are bit-identical to the plan that launches both multiplies
    (tuning switch fuse=0)."""
    wts = synth.llm_weights(TINY)
    ids = np.random.default_rng(23).integers(0, TINY.vocab, TINY.requests * TINY.prompt)
    ids = ids.astype(np.uint32)
    out = {}
    for mode in ("chained", "launched"):
        tuning("fuse", -1 if mode == "chained" else 0)
        p = synth.build_llm_graph(TINY, wts, decode=False, wavec_mod=wavec).compile()
        p.init_gpu()
        rep = p.exec_report()
        chains = [a for a in rep["aux"] if a["chain"]]
        inner = [a for a in rep["aux"] if a["fused"] and a["type"] == "SWIGLU_MUL_1D"]
        _log(f"[prefill chain {mode}] {len(chains)} chained multiplies, {len(inner)} not "
             f"launched, {rep['launches_per_run']} launches per run")
        assert (len(chains), len(inner)) == ((TINY.layers, TINY.layers) if mode == "chained"
                                             else (0, 0))
        p.set_ids(ids)
        p.execute(1)
        head = next(c for c in p.cmds if c["name"].split("/")[0] == "head")
        T = stride_of(ids.size)
        out[mode] = (p.get_ids(ids.size), _read(p, head["y_off"], head["logical_Cout"], T))
        p.release_gpu()
    assert np.array_equal(out["chained"][0], out["launched"][0])
    assert np.array_equal(out["chained"][1].view(np.uint16), out["launched"][1].view(np.uint16))


def test_decode_step_full_width_against_oracle(wavec):
    """One decode step of the config-5 decoder at its real widths (d 2048, FFN 5632, vocab
    32,000, 16 requests; 2 of the 16 layers, zero token-shift history): folded multiplies,
    relocated operands, split-K chunking, union tiles of up to 11 clusters and the 500-tile
    head, against the fp64-accumulating oracle end to end."""
    spec = synth.LLMSpec(layers=2)
    wts = synth.llm_weights(spec)
    dec = synth.build_llm_graph(spec, wts, decode=True, wavec_mod=wavec).compile()
    dec.init_gpu()
    rep = dec.exec_report()
    n_mul = sum(a["fused"] and a["type"] == "SWIGLU_MUL_1D" for a in rep["aux"])
    n_shift = sum(a["fused"] and a["type"] == "TOKEN_SHIFT_1D" for a in rep["aux"])
    _log(f"[decode full width] {len(rep['waves'])} waves, {n_mul} multiplies folded, "
         f"{n_shift} token shifts run by their RMSNorm, {rep['launches_per_run']} launches per step")
    assert n_mul == 3 * spec.layers and n_shift == spec.layers
    R = spec.requests
    ids = np.random.default_rng(11).integers(0, spec.vocab, R).astype(np.uint32)
    dec.set_ids(ids)
    dec.execute(1)
    head = next(c for c in dec.cmds if c["name"].split("/")[0] == "head")
    logits = _read(dec, head["y_off"], head["logical_Cout"], 64)[:, :R].astype(np.float64)
    zero = [np.zeros((spec.d, spec.rf - 1, 64), np.float16) for _ in range(spec.layers)]
    ref = lo.llm_forward(spec, wts, ids, decode=True, shift_state=zero)
    want = ref.tensors["logits"][:, :R].astype(np.float64)
    scale = np.abs(want).max()
    err = np.abs(logits - want).max() / scale
    _log(f"[decode full width] max|d| / max|logit| = {err:.3e} (max|logit| {scale:.2f})")
    assert err <= E2E_TOL
    srt = np.sort(want, axis=0)
    clear = (srt[-1] - srt[-2]) > 0.05
    assert np.array_equal(dec.get_ids(R)[clear], ref.ids[clear])


@pytest.mark.parametrize("decode", [False, True])
@pytest.mark.parametrize("mode", ["commands", "runs"])
def test_plan_checker_tiny(wavec, decode, mode):
    """The node-by-node checker of the full-size tests (tests/llm_check.py) on the tiny decoder:
    command-wise and run-wise (group launches, folded multiplies, fused RMSNorm + token shift),
    prefill and a decode step after the hand-over."""
    from llm_check import PlanChecker

    wts = synth.llm_weights(TINY)
    pre = synth.build_llm_graph(TINY, wts, decode=False, wavec_mod=wavec).compile()
    pre.init_gpu()
    R, P = TINY.requests, TINY.prompt
    ids = np.random.default_rng(21).integers(0, TINY.vocab, R * P).astype(np.uint32)
    if not decode:
        PlanChecker(pre, TINY, wts, R * P, False, log=_log).run(mode, ids, f"tiny prefill {mode}")
        return
    pre.set_ids(ids)
    pre.execute(1)
    dec = synth.build_llm_graph(TINY, wts, decode=True, wavec_mod=wavec).compile()
    dec.init_gpu()
    synth.llm_handoff(TINY, pre, dec)
    chk = PlanChecker(dec, TINY, wts, R, True, log=_log)
    for step in range(2):
        chk.run(mode, dec.get_ids(R), f"tiny decode {mode} step {step}")


def _norm_shift_graph(wavec, D, req, rf, mu, gamma, dead_input):
    """tok -> embedding e (dead_input: e is read only by the RMSNorm) or input x (kept alive as
    the plan input) -> RMSNorm u -> decode token shift s."""
    g = wavec.WaveGraph(kv_cache_max_seq=0, fold_rmsnorm_gamma=False)
    if dead_input:
        table = (np.random.default_rng(rf).standard_normal((50, D)) * 2).astype(np.float16)
        g.add_input("tok", 1, 1, req, is_1d=True)
        g.add_embedding("emb", "tok", "x", table)
    else:
        table = None
        g.add_input("x", D, 1, req, is_1d=True)
    g.add_rmsnorm("n", "x", "u", D, gamma)
    g.add_token_shift("ts", "u", "s", mu, 1, decode=True)
    g.set_output("s")
    return g, table


@pytest.mark.parametrize("D,rf,seq_len,dead_input", [(2048, 4, 512, False), (256, 1, 128, False),
                                                     (2048, 2, 256, False), (1024, 5, 128, False),
                                                     (2048, 4, 512, True)])
def test_fused_prefill_norm_shift(wavec, tuning, D, rf, seq_len, dead_input):
    """Prefill RMSNorm -> token shift over 8,192 tokens (the register-resident norm's size): run
    as one kernel (each 32-token workgroup also normalizes the tokens before its block) unless
    the norm's input dies at the norm and the allocator hands its range to an output.  Norm
    output, shift output and state block bit for bit equal to the plan with fusion off, and
    within tolerance of the oracle."""
    T = 8192
    rng = np.random.default_rng(D + rf + seq_len)
    mu = (rng.standard_normal((D, rf)) * 0.5).astype(np.float16)
    gamma = rng.uniform(0.5, 1.5, D).astype(np.float32)
    table = (rng.standard_normal((50, D)) * 2).astype(np.float16)
    ids = rng.integers(0, 50, T).astype(np.uint32)
    x_in = (rng.standard_normal((D, T)) * 2).astype(np.float16)
    outs = {}
    for mode in ("fused", "unfused"):
        tuning("fuse", 0 if mode == "unfused" else -1)
        g = wavec.WaveGraph(kv_cache_max_seq=0, fold_rmsnorm_gamma=False)
        if dead_input:
            g.add_input("tok", 1, 1, T, is_1d=True)
            g.add_embedding("emb", "tok", "x", table)
        else:
            g.add_input("x", D, 1, T, is_1d=True)
        g.add_rmsnorm("n", "x", "u", D, gamma)
        g.add_token_shift("ts", "u", "s", mu, seq_len, decode=False)
        g.set_output("s")
        plan = g.compile()
        plan.init_gpu()
        n_cmd, s_cmd = plan.cmds[-2], plan.cmds[-1]
        fused = [a["name"] for a in plan.exec_report()["aux"] if a["fused"]]
        rd = {int(n_cmd["src_off"])}
        clash = int(s_cmd["y_off"]) in rd or int(n_cmd["y_off"]) in rd
        _log(f"[prefill norm+shift D={D} rf={rf} seq={seq_len} dead={dead_input} {mode}] "
             f"fused {fused}, output reuses the norm input: {clash}")
        assert bool(fused) == (mode == "fused" and not clash)
        if dead_input:
            plan.set_ids(ids)
            x = lo.embed(table, ids, T)
        else:
            x = x_in
            plan.write_canvas(int(n_cmd["src_off"]), x)
        plan.execute(1)
        u = _read(plan, n_cmd["y_off"], D, T)
        sh = _read(plan, s_cmd["y_off"], D, T)
        has_state = rf > 1
        st = (_read(plan, s_cmd["state_off"], D * (rf - 1), 64).reshape(D, rf - 1, 64)
              if has_state else None)
        u_ref = lo.rmsnorm_f64(x, gamma.astype(np.float16))
        assert lo.orc.rel_err(u.astype(np.float64), u_ref) <= TOL
        s_ref, st_ref = lo.token_shift(u, mu, seq_len, T, f64=True)
        assert lo.orc.rel_err(sh.astype(np.float64), s_ref) <= TOL
        if st is not None:
            assert np.array_equal(st.view(np.uint16), st_ref.view(np.uint16))
        outs[mode] = (u.copy(), sh.copy(), None if st is None else st.copy())
        plan.release_gpu()
    for a, b in zip(outs["fused"], outs["unfused"]):
        if a is not None:
            assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


@pytest.mark.parametrize("dead_input", [False, True])
@pytest.mark.parametrize("rf", [1, 2, 5, 9])
def test_fused_norm_shift_every_rf(wavec, tuning, rf, dead_input):
    """Decode RMSNorm -> token shift for receptive fields 1, 2, 5 and 9.  With the norm's input
    alive after it (the plan input) the two run as one kernel; with an input that dies at the
    norm, the canvas allocator gives its range to the shift output and the executor must keep
    two launches (one fused kernel would overwrite rows other workgroups still sum).  Either
    way: outputs and state bit for bit equal to the plan with fusion off, and within tolerance
    of the oracle, over two steps."""
    D, req = 2048, 16
    rng = np.random.default_rng(100 + rf)
    mu = (rng.standard_normal((D, rf)) * 0.5).astype(np.float16)
    gamma = rng.uniform(0.5, 1.5, D).astype(np.float32)
    outs = {}
    for mode in ("fused", "unfused"):
        tuning("fuse", 0 if mode == "unfused" else -1)
        g, table = _norm_shift_graph(wavec, D, req, rf, mu, gamma, dead_input)
        plan = g.compile()
        plan.init_gpu()
        n_cmd, s_cmd = plan.cmds[-2], plan.cmds[-1]
        fused = [a for a in plan.exec_report()["aux"] if a["fused"]]
        overlap = int(s_cmd["y_off"]) == int(n_cmd["src_off"])
        _log(f"[norm+shift rf={rf} dead_input={dead_input} {mode}] shift output reuses the "
             f"norm input: {overlap}; fused: {[a['name'] for a in fused]}")
        if dead_input:
            assert overlap  # the allocator case the executor must not fuse
        assert bool(fused) == (mode == "fused" and not overlap)
        rng2 = np.random.default_rng(7)
        state = np.zeros((D, max(rf - 1, 0), 64), np.float16)
        if rf > 1:
            state = rng2.standard_normal(state.shape).astype(np.float16)
            plan.write_canvas(int(s_cmd["state_off"]), state.reshape(D * (rf - 1), 64))
        res = []
        for step in range(2):
            if dead_input:
                ids = rng2.integers(0, 50, req).astype(np.uint32)
                plan.set_ids(ids)
                x = lo.embed(table, ids, 64)
            else:
                x = np.zeros((D, 64), np.float16)
                x[:, :req] = rng2.standard_normal((D, req)).astype(np.float16)
                plan.write_canvas(int(n_cmd["src_off"]), x)
            plan.execute(1)
            u = _read(plan, n_cmd["y_off"], D, 64)
            s = _read(plan, s_cmd["y_off"], D, 64)
            st = (_read(plan, s_cmd["state_off"], D * (rf - 1), 64).reshape(D, rf - 1, 64)
                  if rf > 1 else None)
            u_ref = lo.rmsnorm_f64(x, gamma.astype(np.float16))
            assert lo.orc.rel_err(u[:, :req].astype(np.float64), u_ref[:, :req]) <= TOL
            s_ref, state = lo.token_shift_decode(u, mu, state, req, f64=True)
            assert lo.orc.rel_err(s[:, :req].astype(np.float64), s_ref[:, :req]) <= TOL
            if rf > 1:
                assert np.array_equal(st[:, :, :req].view(np.uint16),
                                      state[:, :, :req].view(np.uint16))
            res.append((u[:, :req].copy(), s[:, :req].copy(), None if st is None else st.copy()))
        outs[mode] = res
    for (ua, sa, ta), (ub, sb, tb) in zip(outs["fused"], outs["unfused"]):
        assert np.array_equal(ua.view(np.uint16), ub.view(np.uint16))
        assert np.array_equal(sa.view(np.uint16), sb.view(np.uint16))
        if ta is not None:
            assert np.array_equal(ta.view(np.uint16), tb.view(np.uint16))


@pytest.mark.parametrize("V,stride,tokens", [(32000, 64, 16), (1000, 128, 100), (300, 1024, 1000)])
def test_standalone_argmax_on_device_buffers(wavec, V, stride, tokens):
    """wavec_argmax_f16 (the decode argmax on caller-owned device memory, partials in a
    stream-ordered workspace) against the lowest-index rule, with planted ties."""
    rng = np.random.default_rng(V + tokens)
    x = (rng.standard_normal((V, stride)) * 3).astype(np.float16)
    for t in range(0, tokens, 5):
        cs = np.sort(rng.choice(V, size=2, replace=False))
        x[cs, t] = np.float16(30.0)
    X = wavec.DeviceBuffer.from_array(x)
    ids = wavec.DeviceBuffer(tokens * 4)
    wavec.argmax_f16(ids, X, V, stride, tokens)
    wavec.device_synchronize()
    got = ids.download(np.uint32, tokens)
    assert np.array_equal(got, lo.argmax(x, tokens))


@pytest.mark.parametrize("V,stride,tokens", [(32000, 64, 16), (1000, 128, 100)])
def test_standalone_argmax_unaligned_logits(wavec, V, stride, tokens):
    """Logits 8 bytes past a 16-byte boundary take the 8-byte-load pass: same ids (lowest
    index on ties) as for aligned logits."""
    rng = np.random.default_rng(V + 7 * tokens)
    x = (rng.standard_normal((V, stride)) * 3).astype(np.float16)
    for t in range(0, tokens, 3):
        cs = np.sort(rng.choice(V, size=3, replace=False))
        x[cs, t] = np.float16(25.0)
    padded = np.concatenate([np.zeros(4, np.float16), x.ravel()])  # 4 halves = 8 bytes
    X = wavec.DeviceBuffer.from_array(padded)
    ids = wavec.DeviceBuffer(tokens * 4)
    wavec.argmax_f16(ids, X.ptr + 8, V, stride, tokens)
    wavec.device_synchronize()
    got = ids.download(np.uint32, tokens)
    assert np.array_equal(got, lo.argmax(x, tokens))

"""Shared helpers for wave parity tests: run one sparse wave on the GPU and on the oracle."""
import numpy as np

from snntome_amd import synth

TOL = 2e-3  # north_star: max |d| / (|ref| + 1e-2) <= 2e-3 against the fp64 oracle
# Values of the executor tuning switch "path" (wavec.set_tuning).
PATH_IDS = {"auto": -1, "valu": 0, "mfma": 1}


def stride_of(tokens: int) -> int:
    return (tokens + 63) // 64 * 64


def run_sparse_case(wavec, orc, *, C, tokens, rows, weights, bias, cluster=1, act="relu",
                    residual=False, seed=11):
    """Compiles x[C, tokens] -> sparse wave(rows, weights) [-> residual x], runs it on the GPU,
    and returns (gpu [cout, stride] float64, oracle [cout, stride] float64, plan)."""
    cout = weights.shape[0]
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", C, 1, tokens, is_1d=True)
    g.add_sparse_wave("w0", "x", "y", rows, weights, bias, cluster=cluster, act=act,
                      res_blob="x" if residual else None)
    plan = g.compile()
    plan.init_gpu()
    plan.fill_input_uniform(seed)
    plan.execute(1)
    canvas = plan.read_canvas(0, int(plan.summary["canvas_elems"]))
    cmd = plan.cmds[0]
    st = stride_of(tokens)
    x0 = int(cmd["src_off"])
    # Device fill == host generator (bit exact), and untouched beyond the input tensor.
    x_host = synth.substrate_rows(seed, np.arange(C), st, valid=tokens).view(np.uint16)
    assert np.array_equal(canvas[x0:x0 + C * st].reshape(C, st), x_host)
    fan = rows.shape[1]
    seg = (x0 + rows.astype(np.uint64) * st).reshape(-1)
    ref = orc.wave_f64(canvas, seg, weights, bias, None, fan, 1, cluster, st, st, st, act,
                       res_off=x0 if residual else None)
    y0 = int(cmd["y_off"])
    y = canvas[y0:y0 + cout * st].view(np.float16).reshape(cout, st).astype(np.float64)
    return y, ref, plan


def random_rows(rng, n_rows, fan, C):
    return rng.integers(0, C, size=(n_rows, fan), dtype=np.int64).astype(np.uint32)


def cluster_rows(starts: np.ndarray, S: int) -> np.ndarray:
    """[rows, K] segment starts -> [rows, K*S] per-synapse positions."""
    r, K = starts.shape
    return (starts[:, :, None].astype(np.int64) + np.arange(S)[None, None, :]).reshape(
        r, K * S).astype(np.uint32)


def sampled_parity(orc, plan, wl, wave_idx, neurons, read_out=True):
    """Oracle check of selected neurons of a workload wave whose input is the plan input 'x'
    filled on the device with wl.seed: the oracle gathers from a compact host copy of exactly
    the substrate rows those neurons read (host generator), the GPU rows are read back."""
    w = wl.waves[wave_idx]
    st = stride_of(wl.tokens)
    neurons = np.asarray(neurons, dtype=np.int64)
    rows = np.unique(neurons // w.cluster)
    starts = w.starts[rows].astype(np.uint64)  # [len(rows), K]
    compact = orc.fill_segments(wl.seed, starts.ravel(), w.S, wl.tokens, st)
    # row r of `rows` -> its K segments are consecutive blocks of S rows in `compact`
    seg = (np.arange(rows.size * w.K, dtype=np.uint64) * w.S * st)
    remap = {int(r): i for i, r in enumerate(rows)}
    sel_local = np.array([remap[int(j // w.cluster)] * w.cluster + int(j % w.cluster)
                          for j in neurons], dtype=np.uint32)
    # weights / bias of the selected rows' neurons, in local order
    wl_idx = np.concatenate([np.arange(r * w.cluster, (r + 1) * w.cluster) for r in rows])
    ref = orc.wave_f64(compact.ravel(), seg, w.weights[wl_idx], w.bias[wl_idx], None, w.K, w.S,
                       w.cluster, st, st, st, w.act, sel=sel_local)
    if not read_out:
        return None, ref
    cmd = plan.cmds[wave_idx]
    y0 = int(cmd["y_off"])
    ys = np.stack([plan.read_canvas(y0 + int(j) * st, st) for j in neurons])
    y = ys.view(np.float16).astype(np.float64)
    return y, ref

"""Pure-Python restatement of the wave-plan compiler and the TCFF v1.0 writer —
TEST INFRASTRUCTURE ONLY (used by tests/ to check libk44wavec.so's plans and .tcff bytes).

Scope: 1-D token graphs — Input, linear (1x1 Convolution), the build's sparse waves,
Concat / Split / Slice views, RMSNorm / SwiGLU nodes (they take canvas space) — and 2-D image
graphs of up to 63 frames — kxk Convolution (stride 1 and the stride-2 polyphase form with its
S2D scratch), max-pooling, 2x upsampling, 2x2 transposed convolution (quadrant wave + scratch),
views.  Restated from the reference's documented behaviour:
  res descriptors        wavec/k44_plan_types.hpp:491-516 (1-D mode), :517-569 (2-D modes)
  tap offsets            wavec/k44_plan_types.hpp:593-600
  2-D shapes, layouts    wavec/k44_wave_compiler.hpp:137-210, 315-366
  conv / deconv waves    wavec/k44_wave_compiler.hpp:609-807
  cluster size           wavec/k44_plan_types.hpp:157-186, 328-343
  WMMA weight order      wavec/k44_plan_types.hpp:363-375
  passes 1, 3, 4, 5      wavec/k44_wave_compiler.hpp:78-223, 315-366, 388-593, 824-988
  dense 1-D waves        wavec/k44_wave_compiler.hpp:692-807
  pack_wave_buffers      wavec/k44_wave_compiler.hpp:1031-1076
  .tcff writer           wavec/k44_tcff_io.hpp:100-300
The sparse-wave emission and the 0x8445 extension tag follow this build's specification
(include/k44wavec.h, snntome_amd/csrc/k44_tcff_io.hpp).
"""
import math
import struct

import numpy as np

from .cnn_oracle import Layout2D

ACT_NAMES = ["NONE", "RELU", "SIGMOID", "SILU", "LEAKY_RELU", "GELU"]


def fnv1a64(data: bytes) -> int:
    h = 0xCBF29CE484222325
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def fnv1a64_np(data: bytes) -> int:
    # Same function, chunked through python ints for large blocks (speed only).
    return fnv1a64(data)


def round_up_16(v):
    return max(16, (v + 15) & ~15)


def round_up_32(v):
    return max(64, (v + 31) & ~31)


def choose_cluster_size(cout, num_tiles, force=0):
    s = force
    while s >= 16:
        if cout % s == 0:
            return s
        s >>= 1
    if cout % 128 == 0 and (cout >= 640 or num_tiles <= 64):
        return 128
    if cout % 64 == 0:
        return 64
    if cout % 32 == 0:
        return 32
    return 16


def res_key_1d(w):
    return 0x80000000 | w


def res_key(h, w, is_1d):
    """Layout key of a tensor shape (k44_wave_compiler.hpp:26-29)."""
    if is_1d:
        return res_key_1d(w)
    return h if h == w else (((h << 14) ^ w) & 0xFFFFFFFF)


def tiles_per_frame_2d(L) -> int:
    """64-element tiles of one frame of a 2-D layout (k44_plan_types.hpp:517-569)."""
    if L.aligned:
        return L.H * (L.W // 64)
    return (L.H * L.W_pad + 63) // 64


def tap_2d(L, base, dy, dx):
    """Gather index of tap (dy, dx) of the channel based at `base` (k44_plan_types.hpp:593-600,
    non-token64 2-D mode: h_tile_off_X is anchored one row and one column before the tile)."""
    return base + (1 + dy) * L.W_pad + (1 + dx)


class Layout1D:
    def __init__(self, w):
        self.W = w
        self.tiles = (w + 63) // 64
        self.channel_stride = self.tiles * 64
        self.W_pad = self.channel_stride
        self.num_tiles = self.tiles


def to_wmma(w_rows: np.ndarray) -> np.ndarray:
    """[Cout][B] fp16 bits -> WMMA block order (flat uint16)."""
    cout, B = w_rows.shape
    out = np.empty(cout * B, dtype=np.uint16)
    g = 0
    for rb in range(cout // 16):
        for kb in range(B // 16):
            for l in range(32):
                r = 16 * rb + (l & 15)
                c = 16 * kb + 8 * (l >> 4)
                out[8 * g:8 * g + 8] = w_rows[r, c:c + 8]
                g += 1
    return out


class Node:
    def __init__(self, op, name, ins=(), outs=(), **kw):
        self.op, self.name = op, name
        self.ins, self.outs = list(ins), list(outs)
        self.cin = kw.get("cin", 0)
        self.cout = kw.get("cout", 0)
        self.h_in = self.w_in = self.h_out = self.w_out = 0
        self.is_1d = kw.get("is_1d", False)
        self.act = kw.get("act", 0)
        self.residual = kw.get("residual", "")
        self.weights = kw.get("weights")  # fp16 bits [cout][fan]
        self.bias = kw.get("bias")  # fp16 bits [cout]
        self.rows = kw.get("rows")  # sparse: [cout/cluster][fan] channel ids
        self.cluster = kw.get("cluster", 1)
        self.seg_len = kw.get("seg_len", 0)
        self.slice_sizes = kw.get("slice_sizes", [])
        self.kh = kw.get("kh", 1)
        self.kw = kw.get("kw", 1)
        self.stride = kw.get("stride", 1)


class Graph:
    def __init__(self, force_cluster_size=0, batch_size=1):
        self.nodes = []
        self.output = "out0"
        self.force = force_cluster_size
        self.batch = batch_size

    def _add(self, n, set_out=True):
        if set_out and n.outs:
            self.output = n.outs[0]
        self.nodes.append(n)

    def input(self, name, c, h, w, is_1d):
        n = Node("Input", name, outs=[name], cin=c, cout=c)
        n.h_in = n.h_out = h
        n.w_in = n.w_out = w
        n.is_1d = is_1d or (h == 1 and (w < 4 or w % 4 != 0))
        self._add(n)

    def linear(self, name, i, o, din, dout, w_bits, b_bits, act=0, residual=""):
        self._add(Node("Convolution", name, [i], [o], cin=din, cout=dout, weights=w_bits,
                       bias=b_bits, act=act, residual=residual))

    def sparse(self, name, i, o, rows, w_bits, b_bits, cluster=1, act=0, residual="",
               seg_len=0):
        cout = w_bits.shape[0]
        self._add(Node("SparseWave", name, [i], [o], cout=cout, weights=w_bits, bias=b_bits,
                       rows=rows, cluster=cluster, act=act, residual=residual,
                       seg_len=seg_len))

    def pruned(self, name, i, o, starts, S, w_bits, b_bits, tile=64, act=0, residual=""):
        """Per-neuron clusters starts [cout][K] of S channels; compiled by pruned_parts."""
        self._add(Node("PrunedWave", name, [i], [o], cout=w_bits.shape[0], weights=w_bits,
                       bias=b_bits, rows=np.asarray(starts), cluster=tile, act=act,
                       residual=residual, seg_len=S))

    def conv2d(self, name, i, o, cin, cout, kh, kw, stride, w_bits, b_bits, act=0, residual=""):
        """w_bits: [cout][cin*kh*kw] fp16 bits (synapse ch*kh*kw + ky*kw + kx)."""
        self._add(Node("Convolution", name, [i], [o], cin=cin, cout=cout, weights=w_bits,
                       bias=b_bits, act=act, residual=residual, kh=kh, kw=kw, stride=stride))

    def maxpool(self, name, i, o, k, stride):
        self._add(Node("Pooling", name, [i], [o], kh=k, kw=k, stride=stride))

    def upsample2x(self, name, i, o):
        self._add(Node("Interp", name, [i], [o]))

    def upconv2x2(self, name, i, o, cin, cout, w_bits, b_bits):
        """w_bits: [cout][cin][4] fp16 bits (quadrant 2*ky + kx)."""
        self._add(Node("Deconvolution", name, [i], [o], cin=cin, cout=cout, weights=w_bits,
                       bias=b_bits, kh=2, kw=2, stride=2))

    def concat(self, name, ins, o):
        self._add(Node("Concat", name, ins, [o]))

    def split(self, name, i, outs):
        self._add(Node("Split", name, [i], outs), set_out=False)

    def slice(self, name, i, outs, sizes):
        self._add(Node("Slice", name, [i], outs, slice_sizes=list(sizes)), set_out=False)

    def rmsnorm(self, name, i, o, dim):
        self._add(Node("RMSNorm", name, [i], [o], cin=dim, cout=dim))

    def swiglu(self, name, g, u, o):
        self._add(Node("SwiGLU", name, [g, u], [o]))


MAX_PACK_CLUSTERS = 12


def pack_union_tiles(pm, nu: int, T: int, max_iter: int):
    """Tiles of T neurons with small cluster unions (restatement of the build's
    k44_host::pack_union_tiles); pm[j] = neuron j's cluster set as a bit mask over nu <= 12
    distinct clusters.  Returns the tiles' neuron lists (each ascending), in creation order.

    1. Greedy, one tile at a time: among the masks containing at least `need` = min(T,
       unassigned) unassigned patterns (subset-sum transform of the pattern counts), take the one
       with the fewest clusters, then the most patterns, then the smallest mask value; of its
       unassigned neurons take the `need` that lie in the fewest other such masks (superset-sum
       transform), ties by index.
    2. Swaps: while the first tile W with the largest union can drop one of its clusters c —
       tried in order of (neurons of W using c, c) — by trading each of its neurons a that use c
       (ascending order of W's current list) for the first neuron b (tiles in order, each
       tile's current list in order) not yet traded, not using c, inside W's union, such that
       b's tile keeps a union below W's: trade them all (a goes to the end of b's tile's list,
       b to the end of W's) and repeat; at most max_iter rounds."""
    pm = np.asarray(pm, dtype=np.int64)
    n, NM = pm.size, 1 << nu
    idx = np.arange(NM)
    pop = np.array([bin(m).count("1") for m in range(NM)])
    left = np.ones(n, dtype=bool)
    tiles = []
    while left.any():
        need = min(T, int(left.sum()))
        cnt = np.bincount(pm[left], minlength=NM).astype(np.int64)
        for b in range(nu):  # cnt[m] = unassigned patterns inside m
            sel = (idx >> b) & 1 == 1
            cnt[sel] += cnt[idx[sel] ^ (1 << b)]
        ok = np.nonzero(cnt >= need)[0]
        best = int(ok[np.lexsort((ok, -cnt[ok], pop[ok]))[0]])
        v = ((cnt >= need) & (idx != best)).astype(np.int64)
        for b in range(nu):  # v[m] = other such masks containing m
            sel = (idx >> b) & 1 == 0
            v[sel] += v[idx[sel] | (1 << b)]
        mem = np.nonzero(left & ((pm & ~best) == 0))[0]
        take = np.sort(mem[np.argsort(v[pm[mem]], kind="stable")[:need]])
        left[take] = False
        tiles.append([int(j) for j in take])
    cc = np.zeros((len(tiles), nu), dtype=np.int64)  # per tile: neurons using each cluster
    bits = [[c for c in range(nu) if m >> c & 1] for m in range(NM)]
    for t, js in enumerate(tiles):
        for j in js:
            cc[t, bits[pm[j]]] += 1
    for _ in range(max_iter):
        sizes = (cc > 0).sum(axis=1)
        m = int(sizes.max())
        W = int(np.argmax(sizes))
        uw = sum(1 << c for c in range(nu) if cc[W, c])
        done = False
        for c in sorted((c for c in range(nu) if cc[W, c]), key=lambda c: (cc[W, c], c)):
            trades, used = [], set()
            for a in [j for j in tiles[W] if pm[j] >> c & 1]:
                hit = None
                for B in range(len(tiles)):
                    if B == W:
                        continue
                    for b in tiles[B]:
                        if b in used or pm[b] >> c & 1 or pm[b] & ~uw:
                            continue
                        after = cc[B].copy()
                        after[bits[pm[b]]] -= 1
                        after[bits[pm[a]]] += 1
                        if (after > 0).sum() <= m - 1:
                            hit = (B, b)
                            break
                    if hit:
                        break
                if hit is None:
                    break
                B, b = hit
                cc[B, bits[pm[b]]] -= 1
                cc[B, bits[pm[a]]] += 1
                cc[W, bits[pm[a]]] -= 1
                cc[W, bits[pm[b]]] += 1
                trades.append((a, B, b))
                used.add(b)
            else:
                for a, B, b in trades:
                    tiles[W].remove(a)
                    tiles[W].append(b)
                    tiles[B].remove(b)
                    tiles[B].append(a)
                done = True
                break
            for a, B, b in reversed(trades):  # this cluster cannot go: undo
                cc[B, bits[pm[b]]] += 1
                cc[B, bits[pm[a]]] -= 1
                cc[W, bits[pm[a]]] += 1
                cc[W, bits[pm[b]]] -= 1
        if not done:
            break
    return [sorted(t) for t in tiles]


def pruned_parts(starts: np.ndarray, S: int, w: np.ndarray, bias: np.ndarray, tile: int):
    """Tiles of a pruned projection (restatement of the build's
    K44WaveGraphCompiler::add_pruned_wave).  Pattern-sorted cutting: neurons grouped by their
    sorted cluster pattern (groups in lexicographic order), full tiles per group, the groups'
    remainders packed in order.  With at most 12 distinct clusters over all neurons,
    pack_union_tiles too, and its tiles replace the cutting's unless they have a larger largest
    union (or the same largest and a larger total).  A tile's index row is the union of its
    neurons' clusters; one part per union size (ascending).  Returns [(union starts [tiles][U], weights [tiles*tile][U*S] u16,
    bias [tiles*tile] u16, cmap [tiles*tile] u16 (0xFFFF = empty))]."""
    cout, K = starts.shape
    order = np.argsort(starts, axis=1, kind="stable")
    pat = np.take_along_axis(starts, order, axis=1)
    univ = sorted({int(v) for v in pat.ravel()})
    # pattern-sorted cutting: full tiles per pattern group, then the groups' remainders
    groups = {}
    for j in range(cout):
        groups.setdefault(tuple(int(v) for v in pat[j]), []).append(j)
    cut, rest = [], []
    for key in sorted(groups):
        g = groups[key]
        full = len(g) // tile
        for f in range(full):
            cut.append(g[f * tile:(f + 1) * tile])
        rest += g[full * tile:]
    for b in range(0, len(rest), tile):
        cut.append(rest[b:b + tile])
    chosen = cut
    if len(univ) <= MAX_PACK_CLUSTERS:
        pos = {u: i for i, u in enumerate(univ)}
        pm = [sum(1 << pos[int(v)] for v in pat[j]) for j in range(cout)]
        packed = pack_union_tiles(pm, len(univ), tile, 4 * (-(-cout // tile)) + 64)

        def cost(ts):  # (largest union, total of unions)
            us = [bin(int(np.bitwise_or.reduce([pm[j] for j in t]))).count("1") for t in ts]
            return max(us), sum(us)

        if cost(packed) <= cost(cut):
            chosen = packed
    tiles = []
    for js in chosen:
        uni = sorted({int(v) for j in js for v in pat[j]})
        tiles.append((list(js) + [-1] * (tile - len(js)), uni))
    parts = []
    for U in sorted({len(t[1]) for t in tiles}):
        sel = [t for t in tiles if len(t[1]) == U]
        rows = np.array([t[1] for t in sel], dtype=np.uint32)
        wp = np.zeros((len(sel) * tile, U * S), dtype=np.uint16)
        bp = np.zeros(len(sel) * tile, dtype=np.uint16)
        cm = np.full(len(sel) * tile, 0xFFFF, dtype=np.uint16)
        for ti, (slots, uni) in enumerate(sel):
            for q, j in enumerate(slots):
                if j < 0:
                    continue
                r = ti * tile + q
                cm[r], bp[r] = j, bias[j]
                for k, u in enumerate(uni):
                    hit = np.nonzero(starts[j] == u)[0]
                    if hit.size:
                        src = int(hit[0])
                        wp[r, k * S:(k + 1) * S] = w[j, src * S:(src + 1) * S]
        parts.append((rows, wp, bp, cm))
    return parts


def compile_plan(g: Graph) -> dict:
    nodes = g.nodes
    graph_1d = bool(nodes) and nodes[0].op == "Input" and nodes[0].is_1d
    if graph_1d and g.batch > 1 and nodes[0].w_out == 1:
        nodes[0].w_in = nodes[0].w_out = g.batch
    shapes = {}  # tensor -> (c, h, w, is_1d)
    for n in nodes:  # pass 1
        if n.op == "Input":
            shapes[n.outs[0]] = (n.cout, n.h_out, n.w_out, n.is_1d)
            plan_in = (n.cout, n.h_out, n.w_out)
        elif n.op in ("Convolution", "SparseWave", "PrunedWave"):
            c, h, w, d = shapes[n.ins[0]]
            if n.op in ("SparseWave", "PrunedWave"):
                assert d, "sparse waves take 1-D token inputs"
                n.cin = c
            elif not d and n.kh == 1 and n.kw == 1 and n.cin == c * h * w and n.cin != c:
                raise NotImplementedError("implicit flatten of a 2-D tensor")
            n.is_1d = d
            n.h_in, n.w_in = h, w
            n.h_out, n.w_out = (1, w) if d else (h // n.stride, w // n.stride)
            shapes[n.outs[0]] = (n.cout, n.h_out, n.w_out, d)
        elif n.op == "Deconvolution":
            c, h, w, d = shapes[n.ins[0]]
            n.h_in, n.w_in, n.h_out, n.w_out = h, w, 2 * h, 2 * w
            shapes[n.outs[0]] = (n.cout, n.h_out, n.w_out, False)
        elif n.op in ("Pooling", "Interp"):
            c, h, w, d = shapes[n.ins[0]]
            n.cin = n.cout = c
            n.h_in, n.w_in = h, w
            n.h_out, n.w_out = (h // n.stride, w // n.stride) if n.op == "Pooling" else (2 * h, 2 * w)
            shapes[n.outs[0]] = (c, n.h_out, n.w_out, False)
        elif n.op == "Concat":
            c0, h, w, d = shapes[n.ins[0]]
            n.is_1d = d
            shapes[n.outs[0]] = (sum(shapes[t][0] for t in n.ins), h, w, d)
        elif n.op == "Split":
            for o in n.outs:
                shapes[o] = shapes[n.ins[0]]
        elif n.op == "Slice":
            c, h, w, d = shapes[n.ins[0]]
            for k, o in enumerate(n.outs):
                cc = n.slice_sizes[k] if n.slice_sizes else c // len(n.outs)
                shapes[o] = (cc, h, w, d)
        elif n.op in ("RMSNorm", "SwiGLU"):
            c, h, w, d = shapes[n.ins[0]]
            n.is_1d = d
            n.h_in = n.h_out = h
            n.w_in = n.w_out = w
            if n.op == "SwiGLU":
                n.cin = n.cout = c
            shapes[n.outs[0]] = (c, h, w, d)
    # pass 3: one layout per shape key (frames per wave: 1 for token graphs, else <= 8); configs
    if not graph_1d:
        assert g.batch < 64, "the 64-frame interleaved image layout is not restated"
    frames = 1 if graph_1d else min(max(1, g.batch), 8)
    res = {}
    for t in sorted(shapes):
        c, h, w, d = shapes[t]
        if res_key(h, w, d) not in res:
            res[res_key(h, w, d)] = Layout1D(w) if d else Layout2D(h, w, frames)
    cfg = {}
    for i, n in enumerate(nodes):
        if n.op == "Convolution":
            cp = round_up_16(n.cout)
            if n.is_1d:
                tiles = max(1, res[res_key_1d(n.w_out)].num_tiles)
            else:
                tiles = max(1, n.h_out * n.w_out)
            cfg[i] = (choose_cluster_size(cp, tiles, g.force), cp)
        elif n.op == "SparseWave":
            lcm = 16 * n.cluster // math.gcd(16, n.cluster)
            cfg[i] = (n.cluster, (n.cout + lcm - 1) // lcm * lcm)

    def out_key(n):
        d = n.is_1d if n.op not in ("Deconvolution", "Pooling", "Interp") else False
        return res_key(n.h_out, n.w_out, d)

    # pass 4: allocation ids, liveness, best-fit placement, then the S2D / quadrant scratch
    ids, allocs, out_aid = {}, {}, {}
    nxt = 0
    for i, n in enumerate(nodes):
        if n.op in ("Split", "Slice"):
            for o in n.outs:
                ids[o] = set(ids[n.ins[0]])
        elif n.op == "Concat":
            ids[n.outs[0]] = set().union(*[ids[t] for t in n.ins])
        else:
            ch = cfg[i][1] if n.op in ("Convolution", "SparseWave") else n.cout
            allocs[nxt] = [out_key(n), ch, 0]
            ids[n.outs[0]] = {nxt}
            out_aid[i] = nxt
            nxt += 1
    last = {0: len(nodes)}
    for a in ids.get(g.output, ()):
        last[a] = len(nodes)
    for i, n in enumerate(nodes):
        for t in n.ins + ([n.residual] if n.residual else []):
            for a in ids.get(t, ()):
                last[a] = max(last.get(a, 0), i)
    s2d_ch, quad_ch = {}, {}
    for n in nodes:
        if n.op == "Convolution" and n.stride == 2 and not n.is_1d:
            k = res_key(n.h_out, n.w_out, False)
            s2d_ch[k] = max(s2d_ch.get(k, 0), 4 * n.cin)
        elif n.op == "Deconvolution":
            k = res_key(n.h_in, n.w_in, False)
            quad_ch[k] = max(quad_ch.get(k, 0), 4 * round_up_16(n.cout))
    free, peak, placed, live = [], 0, {}, []
    for i, n in enumerate(nodes):
        if i in out_aid:
            a = out_aid[i]
            key, ch, _ = allocs[a]
            need = (ch * res[key].channel_stride + 63) // 64 * 64
            fits = [k for k, f in enumerate(free) if f[1] >= need]
            if fits:
                k = min(fits, key=lambda q: (free[q][1], q))
                at = free[k][0]
                if free[k][1] == need:
                    free.pop(k)
                else:
                    free[k] = (free[k][0] + need, free[k][1] - need)
            elif free and free[-1][0] + free[-1][1] == peak:
                at = free.pop()[0]
                peak = at + need
            else:
                at = peak
                peak += need
            placed[a] = (at, need)
            allocs[a][2] = at
            live.append(a)
        gone = sorted(a for a in live if last.get(a, 0) <= i)
        for a in gone:
            live.remove(a)
            free.append(placed[a])
        if gone and len(free) > 1:
            free.sort()
            merged = []
            for f in free:
                if merged and merged[-1][0] + merged[-1][1] == f[0]:
                    merged[-1] = (merged[-1][0], merged[-1][1] + f[1])
                else:
                    merged.append(f)
            free = merged
    cur = (peak + 63) // 64 * 64
    s2d_base = {k: cur for k in s2d_ch}
    cur += (max([s2d_ch[k] * res[k].channel_stride for k in s2d_ch], default=0) + 63) // 64 * 64
    quad_base = {k: cur for k in quad_ch}
    cur += (max([quad_ch[k] * res[k].channel_stride for k in quad_ch], default=0) + 63) // 64 * 64
    canvas = (cur + 127) // 128 * 128 or 128
    plan = {"canvas_elems": canvas, "input_off": allocs[0][2], "cmds": [], "res": res,
            "total_w_bytes": 0, "total_idx_bytes": 0, "input": plan_in}

    def geom_1d(c, Lo):
        toks = max(1, c["w_out"])
        return [2 if toks > 1 else 1, toks, c["logical_Cout"], 1, 1, 1, Lo.channel_stride, 1, 1, 0]

    def geom_2d(c, Lo):
        return [3, 1, c["logical_Cout"], c["h_out"], c["w_out"], c["Cout"] * Lo.channel_stride,
                Lo.channel_stride, Lo.W_pad, 1, Lo.W_pad + 4]

    # pass 5
    chan = {}
    for i, n in enumerate(nodes):
        if n.op == "Input":
            key, ch, at = allocs[out_aid[i]]
            chan[n.outs[0]] = [at + c * res[key].channel_stride for c in range(n.cout)]
        elif n.op == "Split":
            for o in n.outs:
                chan[o] = list(chan[n.ins[0]])
        elif n.op == "Slice":
            src, at = chan[n.ins[0]], 0
            for k, o in enumerate(n.outs):
                ln = n.slice_sizes[k] if n.slice_sizes else len(src) // len(n.outs)
                chan[o] = src[at:at + ln]
                at += ln
        elif n.op == "Concat":
            chan[n.outs[0]] = [x for t in n.ins for x in chan[t]]
        elif n.op in ("RMSNorm", "SwiGLU", "Pooling", "Interp"):
            key, ch, at = allocs[out_aid[i]]
            chan[n.outs[0]] = [at + c * res[key].channel_stride for c in range(n.cout)]
            plan["cmds"].append({"type": {"RMSNorm": 7, "SwiGLU": 8, "Pooling": 3,
                                          "Interp": 4}[n.op], "name": n.name})
        elif n.op == "Deconvolution":
            key, ch, dst = allocs[out_aid[i]]
            chan[n.outs[0]] = [dst + c * res[key].channel_stride for c in range(n.cout)]
            kin = res_key(n.h_in, n.w_in, False)
            Li = res[kin]
            in_chs = chan[n.ins[0]]
            cal = round_up_16(n.cout)
            cq = 4 * cal
            cl = choose_cluster_size(cq, tiles_per_frame_2d(Li), g.force)
            B = round_up_32(n.cin)
            idx = np.zeros((cq // cl, B), dtype=np.uint64)
            idx[:, :n.cin] = np.asarray([tap_2d(Li, in_chs[c], 0, 0) for c in range(n.cin)],
                                        dtype=np.uint64)[None, :]
            w = np.zeros((cq, B), dtype=np.uint16)
            bias = np.zeros(cq, dtype=np.uint16)
            wq = np.asarray(n.weights).reshape(n.cout, n.cin, 4)
            for q in range(4):
                w[q * cal:q * cal + n.cout, :n.cin] = wq[:, :, q]
                bias[q * cal:q * cal + n.cout] = n.bias[:n.cout]
            cmd = {"type": 0, "name": n.name, "Cin": n.cin, "Cout": cq, "logical_Cout": 4 * n.cout,
                   "cluster": cl, "B": B, "B_raw": n.cin, "act": 0, "has_res": False,
                   "h_out": n.h_in, "w_out": n.w_in, "src_off": 0, "y_off": quad_base[kin],
                   "res_off": 0, "x_base_off": 0, "idx_mode": 0, "idx_stride": 1,
                   "seg_len": 0, "idx": idx.astype(np.uint32), "w_rows": w, "bias": bias,
                   "out_stride": Li.channel_stride}
            cmd["geom"] = geom_2d(cmd, Li)
            plan["total_w_bytes"] += cq * B * 2
            plan["total_idx_bytes"] += idx.size * 4 + cq * 2
            plan["cmds"].append(cmd)
            plan["cmds"].append({"type": 6, "name": n.name + "_scatter2x2"})
        elif n.op == "Convolution" and not n.is_1d:
            key, ch, dst = allocs[out_aid[i]]
            Lo = res[key]
            chan[n.outs[0]] = [dst + c * Lo.channel_stride for c in range(n.cout)]
            in_chs = chan[n.ins[0]]
            S_cl, cout_pad = cfg[i]
            has_res = bool(n.residual)
            res_off = chan[n.residual][0] if has_res else 0
            if has_res:
                end = res_off + cout_pad * Lo.channel_stride
                if end > plan["canvas_elems"]:
                    plan["canvas_elems"] = (end + 127) // 128 * 128
            taps = n.kh * n.kw
            b_raw = taps * n.cin
            B = round_up_32(b_raw)
            poly = n.stride == 2
            if poly:
                s2d = s2d_base[key]
                plan["cmds"].append({"type": 5, "name": n.name + "_s2d_2x2"})
            row = np.zeros(b_raw, dtype=np.uint64)
            for c in range(n.cin):
                for ky in range(n.kh):
                    for kx in range(n.kw):
                        if poly:  # stride 2 = stride-1 taps over polyphase channel 4c+2py+px
                            dy, py = (-1, 1) if ky == 0 else (0, 0 if ky == 1 else 1)
                            dx, px = (-1, 1) if kx == 0 else (0, 0 if kx == 1 else 1)
                            base = s2d + (4 * c + 2 * py + px) * Lo.channel_stride
                            v = tap_2d(Lo, base, dy, dx)
                        else:
                            v = tap_2d(Lo, in_chs[c], ky - n.kh // 2, kx - n.kw // 2)
                        row[c * taps + ky * n.kw + kx] = v
            idx = np.zeros((cout_pad // S_cl, B), dtype=np.uint64)
            idx[:, :b_raw] = row[None, :]
            log_c = min(cout_pad, n.cout)
            w = np.zeros((cout_pad, B), dtype=np.uint16)
            w[:log_c, :b_raw] = n.weights[:log_c]
            bias = np.zeros(cout_pad, dtype=np.uint16)
            bias[:log_c] = n.bias[:log_c]
            cmd = {"type": 0, "name": n.name, "Cin": n.cin, "Cout": cout_pad,
                   "logical_Cout": log_c, "cluster": S_cl, "B": B, "B_raw": b_raw,
                   "act": n.act, "has_res": has_res, "h_out": n.h_out, "w_out": n.w_out,
                   "src_off": s2d if poly else in_chs[0], "y_off": dst, "res_off": res_off,
                   "x_base_off": 0, "idx_mode": 0, "idx_stride": 1, "seg_len": 0,
                   "idx": idx.astype(np.uint32), "w_rows": w, "bias": bias,
                   "out_stride": Lo.channel_stride}
            assert int(idx.max()) < 0x70000000
            cmd["geom"] = geom_2d(cmd, Lo)
            plan["total_w_bytes"] += cout_pad * B * 2
            plan["total_idx_bytes"] += idx.size * 4 + cout_pad * 2
            plan["cmds"].append(cmd)
        elif n.op == "PrunedWave":
            key, ch, dst = allocs[out_aid[i]]
            Lo = res[key]
            chan[n.outs[0]] = [dst + c * Lo.channel_stride for c in range(n.cout)]
            in_chs = np.asarray(chan[n.ins[0]], dtype=np.uint64)
            has_res = bool(n.residual)
            res_off = chan[n.residual][0] if has_res else 0
            S = n.seg_len
            parts = pruned_parts(n.rows, S, n.weights, n.bias, n.cluster)
            for p, (rows_u, wp, bp, cm) in enumerate(parts):
                slots, U = wp.shape[0], rows_u.shape[1]
                b_raw = U * S
                B = round_up_32(b_raw)
                lcm = 16 * n.cluster // math.gcd(16, n.cluster)
                cout_pad = (slots + lcm - 1) // lcm * lcm
                syn = (rows_u[:, :, None].astype(np.int64) + np.arange(S)[None, None, :]).reshape(
                    rows_u.shape[0], b_raw)
                idx = np.zeros((cout_pad // n.cluster, B), dtype=np.uint64)
                idx[: syn.shape[0], :b_raw] = in_chs[syn]
                w = np.zeros((cout_pad, B), dtype=np.uint16)
                w[:slots, :b_raw] = wp
                bias = np.zeros(cout_pad, dtype=np.uint16)
                bias[:slots] = bp
                cmap = np.full(cout_pad, 0xFFFF, dtype=np.uint16)
                cmap[:slots] = cm
                x_base = 0
                real = idx[:, :b_raw]
                if int(real.max()) >= 0x70000000:
                    x_base = int(real.min()) & ~63
                    idx[:, :b_raw] -= np.uint64(x_base)
                    idx[:, b_raw:] = 0
                plan["total_w_bytes"] += cout_pad * B * 2
                plan["total_idx_bytes"] += idx.size * 4 + cout_pad * 2 + cout_pad * 2
                plan["cmds"].append({
                    "type": 0, "name": n.name if len(parts) == 1 else f"{n.name}/{p}",
                    "Cin": n.cin, "Cout": cout_pad, "logical_Cout": n.cout,
                    "cluster": n.cluster, "B": B, "B_raw": b_raw, "act": n.act,
                    "has_res": has_res, "h_out": 1, "w_out": n.w_out, "src_off": int(in_chs[0]),
                    "y_off": dst, "res_off": res_off, "x_base_off": x_base, "idx_mode": 0,
                    "idx_stride": 1, "seg_len": S, "idx": idx.astype(np.uint32), "w_rows": w,
                    "bias": bias, "cmap": cmap, "out_stride": Lo.channel_stride,
                })
        elif n.op in ("Convolution", "SparseWave"):
            key, ch, dst = allocs[out_aid[i]]
            Lo = res[key]
            chan[n.outs[0]] = [dst + c * Lo.channel_stride for c in range(n.cout)]
            in_chs = chan[n.ins[0]]
            S_cl, cout_pad = cfg[i]
            has_res = bool(n.residual)
            res_off = chan[n.residual][0] if has_res else 0
            if has_res:
                end = res_off + cout_pad * Lo.channel_stride
                if end > plan["canvas_elems"]:
                    plan["canvas_elems"] = (end + 127) // 128 * 128
            idx_mode, idx_stride = 0, 1
            if n.op == "Convolution":
                b_raw = n.cin
                B = round_up_32(b_raw)
                rows = cout_pad // S_cl
                row = [in_chs[c] for c in range(n.cin)]
                idx = np.zeros((rows, B), dtype=np.uint64)
                idx[:, :b_raw] = np.asarray(row, dtype=np.uint64)[None, :]
                log_c = min(cout_pad, n.cout)
                seg_len = n.cin
            else:
                b_raw = n.weights.shape[1]
                B = round_up_32(b_raw)
                rows = cout_pad // n.cluster
                offs = np.asarray(in_chs, dtype=np.uint64)[np.asarray(n.rows, dtype=np.int64)]
                idx = np.zeros((rows, B), dtype=np.uint64)
                if int(offs.max()) > 0xFFFFFFFF:
                    idx_mode, idx_stride = 1, res[res_key_1d(n.w_in)].channel_stride
                    idx[: n.rows.shape[0], :b_raw] = np.asarray(n.rows, dtype=np.uint64)
                else:
                    idx[: n.rows.shape[0], :b_raw] = offs
                log_c = n.cout
                seg_len = n.seg_len
            w = np.zeros((cout_pad, B), dtype=np.uint16)
            w[:log_c, :b_raw] = n.weights[:log_c]
            bias = np.zeros(cout_pad, dtype=np.uint16)
            bias[:log_c] = n.bias[:log_c]
            x_base = 0
            if idx_mode == 0:
                real = idx[:, :b_raw]
                if int(real.max()) >= 0x70000000:
                    x_base = int(real.min()) & ~63
                    idx[:, :b_raw] -= np.uint64(x_base)
                    idx[:, b_raw:] = 0
            else:
                x_base = in_chs[0]
            plan["total_w_bytes"] += cout_pad * B * 2
            plan["total_idx_bytes"] += idx.size * 4 + cout_pad * 2
            plan["cmds"].append({
                "type": 0, "name": n.name, "Cin": n.cin, "Cout": cout_pad, "logical_Cout": log_c,
                "cluster": S_cl, "B": B, "B_raw": b_raw, "act": n.act, "has_res": has_res,
                "h_out": 1, "w_out": n.w_out, "src_off": in_chs[0], "y_off": dst,
                "res_off": res_off, "x_base_off": x_base, "idx_mode": idx_mode,
                "idx_stride": idx_stride, "seg_len": seg_len,
                "idx": idx.astype(np.uint32), "w_rows": w, "bias": bias,
                "out_stride": Lo.channel_stride,
            })
    out_c, out_h, out_w, _ = shapes[g.output]
    plan["output"] = (out_c, out_h, out_w)
    plan["output_off"] = chan[g.output][0]
    return plan


def tcff_bytes(plan: dict, prefix="K44Model", include_geometry=True) -> bytes:
    waves = [c for c in plan["cmds"] if c["type"] == 0]
    A = 256
    buf = bytearray()

    def pad():
        buf.extend(b"\0" * ((-len(buf)) % A))

    buf += b"II" + struct.pack("<HI", 42, 0) + b"TCFFv1.0"
    buf += struct.pack("<IIII", A, len(waves), (plan["canvas_elems"] * 2) & 0xFFFFFFFF, 1)
    buf += struct.pack("<Q", fnv1a64(bytes(buf[8:32])))
    pad()
    link = 4
    lo = lambda v: v & 0xFFFFFFFF
    for wi, c in enumerate(waves):
        start = len(buf)
        w_off = len(buf)
        wb = to_wmma(c["w_rows"]).tobytes()
        buf += wb
        pad()
        i_off = len(buf)
        ib = c["idx"].astype("<u4").tobytes()
        buf += ib
        pad()
        b_off = len(buf)
        bb = c["bias"].astype("<u2").tobytes()
        buf += bb
        pad()
        end = len(buf)
        h64 = fnv1a64(bytes(buf[start:end]))
        ifd = len(buf)
        struct.pack_into("<I", buf, link, ifd)
        ext = (c["idx_mode"] != 0 or max(c["x_base_off"], c["src_off"], c["y_off"],
                                         c["res_off"]) >= 1 << 32)
        ntags = 21 + (1 if include_geometry else 0) + (1 if ext else 0)
        base = ifd + 2 + 12 * ntags + 4
        tail = bytearray()

        def stash(data: bytes) -> int:
            if len(tail) & 1:
                tail.append(0)
            at = base + len(tail)
            tail.extend(data)
            return at

        u32s = lambda *v: struct.pack("<%dI" % len(v), *v)
        act = ACT_NAMES[c["act"]]
        page = "%s_Wave_%03u_%ux%u_S%u" % (prefix, wi, c["B"], c["Cout"], c["cluster"])
        desc = ("TCFF %s Wave %u/%u | Cin=%u Cout=%u(log=%u) B=%u S=%u Act=%s Res=%d | "
                "W=0x%x Idx=0x%x Bias=0x%x | FNV1a64=0x%016x" % (
                    prefix, wi, len(waves), c["Cin"], c["Cout"], c["logical_Cout"], c["B"],
                    c["cluster"], act, int(c["has_res"]), w_off, i_off, b_off, h64))
        d_at = stash(desc.encode() + b"\0")
        p_at = stash(page.encode() + b"\0")
        r_at = stash(u32s(1, 1))
        par_at = stash(u32s(c["Cin"], c["Cout"], c["B"], c["cluster"], 16, 3, c["act"],
                            int(c["has_res"]), c["h_out"], c["w_out"]))
        aux_at = stash(u32s(w_off, len(wb), i_off, len(ib), b_off, len(bb), lo(c["src_off"]),
                            lo(c["y_off"]), start, end, lo(c["res_off"])))
        h_at = stash(u32s(h64 & 0xFFFFFFFF, h64 >> 32))
        tags = [(254, 4, 1, 2), (256, 4, 1, c["B"]), (257, 4, 1, c["Cout"]), (258, 3, 1, 16),
                (259, 3, 1, 1), (262, 3, 1, 1), (266, 3, 1, 1), (270, 2, len(desc) + 1, d_at),
                (273, 4, 1, w_off), (277, 3, 1, 1), (278, 4, 1, c["Cout"]), (279, 4, 1, len(wb)),
                (282, 5, 1, r_at), (283, 5, 1, r_at), (285, 2, len(page) + 1, p_at),
                (297, 3, 2, wi | (len(waves) << 16)), (339, 3, 1, 3), (0x8440, 4, 1, 0x45564157),
                (0x8441, 4, 10, par_at), (0x8442, 4, 11, aux_at), (0x8443, 4, 2, h_at)]
        if include_geometry:
            if "geom" in c:
                g_at = stash(u32s(*c["geom"]))
            else:
                toks = max(1, c["w_out"])
                g_at = stash(u32s(2 if toks > 1 else 1, toks, c["logical_Cout"], 1, 1, 1,
                                  c["out_stride"], 1, 1, 0))
            tags.append((0x8444, 4, 10, g_at))
        if ext:
            v = [c["idx_mode"], lo(c["idx_stride"]), c["idx_stride"] >> 32, lo(c["x_base_off"]),
                 c["x_base_off"] >> 32, lo(c["src_off"]), c["src_off"] >> 32, lo(c["y_off"]),
                 c["y_off"] >> 32, lo(c["res_off"]), c["res_off"] >> 32, c["seg_len"]]
            tags.append((0x8445, 4, 12, stash(u32s(*v))))
        buf += struct.pack("<H", len(tags))
        for t in tags:
            buf += struct.pack("<HHII", *t)
        link = len(buf)
        buf += struct.pack("<I", 0)
        buf += tail
        pad()
    return bytes(buf)

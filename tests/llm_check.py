"""Node-by-node parity checks of LLM-shaped plans (the config-5 decoder) on the GPU.

PlanChecker runs a compiled plan either command by command (wavec_gpu_execute_range: every
command as compiled, launched alone) or run by run (wavec_gpu_execute_runs: the whole-plan
schedule, with its group launches, folded multiplies and fused RMSNorm + token shift exactly as
wavec_gpu_execute launches them).  Before each step it reads the inputs the step's commands
read; after it, their outputs; every node is compared with the CPU restatement applied to the
inputs the device itself read:

  * projections (all sub-waves of a pruned wave): every output row, on the sampled token
    columns, against llm_oracle.project_dense_f64 (float64, pinned against orc_wave_f64) at the
    north_star bound max|d|/(|ref|+1e-2) <= 2e-3;
  * RMSNorm (per token column) and token shift (whole tensor, with its state block bit for bit)
    against llm_oracle at the same bound; multiply, embedding and argmax bit for bit.

Token columns: `windows` — (first column, count) ranges of the plan's token axis; the full
check of a 16 x 512-token prefill samples three 64-token windows (the first request's start, a
request boundary, the last tokens).  Waves whose gather multiplies operands (folded multiplies,
run mode) are checked on the oracle's product of the operand tensors the device read, waves
that gather through a folded RMSNorm (run mode, decode) on that norm run alone into its own
output range (checked against the oracle), and a multiply that runs its inner multiply (run mode: a * (b * c) in one kernel) on the
oracle's chain of the three operands it read.
"""
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from oracle import llm_oracle as lo

TOL = 2e-3
ACTS = {"q": "sigmoid", "k": "silu", "g": "silu"}
F16 = np.float16


def _base(name: str) -> str:
    return name.split("/")[0]


class PlanChecker:
    def __init__(self, plan, spec, wts, valid: int, decode: bool,
                 windows: Optional[Sequence[Tuple[int, int]]] = None, log=print):
        self.plan, self.spec, self.wts = plan, spec, wts
        self.valid, self.decode = valid, decode
        self.T = (valid + 63) // 64 * 64
        self.windows = list(windows) if windows else [(0, valid)]
        self.cols = np.concatenate([np.arange(a, a + n) for a, n in self.windows])
        assert self.cols.max() < valid
        self.log = log
        self.cmds = plan.cmds
        rep = plan.exec_report()
        self.wave_rep = {w["cmd"]: w for w in rep["waves"]}
        self.aux_rep = {a["cmd"]: a for a in rep["aux"]}
        self.runs: List[List[int]] = rep["runs"]
        self.proj = {"head": (wts.head, None)}
        for l in range(spec.layers):
            for k, p in wts.proj[l].items():
                self.proj[f"l{l}.{k}"] = (p, ACTS.get(k))
        self.mix = {f"l{l}.shift": wts.mix[l] for l in range(spec.layers)}
        self.subwaves: Dict[str, List[int]] = {}
        for i, c in enumerate(self.cmds):
            if c["type"] == "K44_WAVE":
                self.subwaves.setdefault(_base(c["name"]), []).append(i)
        self.worst: Dict[str, float] = {}
        self.checked: Dict[str, int] = {}

    # ------------------------------------------------------------------ canvas reads
    def rows(self, off: int, n: int) -> np.ndarray:
        """[n, len(cols)] fp16: the sampled token columns of n channel rows at `off`."""
        parts = [self.plan.read_canvas_2d(int(off) + a, int(n), self.T, k)
                 for a, k in self.windows]
        return np.concatenate(parts, axis=1).view(F16)

    def full(self, off: int, n: int) -> np.ndarray:
        return self.plan.read_canvas(int(off), int(n) * self.T).view(F16).reshape(int(n), self.T)

    def _state(self, c) -> np.ndarray:
        rf = self.spec.rf
        n = self.spec.d * (rf - 1)
        return self.plan.read_canvas(int(c["state_off"]), n * 64).view(F16).reshape(
            self.spec.d, rf - 1, 64)

    def _note(self, kind: str, err: float, what: str):
        self.worst[kind] = max(self.worst.get(kind, 0.0), err)
        self.checked[kind] = self.checked.get(kind, 0) + 1
        assert err <= TOL, f"{what}: max|d|/(|ref|+1e-2) = {err:.3e}"

    # ------------------------------------------------------------------ wave inputs
    def _wave_input(self, i: int, fused: bool) -> np.ndarray:
        c = self.cmds[i]
        w = self.wave_rep[i]
        if fused and w["xprod"] == 4:  # a folded RMSNorm: the norm run alone materialises it
            self._materialise_norm(i)
            return self.rows(c["src_off"], c["Cin"])
        if fused and w["xprod"] == 5:  # folded RMSNorm + token shift: both run alone
            self._materialise_norm_shift(i, int(w["shift_cmd"]))
            return self.rows(c["src_off"], c["Cin"])
        if fused and w["xprod"]:
            leaves = [self.rows(int(c["src_off"]) + int(d), c["Cin"]) for d in w["xd"][:w["xprod"]]]
            if w["xprod"] == 2:
                return lo.mul(leaves[0], leaves[1])
            return lo.mul(leaves[0], lo.mul(leaves[1], leaves[2]))
        return self.rows(c["src_off"], c["Cin"])

    def _materialise_norm(self, i: int):
        """Run mode, a wave gathering through a folded RMSNorm: the norm command it reads (the
        latest one before it writing its input tensor) is run alone (execute_range: the norm
        kernel with its own exact sums of squares) into the norm's output range, which the
        canvas allocator holds for the norm's output until its last reader and which the
        whole-plan schedule leaves unwritten; the result is checked against the oracle and is
        the wave's input, equal bit for bit to what its gather forms (the folded and unfolded
        decode plans give identical ids and logits: test_folded_multiplies_match_unfolded)."""
        off = int(self.cmds[i]["src_off"])
        n = max(k for k in range(i) if self.cmds[k]["type"] == "RMSNORM_1D"
                and int(self.cmds[k]["y_off"]) == off)
        assert self.aux_rep[n]["fused"], f"{self.cmds[n]['name']}: not a folded norm"
        if n in self._materialised:
            return
        c = self.cmds[n]
        x = self.rows(c["src_off"], c["Cin"])
        self.plan.execute_range(n, 1)
        y = self.rows(c["y_off"], c["Cin"]).astype(np.float64)
        self._note("RMSNORM_1D", lo.orc.rel_err(y, lo.rmsnorm_f64(x)), f"{c['name']} (folded)")
        self._materialised.add(n)

    def _materialise_norm_shift(self, i: int, t: int):
        """Run mode, a wave gathering through a folded RMSNorm and decode token shift (gather
        form 5): the norm and the shift commands are run alone (execute_range) into their own
        output ranges — the place and order of the unfolded plan, whose schedule is the same up
        to this run — and checked against the oracle; the shift's state update is then undone
        (the gathers read the old state), and the state the shift computed is what the launch
        that copies back the folded state must leave (checked in _after)."""
        c = self.cmds[t]
        assert int(c["y_off"]) == int(self.cmds[i]["src_off"]), f"{c['name']}: not the wave's input"
        n = max(k for k in range(t) if self.cmds[k]["type"] == "RMSNORM_1D"
                and int(self.cmds[k]["y_off"]) == int(c["src_off"]))
        assert self.aux_rep[n]["fused"], f"{self.cmds[n]['name']}: not a folded norm"
        if t in self._materialised:
            return
        cn = self.cmds[n]
        x = self.rows(cn["src_off"], cn["Cin"])
        st_raw = self.plan.read_canvas(int(c["state_off"]), self.spec.d * (self.spec.rf - 1) * 64)
        self.plan.execute_range(n, 1)
        y = self.rows(cn["y_off"], cn["Cin"]).astype(np.float64)
        self._note("RMSNORM_1D", lo.orc.rel_err(y, lo.rmsnorm_f64(x)), f"{cn['name']} (folded)")
        xs = self.full(c["src_off"], c["Cin"])
        st_in = st_raw.view(F16).reshape(self.spec.d, self.spec.rf - 1, 64)
        self.plan.execute_range(t, 1)
        ys = self.full(c["y_off"], c["Cin"])
        ref, st_ref = lo.token_shift_decode(xs, self.mix[c["name"]], st_in, self.valid, f64=True)
        st = self._state(c)
        assert np.array_equal(st[:, :, :self.valid].view(np.uint16),
                              st_ref[:, :, :self.valid].view(np.uint16)), \
            f"{c['name']} (folded): state block differs"
        v = self.valid
        self._note("TOKEN_SHIFT_1D", lo.orc.rel_err(ys[:, :v].astype(np.float64), ref[:, :v]),
                   f"{c['name']} (folded)")
        self._pending_state[t] = st.copy()
        self.plan.write_canvas(int(c["state_off"]), st_raw)
        self._materialised.add(t)

    def _y_off(self, i: int, fused: bool) -> int:
        return int(self.wave_rep[i]["y_off_run"] if fused else self.cmds[i]["y_off"])

    # ------------------------------------------------------------------ one step
    def _before(self, members: Sequence[int], fused: bool, state: dict):
        """Reads what the step's commands read (the first time a projection runs: its input and
        residual; later sub-waves must see the same input)."""
        for i in members:
            c = self.cmds[i]
            t = c["type"]
            if t == "K44_WAVE":
                node = _base(c["name"])
                x = self._wave_input(i, fused)
                if node in state["proj_in"]:
                    assert np.array_equal(x.view(np.uint16), state["proj_in"][node][0].view(np.uint16)), \
                        f"{node}: input changed between its sub-waves"
                    continue
                res = self.rows(c["res_off"], c["logical_Cout"]) if c["has_residual"] else None
                state["proj_in"][node] = (x, res)
            elif t == "RMSNORM_1D":
                state[i] = self.rows(c["src_off"], c["Cin"])
            elif t == "TOKEN_SHIFT_1D":
                if not self.decode:  # prefill: the sampled windows and each request's tail
                    # a shift fused into its norm reads the norm's output, read after the step
                    state[i] = None if self._shift_fused(i, fused) else self._shift_inputs(c)
                    continue
                st = self._state(c)
                # a shift fused into its norm reads the norm's output, read after the step
                state[i] = (None if self._shift_fused(i, fused) else self.full(c["src_off"], c["Cin"]), st)
            elif t == "SWIGLU_MUL_1D":
                if fused and self.aux_rep[i]["chain"]:  # runs its inner multiply: a * (b * c)
                    state[i] = tuple(self.rows(o, c["logical_Cout"])
                                     for o in self.aux_rep[i]["operands"])
                else:
                    state[i] = (self.rows(c["src_off"], c["logical_Cout"]),
                                self.rows(c["src2_off"], c["logical_Cout"]))
            elif t == "ARGMAX_1D":
                state[i] = self.rows(c["src_off"], c["Cin"])

    def _shift_fused(self, i: int, fused: bool) -> bool:
        return fused and self.aux_rep.get(i, {}).get("fused", False)

    def _after(self, members: Sequence[int], fused: bool, state: dict, tag: str):
        for i in members:
            c = self.cmds[i]
            t, name = c["type"], c["name"]
            what = f"{tag} {name}"
            if t == "K44_WAVE":
                node = _base(name)
                cp = int(self.wave_rep[i].get("copies_state_of", -1)) if fused else -1
                if cp >= 0:  # this launch copied back a folded token shift's state
                    want = self._pending_state.pop(cp)
                    assert np.array_equal(self._state(self.cmds[cp]).view(np.uint16),
                                          want.view(np.uint16)), \
                        f"{what}: state copied back for {self.cmds[cp]['name']} differs"
                    self.checked["state copy"] = self.checked.get("state copy", 0) + 1
                state["done"].setdefault(node, set()).add(i)
                if state["done"][node] != set(self.subwaves[node]):
                    continue  # the node's other sub-waves have not run yet
                p, act = self.proj[node]
                x, res = state["proj_in"].pop(node)
                ref = lo.project_dense_f64(x, p.starts, self.spec.S, p.weights, p.bias, act, res)
                offs = {self._y_off(j, fused) for j in self.subwaves[node]}
                assert len(offs) == 1, f"{node}: sub-waves store to different tensors"
                y = self.rows(offs.pop(), c["logical_Cout"]).astype(np.float64)
                self._note("K44_WAVE", lo.orc.rel_err(y, ref), what)
            elif t == "RMSNORM_1D":
                y = self.rows(c["y_off"], c["Cin"]).astype(np.float64)
                self._note(t, lo.orc.rel_err(y, lo.rmsnorm_f64(state[i])), what)
            elif t == "TOKEN_SHIFT_1D" and not self.decode:
                inputs = state[i] if state[i] is not None else self._shift_inputs(c)
                self._check_shift_prefill(c, inputs, what)
            elif t == "TOKEN_SHIFT_1D":
                x, st_in = state[i]
                if x is None:  # fused: its input is the norm output the step just wrote
                    x = self.full(c["src_off"], c["Cin"])
                y = self.full(c["y_off"], c["Cin"])
                ref, st_ref = lo.token_shift_decode(x, self.mix[name], st_in, self.valid, f64=True)
                st = self._state(c)
                # request slots past the batch are not touched
                assert np.array_equal(st[:, :, :self.valid].view(np.uint16),
                                      st_ref[:, :, :self.valid].view(np.uint16)), \
                    f"{what}: state block differs"
                v = self.valid
                self._note(t, lo.orc.rel_err(y[:, :v].astype(np.float64), ref[:, :v]), what)
            elif t == "SWIGLU_MUL_1D":
                if fused and self.aux_rep[i]["fused"]:
                    continue  # folded: checked through its readers' inputs
                y = self.rows(c["y_off"], c["logical_Cout"])
                if len(state[i]) == 3:
                    a, b, c3 = state[i]
                    want = lo.mul(a, lo.mul(b, c3))
                else:
                    a, b = state[i]
                    want = lo.mul(a, b)
                assert np.array_equal(y.view(np.uint16), want.view(np.uint16)), what
                self.checked[t] = self.checked.get(t, 0) + 1
            elif t == "EMBED_1D":
                y = self.rows(c["y_off"], c["logical_Cout"])
                want = lo.embed(self.wts.embed, state["ids"][self.cols], len(self.cols))
                assert np.array_equal(y.view(np.uint16), want.view(np.uint16)), what
                self.checked[t] = self.checked.get(t, 0) + 1
            elif t == "ARGMAX_1D":
                got = self.plan.get_ids(self.valid)[self.cols]
                assert np.array_equal(got, lo.argmax(state[i], len(self.cols))), what
                self.checked[t] = self.checked.get(t, 0) + 1

    def _progress(self, tag: str, mode: str, k: int, n: int):
        if n >= 100 and (k + 1) % 50 == 0:
            self.log(f"[{tag}] {mode}: {k + 1} of {n} steps checked")

    # ------------------------------------------------------------------ prefill token shift
    def _shift_inputs(self, c):
        """Input columns a prefill token shift needs for the sampled windows (each window with
        the rf-1 columns before it) and for the state block (each request's last rf-1)."""
        rf, seq, D = self.spec.rf, self.spec.prompt, c["Cin"]
        T = self.T
        wins = []
        for a, n in self.windows:
            lo_ = max(0, a - (rf - 1))
            wins.append((a, n, lo_, self.plan.read_canvas_2d(int(c["src_off"]) + lo_, D, T,
                                                             a + n - lo_).view(F16)))
        tail = min(rf - 1, seq)
        R = self.valid // seq
        tails = [self.plan.read_canvas_2d(int(c["src_off"]) + r * seq + seq - tail, D, T,
                                          tail).view(F16) for r in range(R)] if tail else []
        return wins, tails

    def _check_shift_prefill(self, c, inputs, what):
        """y[:, t] = sum_{i < rf, i <= t % seq} mu[:, i] x[:, t - i] on the sampled windows
        (the window form of llm_oracle.token_shift); state[c][i][r] = x[c][r*seq + seq-1-i]
        bit for bit (zero beyond the requests)."""
        wins, tails = inputs
        mu = self.mix[c["name"]].astype(np.float64)
        rf, seq = mu.shape[1], self.spec.prompt
        ys, refs = [], []
        for a, n, lo_, xw in wins:
            xf = xw.astype(np.float64)
            ref = np.zeros((xf.shape[0], n))
            for k in range(n):
                t = a + k
                for i in range(min(rf, t % seq + 1)):
                    ref[:, k] += mu[:, i] * xf[:, t - i - lo_]
            refs.append(ref)
            ys.append(self.plan.read_canvas_2d(int(c["y_off"]) + a, c["Cin"], self.T, n).view(F16))
        err = lo.orc.rel_err(np.concatenate(ys, 1).astype(np.float64), np.concatenate(refs, 1))
        want = np.zeros((c["Cin"], max(rf - 1, 0), 64), F16)
        for r, tail in enumerate(tails):
            for i in range(tail.shape[1]):
                want[:, i, r] = tail[:, tail.shape[1] - 1 - i]
        assert np.array_equal(self._state(c).view(np.uint16), want.view(np.uint16)), \
            f"{what}: state block differs"
        self._note("TOKEN_SHIFT_1D", err, what)

    # ------------------------------------------------------------------ drivers
    def run(self, mode: str, ids: np.ndarray, tag: str):
        """mode 'commands' (execute_range per graph node) or 'runs' (execute_runs per run)."""
        self.plan.set_ids(ids)
        state = {"proj_in": {}, "done": {}, "ids": np.asarray(ids, dtype=np.uint32)}
        self._materialised = set()
        self._pending_state = {}
        if mode == "commands":
            steps, i = [], 0
            while i < len(self.cmds):  # consecutive commands of one node (pruned sub-waves)
                j = i + 1
                while j < len(self.cmds) and _base(self.cmds[j]["name"]) == _base(self.cmds[i]["name"]):
                    j += 1
                steps.append(list(range(i, j)))
                i = j
            for k, s in enumerate(steps):
                self._before(s, False, state)
                self.plan.execute_range(s[0], len(s))
                self._after(s, False, state, tag)
                self._progress(tag, mode, k, len(steps))
        else:
            for r, members in enumerate(self.runs):
                self._before(members, True, state)
                self.plan.execute_runs(r, 1)
                self._after(members, True, state, tag)
                self._progress(tag, mode, r, len(self.runs))
        assert not state["proj_in"], f"projections never completed: {sorted(state['proj_in'])}"
        assert not self._pending_state, f"folded states never copied back: {sorted(self._pending_state)}"
        self.log(f"[{tag}] {mode}: checked " + ", ".join(
            f"{k} x{n}" + (f" (worst {self.worst[k]:.2e})" if k in self.worst else "")
            for k, n in sorted(self.checked.items())))

"""MoELayer: the Python call surface the reference's engine sees at a layer's experts, on the HIP library.

Names and argument meaning follow the reference:
  routing_fn(bsz, cfg, z, params) -> (sel int64 [bsz, k], w fp16 [bsz, k])     exllamav3 BlockSparseMLP.routing_fn,
                                                                                hooked at engine/tiers.py:707-726
  layer(li, sel, w, z, bsz) -> (sel, w, cpu_flag)                               engine/nv2.py:374-437 (Nv2.layer)
  run_bszN(z, sel, rw) -> out [bsz, H] fp32                                     exllamav3 bc.run_bszN, engine/nv2.py:634
  cpu_split_combine(fhs, cpu_partial, cpu_pending, shape) -> fhs                engine/tiers.py:730-739
  combine(fhs) -> fhs                                                           engine/nv2.py:489-493 (Nv2.combine)
  run_single_expert(y, e, x), run_single_expert_dq                             engine/tiers.py:597-605
Every call enqueues on torch's current stream; nothing synchronises the host (verify_on_cpu, a host-side check with
the exact CPU lane, excepted).
"""
import ctypes

import torch

from . import _lib as L
from . import ops


class MoELayer:
    """One MoE layer's experts on the HIP library. table: the layer's ExpertTable; topk, first (routing_first); router:
    score (SCORE_SOFTMAX / SCORE_SIGMOID / SCORE_SQRTSP), selection bias fp32 [E], group limit, renorm, scale
    (routed_scaling_factor); activation, gated, act_limit; router_weight: fp16 [E, H] gate weight (checkpoint layout),
    used when no logits are given; shared_gate: fp16 [H] gate vector of the shared expert (its output scaled by
    sigmoid(x . shared_gate)) or None; slots / li: an ExpertSlots table and this layer's index in it."""

    def __init__(self, table, topk, first=0, score=L.SCORE_SIGMOID, bias=None, n_group=1, topk_group=1, renorm=True,
                 scale=1.0, act=L.ACT_SILU, gated=True, act_limit=0.0, router_weight=None, slots=None, li=0,
                 shared_gate=None):
        self.table = table
        self.num_experts_per_tok = topk
        self.routing_first = first
        self.num_local_experts = table.E
        self.hidden_size, self.intermediate_size = table.H, table.I
        self.score, self.bias, self.n_group, self.topk_group = score, bias, n_group, topk_group
        self.renorm, self.scale = renorm, scale
        self.act, self.gated, self.act_limit = act, gated, act_limit
        if router_weight is not None and (router_weight.dtype != torch.float16 or not router_weight.is_cuda or
                                          tuple(router_weight.shape) != (table.E, table.H) or
                                          not router_weight.is_contiguous()):
            raise ValueError(f"router_weight must be a contiguous fp16 device tensor [E, H] = [{table.E}, {table.H}]")
        self.router_weight = router_weight        # fp16 [E, H] or None (logits passed in params["logits"])
        self.shared_gate = shared_gate
        self.slots, self.li = slots, li           # optional ExpertSlots (expert-slot table) and this layer's index
        self.desc = table.desc(topk, first, act, gated, act_limit, shared_gate=shared_gate)
        self.slot_desc = (slots.desc(li, topk, first, act, gated, act_limit, shared_gate=shared_gate)
                          if slots is not None else None)
        self.router = L.RouterDesc(score, int(renorm), n_group, topk_group, scale, 0,
                                   bias.data_ptr() if bias is not None else None,
                                   router_weight.data_ptr() if router_weight is not None else None)
        self._ws = None
        self.out_bszn = None

    # ---- router ----
    def router_logits(self, z):
        """fp16 [T, E] router logits of the MoE input z, projected on the GPU (bmx_router_logits)."""
        if self.router_weight is None:
            raise ValueError("MoELayer: no router weight; pass params['logits']")
        x = z.view(-1, self.hidden_size)
        if x.dtype != torch.float16 or not x.is_contiguous():
            x = x.half().contiguous()
        return ops.router_logits(x, self.router_weight)

    def routing_fn(self, bsz, cfg, z, params):
        logits = params.get("logits") if params else None
        if logits is None:
            logits = self.router_logits(z)
        logits = logits.view(bsz, -1).to(torch.float16).contiguous()
        return ops.router_topk(logits, self.num_experts_per_tok, self.bias, self.n_group, self.topk_group, self.score,
                               self.renorm, self.scale, self.routing_first)

    # ---- engine hook: residency before the experts run ----
    def layer(self, li, sel, w, z, bsz):
        """The slot-table step of this call. With a planned table (ExpertSlots.plan) the agent's planner answers the
        step: returns the selection the GPU computes (CPU-lane picks masked) and whether a CPU job may add to this call
        (combine() adds it), as the reference's Nv2.layer (engine/nv2.py:374-437)."""
        self._cpu_seq = None
        self._staged = None
        if self.slots is None:
            return sel, w, False
        if self.slots.stage_prefill(li, sel, first=self.routing_first):
            # a prefill-size call (the reference's staged call, engine/nv2.py:378-386): hits marked, nothing admitted,
            # the layer's table points at the staging arena until its products are done
            self._staged = li
            return sel, w, False
        if getattr(self.slots, "planned", False):
            sel_gpu, w_gpu, _, seq = self.slots.step_planned(li, sel, w, z, True, first=self.routing_first,
                                                             bsz=bsz)
            if self.slots.cpu_ready and z is not None and bsz <= L.PLAN_MAXT and sel.numel() <= L.PLAN_MAXP:
                self._cpu_seq = seq
            return sel_gpu.view(sel.shape), w_gpu.view(w.shape), self._cpu_seq is not None
        self.slots.step(li, sel, True, first=self.routing_first)
        return sel, w, False

    def route_layer(self, li, z, bsz, params=None):
        """routing_fn followed by layer() (the reference's routing hook, then the step of Nv2.layer): for a one-token
        call on a slot table that is not planned, both in one launch (ExpertSlots.route_step, bmx_route_slot_step: the
        same picks, weights and table state); other calls run the two hooks. Returns (sel, w, cpu_job) as layer()."""
        if self.slots is None or bsz != 1 or getattr(self.slots, "planned", False):
            sel, w = self.routing_fn(bsz, None, z, params)
            return self.layer(li, sel, w, z, bsz)
        logits = params.get("logits") if params else None
        if logits is None:
            logits = self.router_logits(z)
        self._cpu_seq = None
        self._staged = None
        if getattr(self.slots, "st_open", False):
            self.slots.stage_end()          # a one-token call ends a staged forward, as in layer()
        sel, w = self.slots.route_step(li, logits.reshape(-1), self.num_experts_per_tok, self.bias, self.n_group,
                                       self.topk_group, self.score, self.renorm, self.scale, True,
                                       first=self.routing_first)
        return sel, w, False

    # ---- experts + combine ----
    def run_bszN(self, z, sel, rw, path=L.PATH_AUTO):
        x = z.view(-1, self.hidden_size)
        if x.dtype != torch.float16 or not x.is_contiguous():
            x = x.half().contiguous()
        sel = sel.view(x.shape[0], -1)
        if sel.dtype != torch.int64 or not sel.is_contiguous():
            sel = sel.long().contiguous()
        rw = rw.view(x.shape[0], -1)
        if rw.dtype != torch.float16 or not rw.is_contiguous():
            rw = rw.half().contiguous()
        staged, self._staged = getattr(self, "_staged", None), None
        if self.slots is not None and staged is not None:
            # every expert's table entry points at a slot or at the staging arena: the plain layer, then the restore
            need = L.lib().bmx_moe_workspace(self.slot_desc, x.shape[0], path)
            if self._ws is None or self._ws.numel() < need:
                self._ws = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
            self.out_bszn = ops.moe_forward(self.slot_desc, x, sel, rw, path, self._ws)
            self.slots.stage_restore(staged)
            return self.out_bszn
        if self.slots is not None:
            self.out_bszn = self._run_slots(x, sel, rw, path)
            return self.out_bszn
        need = L.lib().bmx_moe_workspace(self.desc, x.shape[0], path)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
        self.out_bszn = ops.moe_forward(self.desc, x, sel, rw, path, self._ws)
        return self.out_bszn

    def _run_slots(self, x, sel, rw, path):
        """Expert products with the slot table: gate / up of the experts resident before this layer's step, then (after
        the copies of the gate / up parts of the experts it admitted) the admitted ones and the activation, the down
        products of the resident experts while the admitted experts' down parts are still being copied, then theirs and
        the combine."""
        T, lib = x.shape[0], L.lib()
        desc = self.slot_desc
        routes = ops.dispatch(sel, self.num_local_experts, self.routing_first, self.table.has_shared,
                              lib.bmx_rows_per_group(T, self.num_experts_per_tok, path))
        need = lib.bmx_experts_workspace(ctypes.byref(desc), T, path)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
        out = torch.empty((T, self.hidden_size), dtype=torch.float32, device=x.device)
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        P = lambda t: ctypes.c_void_p(t.data_ptr())

        def stage(st):
            L.check(lib.bmx_moe_stage(ctypes.byref(desc), st, P(x), T, ctypes.byref(routes.struct), None, None, P(rw),
                                      P(out), P(self._ws), self._ws.numel(), path, s), "bmx_moe_stage")

        stage(L.STAGE_PREP)
        stage(L.STAGE_GATE_UP_RESIDENT)
        self.slots.wait_copies(self.li, part="gate_up")
        stage(L.STAGE_GATE_UP_STAGED)
        stage(L.STAGE_ACT)
        stage(L.STAGE_DOWN_RESIDENT)
        self.slots.wait_copies(self.li, part="down")
        stage(L.STAGE_DOWN_STAGED)
        stage(L.STAGE_COMBINE)
        self._routes = routes
        return out

    # ---- single-expert paths ----
    def run_single_expert(self, y, e, x, path=L.PATH_AUTO):
        """Expert e (local id) on the rows x (fp16 [n, H]): its down output after svh (what the combine weights) into
        y (fp32 [n, H]), through the routed layer's kernels with every row routed to e alone (top-1, weight 1, no
        shared expert). exllamav3's BlockSparseMLP run_single_expert, which the reference wraps
        (engine/tiers.py:602-605) to copy the expert's bytes into its bounce slot first; here the expert table already
        points at the expert's slot or home. Returns y."""
        x = x.view(-1, self.hidden_size)
        if x.dtype != torch.float16 or not x.is_contiguous():
            x = x.half().contiguous()
        n, E = x.shape[0], self.num_local_experts
        if not 0 <= int(e) < E:
            raise ValueError(f"run_single_expert: expert {e} outside [0, {E})")
        if tuple(y.shape) != (n, self.hidden_size) or y.dtype != torch.float32:
            raise ValueError("run_single_expert: y must be fp32 [n, H]")
        if n == 0:
            return y
        sel = torch.full((n, 1), int(e) + self.routing_first, dtype=torch.int64, device=x.device)
        desc = self.table.desc(1, self.routing_first, self.act, self.gated, self.act_limit)
        desc.shared = None
        routes = ops.dispatch(sel, E, self.routing_first, False, L.lib().bmx_rows_per_group(n, 1, path))
        rows, _ = ops.moe_experts(desc, x, routes, path)
        y.copy_(rows[:n])            # one expert: its rows are the tokens in order
        return y

    def run_single_expert_dq(self, y, e, x, path=L.PATH_AUTO):
        """The reference's other per-expert entry (engine/tiers.py:597-600: exllamav3 reconstructs the expert's fp16
        weights first). The trellis kernels compute the same products without a reconstructed copy: run_single_expert."""
        return self.run_single_expert(y, e, x, path)

    def verify_on_cpu(self, z, sel, rw, threads=16, y_rows=None):
        """Recompute every expert row of a decode-path call on the host with the exact CPU lane and compare it with the
        GPU's, bit for bit (a check for silent corruption: the two must agree exactly). Synchronises. Returns the
        mismatching (row, expert) pairs; y_rows: the GPU's rows to check (default: computed here)."""
        import numpy as np
        from . import cpu_lane
        x = z.view(-1, self.hidden_size)
        if x.dtype != torch.float16 or not x.is_contiguous():
            x = x.half().contiguous()
        T = x.shape[0]
        sel = sel.view(T, -1).long().contiguous()
        routes = ops.dispatch(sel, self.num_local_experts, self.routing_first, self.table.has_shared,
                              L.lib().bmx_rows_per_group(T, self.num_experts_per_tok, L.PATH_DECODE))
        if y_rows is None:
            y_rows, _ = ops.moe_experts(self.desc, x, routes, L.PATH_DECODE)
        ks_gu, ks_dn, grouped = cpu_lane.decode_splits(self.desc, T)
        y = y_rows.cpu().numpy()
        offs = routes.offsets.cpu().numpy()
        rt = routes.row_token.cpu().numpy()
        xs = x.cpu().numpy()
        bad = []
        for e in range(self.num_local_experts + (1 if self.table.has_shared else 0)):
            r0, r1 = int(offs[e]), int(offs[e + 1])
            if r1 <= r0:
                continue
            yc = cpu_lane.expert_rows(self.table.host_expert(e), self.hidden_size, self.intermediate_size, xs[rt[r0:r1]],
                                      ks_gu, ks_dn, grouped, self.act, self.gated, self.act_limit, threads)
            for i in np.flatnonzero((yc.view(np.uint32) != y[r0:r1].view(np.uint32)).any(1)):
                bad.append((r0 + int(i), e))
        return bad

    def cpu_split_combine(self, fhs, cpu_partial=None, cpu_pending=False, shape=None):
        if cpu_pending and cpu_partial is not None:
            fhs = fhs + cpu_partial.to(fhs.dtype)
        return fhs.view(shape) if shape is not None else fhs

    def combine(self, fhs):
        """Nv2.combine (engine/nv2.py:489-493): adds the CPU lane's partial of this call's planned step, if any."""
        fhs = fhs if fhs.is_contiguous() else fhs.contiguous()
        seq, self._cpu_seq = getattr(self, "_cpu_seq", None), None
        if seq is not None:
            self.slots.cpu_add(seq, fhs.view(-1, self.hidden_size))
        return fhs

    def forward(self, z, logits=None, path=L.PATH_AUTO):
        if (logits is not None or self.router_weight is not None) and self.slots is None:
            # the whole call in one library entry (router + dispatch fused at decode sizes; the router projection of z
            # first when no logits are given)
            x = z.view(-1, self.hidden_size)
            if x.dtype != torch.float16 or not x.is_contiguous():
                x = x.half().contiguous()
            lg = logits.view(x.shape[0], -1).to(torch.float16).contiguous() if logits is not None else None
            need = L.lib().bmx_moe_layer_workspace(self.desc, x.shape[0], path)
            if self._ws is None or self._ws.numel() < need:
                self._ws = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
            out, self.sel, self.w = ops.moe_layer(self.desc, self.router, x, lg, path, self._ws)
            self.out_bszn = out
            return out
        bsz = z.shape[0]
        sel, w = self.routing_fn(bsz, None, z, {"logits": logits} if logits is not None else {})
        sel, w, _ = self.layer(self.li, sel, w, z, bsz)
        out = self.run_bszN(z, sel, w, path)
        return self.cpu_split_combine(self.combine(out), None, False, None)

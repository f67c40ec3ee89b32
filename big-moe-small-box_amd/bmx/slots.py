"""ExpertSlots: the VRAM expert-slot table over a stack of MoE layers (the reference's Pool: slot geometry, slotof /
owner / reference bits / pins, per-layer pointer tables and homes; engine/tiers.py:275-373, step kernel ec_step_k at
engine/ec.py:16-76, copies ec_copy_k engine/ec.py:78-105 and stage_layer engine/kernels/nv2/nv2_host.cpp:1558-1593).

Every layer keeps its experts' trellis at home (an ExpertTable, typically with its arena in pinned host memory); S
uniform slots of the layers' record size live in VRAM. step(li, sel) runs the CLOCK step of layer li on the current
stream (hits pinned, misses admitted, table pointers rewritten) and the copies of its admissions on a side stream;
the layer's expert products wait for those copies only in their staged part (MoELayer.run_bszN). prefetch(lj, guess)
admits a later layer's guessed experts ahead of its step (the reference's layer-ahead routing guess, engine/nv2.py:
450-487) with copies on the same side stream. No host synchronisation anywhere."""
import ctypes
import os
import weakref

import torch

from . import _lib as L


class ExpertSlots:
    def __init__(self, layers, S, maxj=32, disabled=(), copies="kernel", first=0):
        """layers: one ExpertTable per layer (same H, I, E and record geometry); S slots; maxj admissions per step;
        disabled: slot indices never used. copies: "kernel" (a copy kernel on the side stream reads the homes) or
        "dma" (a host thread of the library issues them on the DMA engines, which leaves the other kernels their
        memory bandwidth; the layer's stages wait on the copies with a small polling kernel). first: global id of
        local expert 0 (routing_first), held here as the reference's Pool holds it (engine/tiers.py:272)."""
        if copies not in ("kernel", "dma"):
            raise ValueError("ExpertSlots: copies must be 'kernel' or 'dma'")
        t0 = layers[0]
        for t in layers:
            if (t.H, t.I, t.E, t.rec, t.off_u, t.off_d) != (t0.H, t0.I, t0.E, t0.rec, t0.off_u, t0.off_d):
                raise ValueError("ExpertSlots: layers must share H, I, E and the record geometry")
        self.layers, self.L, self.E, self.S, self.maxj = layers, len(layers), t0.E, S, maxj
        self.first = int(first)
        dev = t0.device
        i32 = dict(dtype=torch.int32, device=dev)
        self.arena = torch.empty((max(S, 1), t0.rec), dtype=torch.uint8, device=dev)
        self.slotof = torch.full((self.L * self.E,), -1, **i32)
        self.owner = torch.full((max(S, 1),), -1, **i32)
        self.refb = torch.zeros(max(S, 1), **i32)
        self.pin = torch.zeros(max(S, 1), **i32)
        for s in disabled:
            self.pin[s] = -1
        self.ctl = torch.zeros(4, **i32)
        self.jobs = torch.zeros(2 * max(maxj, 1), **i32)
        self.fresh = torch.zeros(self.E, **i32)
        self.pjobs = torch.zeros(2 * (1 + 2 * max(maxj, 1)), **i32)
        self.pfl = torch.zeros(max(S, 1), **i32)
        self.stats_t = torch.zeros(8, dtype=torch.int64, device=dev)
        home = [a for t in layers for e in range(t.E) for a in t.addr[e]]
        self.home = torch.tensor(home, dtype=torch.int64, device=dev)       # uint64 addresses, int64 storage
        base = self.arena.data_ptr()
        self.slot_base = torch.tensor([base + s * t0.rec for s in range(max(S, 1))], dtype=torch.int64, device=dev)
        self.tables = torch.tensor([t.table().data_ptr() for t in layers], dtype=torch.int64, device=dev)
        P = lambda x: x.data_ptr()
        self.struct = L.SlotTable(self.L, self.E, S, maxj, t0.H, t0.I, t0.rec, t0.off_u, t0.off_d,
                                  P(self.slotof), P(self.owner), P(self.refb), P(self.pin), P(self.ctl), P(self.jobs),
                                  P(self.fresh), P(self.stats_t), P(self.home), P(self.slot_base), P(self.tables),
                                  P(self.pjobs), P(self.pfl))
        self.side = torch.cuda.Stream(device=dev)
        self.copied = [None] * self.L        # event: copies of the layer's last step done
        self.last_copied = None              # event: copies of the last step (any layer) done: they read its job buffer
        self.pf_copied = [None, None]        # event per prefetch job buffer: its last copies done
        self.pf_calls = 0
        self.copies = copies
        self.agent = None
        self.seq = [0] * self.L               # dma: sequence number of each layer's last step
        self.planned = False                  # dma: layer calls use planned steps (plan())
        self.cpu_ready = False                # dma: the agent has a CPU lane (cpu_lane())
        self.last_seq = 0                     # dma: the last sequence number the agent was given
        # staged prefill (stage_prefill): calls of at least stage_min picks admit nothing; each layer's experts that are
        # not resident are copied into one of two staging arenas one layer ahead on copy streams
        self.stage_min = 8192                 # picks (the reference's EC_STAGE_MIN default, engine/tiers.py:673)
        # copy streams the staging copies alternate over: a copy's set-up overlaps the transfer before it
        self.stage_streams = int(os.environ.get("BMX_STAGE_STREAMS", "2"))
        self.cstreams = []
        self.st_buf = [None, None]            # staging arenas, uint8 [n * rec] each
        self.st_ready = [[], []]              # events: the arena's last staging copies done (one per copy stream)
        self.st_open = False
        self.st_last = None                   # layer of the last staged call of the open forward
        self.st_layers = {}                   # li -> (experts np.int32, experts on the device, copy runs)
        self.st_sub = set()                   # layers whose copies are enqueued in this forward
        self.st_stats = dict(forwards=0, layers=0, experts=0, bytes=0)
        if copies == "dma":
            homes = (ctypes.c_uint64 * (self.L * self.E))(*[t.addr[e][0] for t in layers for e in range(t.E)])
            nb = (ctypes.c_int64 * (self.L * self.E * 3))(*[t.mat_bytes(e, m) for t in layers for e in range(t.E)
                                                            for m in range(3)])
            ag = ctypes.c_void_p()
            L.check(L.lib().bmx_copy_agent_create(ctypes.byref(self.struct), homes, nb, ctypes.byref(ag)),
                    "bmx_copy_agent_create")
            self.agent = ag
            self._finalizer = weakref.finalize(self, ExpertSlots._destroy_agent, ag.value)

    @staticmethod
    def _destroy_agent(ptr):
        try:
            torch.cuda.synchronize()
        finally:
            L.lib().bmx_copy_agent_destroy(ctypes.c_void_p(ptr))

    def close(self):
        """Stop the copy agent (dma): synchronises the device first."""
        if self.agent is not None:
            self._finalizer()
            self.agent = None

    def agent_status(self):
        """dma: (records, copies, bytes copied, gate / up mark, down mark, a wait ran out of time); raises if a copy
        failed, the agent aborted or a wait ran out of time (final: the slot contents of copies that had not completed
        are not trusted, so the layer calls since the failure are to be discarded)."""
        st = (ctypes.c_int64 * 6)()
        L.check(L.lib().bmx_copy_agent_status(self.agent, st), "bmx_copy_agent_status")
        return tuple(st)

    def plan_stats(self):
        """(requests answered, experts put on the CPU lane summed over requests, CPU jobs done, microseconds the CPU
        lane's worker spent on them, its running mean per CPU pick in nanoseconds) of the agent's planner."""
        st = (ctypes.c_int64 * 5)()
        L.check(L.lib().bmx_copy_agent_plan_stats(self.agent, st), "bmx_copy_agent_plan_stats")
        return tuple(st)

    def check(self):
        """Raise if the copy agent has failed (dma; a host read of shared memory, no synchronisation)."""
        if self.agent is not None:
            L.check(L.lib().bmx_copy_agent_status(self.agent, None), "ExpertSlots")

    def step(self, li, sel, admit=True, *, first=None):
        """CLOCK step of layer li over the picks sel (int64 device tensor of global ids) on the current stream, then the
        copies of its admissions on the side stream: Pool.step(li, sel, admit) (engine/tiers.py:360-373). first
        overrides the table's routing_first for this call. Raises if the copy agent has failed."""
        if sel.dtype != torch.int64 or not sel.is_contiguous():
            sel = sel.long().contiguous()
        first = self.first if first is None else int(first)
        cur = torch.cuda.current_stream()
        if self.agent is not None:
            q = ctypes.c_int64()
            L.check(L.lib().bmx_slot_step_agent(ctypes.byref(self.struct), self.agent, li,
                                                ctypes.c_void_p(sel.data_ptr()), sel.numel(), int(first), int(admit),
                                                ctypes.byref(q), ctypes.c_void_p(cur.cuda_stream)), "bmx_slot_step_agent")
            self.seq[li] = q.value
            self.last_seq = max(self.last_seq, q.value)
            return None
        if self.last_copied is not None:       # the previous step's copies read the job buffer this step rewrites
            cur.wait_event(self.last_copied)
        L.check(L.lib().bmx_slot_step(ctypes.byref(self.struct), li, ctypes.c_void_p(sel.data_ptr()), sel.numel(),
                                      int(first), int(admit), ctypes.c_void_p(cur.cuda_stream)), "bmx_slot_step")
        return self._copy_after_step(li, cur)

    def _copy_after_step(self, li, cur):
        """The copies of a plain step's admissions on the side stream, after the step on stream cur."""
        stepped = torch.cuda.Event()
        stepped.record(cur)
        self.side.wait_event(stepped)
        evs = []
        for mats in (3, 4):          # gate and up first, down behind them
            L.check(L.lib().bmx_slot_copy_mats(ctypes.byref(self.struct), li, mats,
                                               ctypes.c_void_p(self.side.cuda_stream)), "bmx_slot_copy_mats")
            ev = torch.cuda.Event()
            ev.record(self.side)
            evs.append(ev)
        self.copied[li] = tuple(evs)
        self.last_copied = evs[1]
        return evs[1]

    def route_step(self, li, logits, topk, bias=None, n_group=1, topk_group=1, score=L.SCORE_SIGMOID, renorm=True,
                   scale=1.0, admit=True, *, first=None):
        """One token's routing and the step of layer li in one launch (bmx_route_slot_step): the same picks, weights
        and table state as ops.router_topk followed by step(li, sel, admit). logits fp16 [1, E] or [E] (device).
        Returns (sel int64 [1, topk], w fp16 [1, topk])."""
        if logits.dtype != torch.float16 or not logits.is_contiguous():
            logits = logits.half().contiguous()
        E = logits.numel()
        if bias is not None and (bias.dtype != torch.float32 or not bias.is_contiguous()):
            bias = bias.float().contiguous()
        first = self.first if first is None else int(first)
        sel = torch.empty((1, topk), dtype=torch.int64, device=logits.device)
        w = torch.empty((1, topk), dtype=torch.float16, device=logits.device)
        cur = torch.cuda.current_stream()
        P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
        if self.agent is None and self.last_copied is not None:   # the previous step's copies read the job buffer
            cur.wait_event(self.last_copied)
        q = ctypes.c_int64()
        L.check(L.lib().bmx_route_slot_step(ctypes.byref(self.struct), self.agent, li, P(logits), P(bias), E, topk,
                                            n_group, topk_group, score, int(renorm), float(scale), first, int(admit),
                                            P(sel), P(w), ctypes.byref(q), ctypes.c_void_p(cur.cuda_stream)),
                "bmx_route_slot_step")
        if self.agent is not None:
            self.seq[li] = q.value
            self.last_seq = max(self.last_seq, q.value)
            return sel, w
        self._copy_after_step(li, cur)
        return sel, w

    def prefetch(self, li, guess, limit=None, *, first=None):
        """Layer-ahead prefetch into layer li's slots: the first `limit` (default maxj) distinct guesses (int64 device
        tensor, best first) that are not resident are admitted on the current stream without advancing the step counter
        (the slots the last step pinned stay pinned) and copied on the side stream, ahead of layer li's step. A hint
        only: layer li's next step hands the prefetched experts it uses to the staged part, so results never change."""
        if guess.dtype != torch.int64 or not guess.is_contiguous():
            guess = guess.long().contiguous()
        first = self.first if first is None else int(first)
        n = guess.numel()
        if n > 512:
            raise ValueError("ExpertSlots.prefetch: at most 512 guesses")
        cur = torch.cuda.current_stream()
        lim = self.maxj if limit is None else int(limit)
        if self.agent is not None:
            q = ctypes.c_int64()
            L.check(L.lib().bmx_slot_prefetch_agent(ctypes.byref(self.struct), self.agent, li,
                                                    ctypes.c_void_p(guess.data_ptr()), n, int(first), lim,
                                                    ctypes.byref(q), ctypes.c_void_p(cur.cuda_stream)),
                    "bmx_slot_prefetch_agent")
            self.last_seq = max(self.last_seq, q.value)
            return None
        b = self.pf_calls & 1
        self.pf_calls += 1
        if self.pf_copied[b] is not None:      # the buffer's previous copies read its jobs while they run
            cur.wait_event(self.pf_copied[b])
        L.check(L.lib().bmx_slot_prefetch(ctypes.byref(self.struct), li, ctypes.c_void_p(guess.data_ptr()), n,
                                          int(first), lim, b, ctypes.c_void_p(cur.cuda_stream)), "bmx_slot_prefetch")
        admitted = torch.cuda.Event()
        admitted.record(cur)
        self.side.wait_event(admitted)
        guess.record_stream(self.side)
        L.check(L.lib().bmx_slot_prefetch_copy(ctypes.byref(self.struct), li, b, 7,
                                               ctypes.c_void_p(self.side.cuda_stream)), "bmx_slot_prefetch_copy")
        ev = torch.cuda.Event()
        ev.record(self.side)
        self.pf_copied[b] = ev
        return ev

    def wait_copies(self, li, stream=None, part="all"):
        """Order `stream` (default: current) after the copies of layer li's last step: part "gate_up" (the admitted
        experts' gate and up matrices), "down" or "all"."""
        if self.agent is not None:
            self.check()
            if self.seq[li]:
                st = stream or torch.cuda.current_stream()
                L.check(L.lib().bmx_copy_wait_layer(self.agent, li, 0 if part == "gate_up" else 1,
                                                    ctypes.c_void_p(st.cuda_stream)), "bmx_copy_wait_layer")
            return
        if self.copied[li] is not None:
            ev = self.copied[li][0 if part == "gate_up" else 1]
            (stream or torch.cuda.current_stream()).wait_event(ev)

    # ---- residency plan (dma) ----
    def plan(self, policy=None):
        """Set the copy agent's planner (a dict of bmx_plan_policy fields; None: every miss admitted). From then on
        layer calls through MoELayer use planned steps."""
        if self.agent is None:
            raise ValueError("ExpertSlots.plan: the residency plan runs on the copy agent (copies='dma')")
        if policy is None:
            L.check(L.lib().bmx_copy_agent_plan(self.agent, None), "bmx_copy_agent_plan")
        else:
            pol = L.PlanPolicy(**policy)
            L.check(L.lib().bmx_copy_agent_plan(self.agent, ctypes.byref(pol)), "bmx_copy_agent_plan")
        self.planned = True

    def cpu_lane(self, topk, act=L.ACT_SILU, gated=True, act_limit=0.0, threads=16, copy=False):
        """Give the copy agent its CPU lane: the experts of every layer (kept here) for the agent's worker.

        copy=False: the lane reads the trellis bytes where they are (the homes, pinned host memory, for a host-homed
        table). copy=True: the lane reads its own copy of each distinct home arena in ordinary host memory, which the
        kernel backs with 2 MB pages (numpy advises huge pages for large arrays). Pinned memory is mapped in 4 KB pages,
        and a cold expert read from a few tens of GB of them waits on page-table walks: measured in a 43-layer stack,
        a fast-mode expert call took 543 us from the pinned homes and 185 us from the copy. The copy costs the homes'
        size again in host memory."""
        if self.agent is None:
            raise ValueError("ExpertSlots.cpu_lane: needs the copy agent (copies='dma')")
        import numpy as np
        keep, exps = [], (L.CpuExpert * (self.L * self.E))()
        copies = {}
        for li, t in enumerate(self.layers):
            src = None
            if copy and t.arena.device.type == "cpu":
                key = t.arena.data_ptr()
                if key not in copies:
                    a = t.arena.numpy()
                    c = np.empty(a.shape, a.dtype)
                    np.copyto(c, a)
                    copies[key] = c
                src = copies[key]
            for e in range(t.E):
                h = t.host_expert(e)
                tr = h["tr"]
                if src is not None:
                    offs = (0, t.off_u, t.off_d)
                    tr = [src[e, offs[m]:offs[m] + t.mat_bytes(e, m)] for m in range(3)]
                arrs = [np.ascontiguousarray(a) for a in tr] + \
                       [np.ascontiguousarray(v, dtype=np.float16) for v in h["suh"] + h["svh"]]
                keep.append(arrs)
                ce = exps[li * self.E + e]
                for m in range(3):
                    ce.tr[m] = arrs[m].ctypes.data
                    ce.suh[m] = arrs[3 + m].ctypes.data
                    ce.svh[m] = arrs[6 + m].ctypes.data
                    ce.fmt[m] = int(h["fmt"][m])
        self._cpu_keep = (keep, exps, copies)
        d = self.layers[0].desc(topk, self.first, act, gated, act_limit)
        L.check(L.lib().bmx_copy_agent_cpu_lane(self.agent, ctypes.byref(d), exps, int(threads)),
                "bmx_copy_agent_cpu_lane")
        self.cpu_ready = True

    def step_planned(self, li, sel, w, x=None, admit=True, *, first=None, bsz=None):
        """A planned step of layer li (bmx_slot_step_planned): publishes the call to the agent's planner, waits for its
        reply and applies it. sel int64 [T, topk], w fp16 [T, topk] (device), x fp16 [T, H] (the call's rows, for the
        CPU lane) or None; bsz: T, required when sel is not two-dimensional (a flattened [T * topk] selection). Returns
        (sel_gpu, w_gpu, lanes, seq): the selection the GPU computes, each pick's lane, and the step's sequence number
        (for cpu_add)."""
        if bsz is not None:
            T = int(bsz)
            if T <= 0 or sel.numel() % T:
                raise ValueError(f"ExpertSlots.step_planned: {sel.numel()} picks are not bsz = {T} tokens of topk")
        elif sel.dim() == 2:
            T = sel.shape[0]
        else:
            raise ValueError("ExpertSlots.step_planned: sel must be [T, topk], or pass bsz with a flattened selection")
        topk = sel.numel() // T
        if w.numel() != sel.numel():
            raise ValueError("ExpertSlots.step_planned: w must hold one weight per pick")
        sel = sel.reshape(-1)
        if sel.dtype != torch.int64 or not sel.is_contiguous():
            sel = sel.long().contiguous()
        w = w.reshape(-1)
        if w.dtype != torch.float16 or not w.is_contiguous():
            w = w.half().contiguous()
        if x is not None:
            x = x.reshape(T, -1)
            if x.dtype != torch.float16 or not x.is_contiguous():
                x = x.half().contiguous()
            self._x_keep = x
        first = self.first if first is None else int(first)
        sel_gpu, w_gpu = torch.empty_like(sel), torch.empty_like(w)
        lanes = torch.empty(sel.numel(), dtype=torch.int32, device=sel.device)
        q = ctypes.c_int64()
        P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
        L.check(L.lib().bmx_slot_step_planned(ctypes.byref(self.struct), self.agent, li, P(sel), P(w), T, topk,
                                              int(first), int(admit), P(x), P(sel_gpu), P(w_gpu), P(lanes),
                                              ctypes.byref(q), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                "bmx_slot_step_planned")
        self.seq[li] = q.value
        self.last_seq = max(self.last_seq, q.value)
        return sel_gpu, w_gpu, lanes, q.value

    def cpu_add(self, seq, out):
        """out [T, H] fp32 += the CPU lane's partial of planned step seq (bounded wait for its job; nothing without one)."""
        L.check(L.lib().bmx_cpu_lane_add(self.agent, int(seq), ctypes.c_void_p(out.data_ptr()), out.shape[0],
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "bmx_cpu_lane_add")
        return out

    def desc(self, li, topk, first=0, act=L.ACT_SILU, gated=True, act_limit=0.0, shared_gate=None):
        return self.layers[li].desc(topk, first, act, gated, act_limit, fresh=self.fresh, shared_gate=shared_gate)

    def warm(self, li, experts):
        """Admit the given local experts of layer li (steps over maxj of them at a time) and wait for their copies."""
        experts = list(experts)
        for i in range(0, len(experts), max(1, self.maxj)):
            sel = torch.as_tensor(experts[i:i + self.maxj], dtype=torch.int64, device=self.arena.device) + self.first
            self.step(li, sel, True)
            self.wait_copies(li)

    def stage_async(self, src, dst, nbytes, stream=None):
        """Host-planned staging: copies src[i] -> dst[i] of nbytes[i] bytes (addresses) with hipMemcpyAsync."""
        n = len(src)
        a = (ctypes.c_void_p * n)(*src)
        b = (ctypes.c_void_p * n)(*dst)
        c = (ctypes.c_size_t * n)(*nbytes)
        s = stream or torch.cuda.current_stream()
        L.check(L.lib().bmx_slot_stage_async(a, b, c, n, ctypes.c_void_p(s.cuda_stream)), "bmx_slot_stage_async")

    # ---- staged prefill ----
    def stage_prefill(self, li, sel, *, first=None):
        """The slot table's part of a prefill-size layer call (engine/nv2.py:378-386 with the staging hook of
        engine/tiers.py:406-463): returns False (and ends an open staged forward) when sel holds fewer than stage_min
        picks. Otherwise marks the hits only (a step that admits nothing, the reference's _ec_hits), and makes layer
        li's table point at a staging arena that holds every expert of the layer not resident in a slot: the copies
        home -> arena (li % 2) run on copy streams (BMX_STAGE_STREAMS, 2), enqueued one layer ahead (layer li + 1's go
        into the other arena while layer li computes), and the current stream waits for layer li's. Residency is snapshotted when a forward
        starts (its first staged call, or a call to a layer at or before the last one; this synchronises), and stays as
        it is because staged calls admit nothing. After the layer's expert products, stage_restore(li) points the
        entries back. The shared expert is not in the slot table and is read where it lives."""
        if sel.numel() < self.stage_min:
            if self.st_open:
                self.stage_end()
            return False
        if not self.st_open or self.st_last is None or li <= self.st_last or li not in self.st_layers:
            self._stage_begin(li)
        self.step(li, sel.reshape(-1), admit=False, first=first)
        cur = torch.cuda.current_stream()
        if li not in self.st_sub:
            self._stage_submit(li)
        b = li % 2
        for ev in self.st_ready[b]:
            cur.wait_event(ev)
        ex, idx, runs = self.st_layers[li]
        if len(ex):
            L.check(L.lib().bmx_slot_stage_rows(ctypes.byref(self.struct), li, ctypes.c_void_p(idx.data_ptr()),
                                                len(ex), self.st_buf[b].data_ptr(), 0, ctypes.c_void_p(cur.cuda_stream)),
                    "bmx_slot_stage_rows")
        if li + 1 in self.st_layers and li + 1 not in self.st_sub:
            self._stage_submit(li + 1)            # the next layer into the other arena, behind this layer's products
        self.st_last = li
        self.st_stats["layers"] += 1
        self.st_stats["experts"] += len(ex)
        return True

    def stage_restore(self, li):
        """After a staged call's expert products (stream order): layer li's staged entries back at their homes."""
        if li not in self.st_layers:
            return
        ex, idx, _ = self.st_layers[li]
        if len(ex):
            L.check(L.lib().bmx_slot_stage_rows(ctypes.byref(self.struct), li, ctypes.c_void_p(idx.data_ptr()),
                                                len(ex), 0, 1, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                    "bmx_slot_stage_rows")

    def stage_end(self):
        """Close a staged forward (the next prefill-size call snapshots residency again). The arenas are kept."""
        self.st_open, self.st_last, self.st_sub = False, None, set()

    def stage_release(self):
        """Close a staged forward and free the staging arenas."""
        self.stage_end()
        self.st_buf, self.st_ready = [None, None], [[], []]

    def _stage_begin(self, li0):
        """A staged forward from layer li0: wait for every copy in flight, snapshot residency, plan each later layer's
        copies (home -> staging record j of its j-th non-resident expert; the matrices a record holds, merged into one
        copy where they are adjacent at both ends), size the arenas."""
        import numpy as np
        self.stage_end()
        cur = torch.cuda.current_stream()
        if self.agent is not None:
            self.check()
            if self.last_seq:
                L.check(L.lib().bmx_copy_wait(self.agent, int(self.last_seq), 1, ctypes.c_void_p(cur.cuda_stream)),
                        "bmx_copy_wait")
        else:
            for ev in [self.last_copied] + list(self.pf_copied):
                if ev is not None:
                    cur.wait_event(ev)
        snap = self.slotof.view(self.L, self.E).cpu().numpy()       # synchronises
        dev = self.arena.device
        self.st_layers, nmax = {}, 0
        for lj in range(li0, self.L):
            t = self.layers[lj]
            ex = np.flatnonzero(snap[lj] < 0).astype(np.int32)
            base, offs, runs = t.arena.data_ptr(), (0, t.off_u, t.off_d), []
            for j, e in enumerate(ex.tolist()):
                for m in range(3):
                    src, dst, nb = base + e * t.rec + offs[m], j * t.rec + offs[m], t.mat_bytes(e, m)
                    if runs:
                        s0, d0, n0 = runs[-1]
                        gap = src - (s0 + n0)
                        if gap == dst - (d0 + n0) and 0 <= gap <= 4096:
                            runs[-1] = (s0, d0, src + nb - s0)
                            continue
                    runs.append((src, dst, nb))
            self.st_layers[lj] = (ex, torch.from_numpy(ex).to(dev), runs)
            nmax = max(nmax, len(ex))
        need = nmax * self.layers[0].rec
        while len(self.cstreams) < max(1, self.stage_streams):
            self.cstreams.append(torch.cuda.Stream(device=dev))
        for b in range(2):
            if self.st_buf[b] is None or self.st_buf[b].numel() < need:
                self.st_buf[b] = None
                buf = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
                for cs in self.cstreams:
                    buf.record_stream(cs)
                self.st_buf[b] = buf
        self.st_open = True
        self.st_stats["forwards"] += 1

    def _stage_submit(self, lj):
        """Enqueue layer lj's staging copies into arena lj % 2 on the copy streams (run i on stream i % streams),
        behind everything the current stream has enqueued so far (the products of the layer that last read that arena,
        and its restore)."""
        b = lj % 2
        _, _, runs = self.st_layers[lj]
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream())
        base = self.st_buf[b].data_ptr()
        ready = []
        for k, cs in enumerate(self.cstreams):
            cs.wait_event(ev)
            part = runs[k::len(self.cstreams)]
            if part:
                n = len(part)
                src = (ctypes.c_void_p * n)(*[r[0] for r in part])
                dst = (ctypes.c_void_p * n)(*[base + r[1] for r in part])
                nb = (ctypes.c_size_t * n)(*[r[2] for r in part])
                L.check(L.lib().bmx_slot_stage_async(src, dst, nb, n, ctypes.c_void_p(cs.cuda_stream)),
                        "bmx_slot_stage_async")
            done = torch.cuda.Event()
            done.record(cs)
            ready.append(done)
        self.st_stats["bytes"] += sum(r[2] for r in runs)
        self.st_ready[b] = ready
        self.st_sub.add(lj)

    def stats(self):
        """(hits, misses, admissions, steps without a victim, evictions, prefetch admissions, prefetched experts used,
        prefetched experts evicted unused) (synchronises)."""
        return tuple(int(v) for v in self.stats_t.cpu())

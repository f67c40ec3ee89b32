#!/usr/bin/env python3
"""MoE layer benchmark on one MI355X.

A step is one pass of the hot path over one batch of synthetic input: router (fp16 logits -> top-k), dispatch, gate/up
products + epilogue, down products + combine (one bmx_moe_layer call). The default run measures, in one process:
  decode     the GLM-shaped layer (288 routed experts, top-8 sigmoid + bias, one shared expert, H 4096, I 1536, EXL3
             3 bpw) on 1 decode token: the headline `value` (bandwidth-bound GEMV path, roofline against HBM)
  prefill    the DeepSeek-shaped layer (384 experts, group-limited top-6, H 4096, I 2048, EXL3 2 / 3 bpw, Zipf routing)
             on an 8192-token chunk (MFMA path, roofline against fp16 MFMA): the `prefill` object
  decode_t8, c1, c5: the GLM-shaped layer on 8 tokens, the 64-expert layer on 1 token, and the 16-token speculative
             verify batch on the DeepSeek shape
Decode steps rotate over input batches (the c1 leg also over 32 layer tables) so each step reads other experts than
the steps before it, as a layer of a model does between two of its calls: the weights are not left in the Infinity
Cache. Inputs and all experts are resident in HBM before the timed region. The reference's CPU lane is timed on the
same routes for the decode and prefill legs (one thread per physical core of the GPU's NUMA node, and one core).
Prints one JSON line. --config cN [--tokens T] runs one workload instead; --config c4 the 43-layer slot-table stack.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--legs decode,prefill,...] [--config c2] [--tokens T] [--no-cpu]
"""
import argparse
import ctypes
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "big-moe-small-box_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MoE layer µs/token (decode) + prefill tok/s; HBM GB/s & MFMA util vs peak"
HBM_PEAK_GBPS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0     # MI355X dense fp16 MFMA


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class TimingEvent:
    """A HIP event for timing only, created with hipEventDisableSystemFence: recording it skips the system-scope release
    (an L2 writeback) that a default event performs, which costs microseconds of GPU time per record and would be
    counted into a microsecond-scale kernel between two records. Elapsed times are read after a device synchronize."""
    _hip = None

    @classmethod
    def hip(cls):
        if cls._hip is None:
            # the HIP runtime this process already runs (torch's; the library resolves to the same one)
            path = next((l.split()[-1] for l in open("/proc/self/maps") if "libamdhip64" in l), "libamdhip64.so")
            h = ctypes.CDLL(path)
            h.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
            h.hipEventDestroy.argtypes = [ctypes.c_void_p]
            cls._hip = h
        return cls._hip

    def __init__(self):
        self.ev = ctypes.c_void_p()
        rc = self.hip().hipEventCreateWithFlags(ctypes.byref(self.ev), 0x20000000)   # hipEventDisableSystemFence
        if rc:
            raise RuntimeError(f"hipEventCreateWithFlags: error {rc}")

    def record(self, stream):
        rc = self._hip.hipEventRecord(self.ev, stream)
        if rc:
            raise RuntimeError(f"hipEventRecord: error {rc}")

    def elapsed_time(self, end):
        ms = ctypes.c_float()
        rc = self._hip.hipEventElapsedTime(ctypes.byref(ms), self.ev, end.ev)
        if rc:
            raise RuntimeError(f"hipEventElapsedTime: error {rc}")
        return ms.value

    def __del__(self):
        if self._hip is not None and self.ev:
            self._hip.hipEventDestroy(self.ev)


def physical_cpus(limit):
    """CPUs of this process, one per physical core first (the reference's lane rule: one lane thread per core)."""
    allowed = sorted(os.sched_getaffinity(0))
    first, sib, seen = [], [], set()
    for c in allowed:
        try:
            core = open(f"/sys/devices/system/cpu/cpu{c}/topology/core_id").read().strip()
            pkg = open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id").read().strip()
        except OSError:
            core, pkg = str(c), "0"
        if (pkg, core) in seen:
            sib.append(c)
        else:
            seen.add((pkg, core))
            first.append(c)
    return (first + sib)[:limit], len(first)


def gpu_numa_cpus():
    """(node, physical-core CPUs of the GPU's NUMA node that this process may use): the node from the GPU's PCI device
    (node 0 when the platform reports none, as a one-node guest does)."""
    import torch
    node = -1
    try:
        p = torch.cuda.get_device_properties(0)
        bdf = f"{p.pci_domain_id:04x}:{p.pci_bus_id:02x}:{p.pci_device_id:02x}.0"
        node = int(open(f"/sys/bus/pci/devices/{bdf}/numa_node").read().strip())
    except (OSError, ValueError, AttributeError):
        pass
    nodes = sorted(int(d[4:]) for d in os.listdir("/sys/devices/system/node") if d.startswith("node") and d[4:].isdigit()) \
        if os.path.isdir("/sys/devices/system/node") else [0]
    if node < 0:
        node = nodes[0] if nodes else 0
    cpus = set(os.sched_getaffinity(0))
    try:
        spec = open(f"/sys/devices/system/node/node{node}/cpulist").read().strip()
        node_cpus = set()
        for part in spec.split(","):
            a, _, b = part.partition("-")
            node_cpus |= set(range(int(a), int(b or a) + 1))
        cpus &= node_cpus
    except OSError:
        pass
    phys, _ = physical_cpus(1 << 30)
    return node, [c for c in phys if c in cpus]


def cpu_model():
    """The host CPU as /proc/cpuinfo names it, with family / model / stepping (a virtual machine may report only the
    vendor line, e.g. "AMD EPYC"; family 26 is AMD Zen 5)."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if not line.strip():
                break
            k, _, v = line.partition(":")
            info[k.strip()] = v.strip()
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    fam = info.get("cpu family")
    gen = {"25": " (Zen 3 / Zen 4)", "26": " (Zen 5)"}.get(fam, "") if info.get("vendor_id") == "AuthenticAMD" else ""
    virt = ", virtual machine" if "hypervisor" in info.get("flags", "").split() else ""
    return f"{name} family {fam} model {info.get('model')} stepping {info.get('stepping')}{gen}{virt}"


def _lane_median(R, T, x, si, wf, k, out, mode, budget_s, min_calls):
    times = []
    t_end = time.perf_counter() + budget_s
    for i in range(100000):
        t0 = time.perf_counter()
        R.ref_lane_forward(x.ctypes.data, T, si.ctypes.data, wf.ctypes.data, k, out.ctypes.data, mode)
        times.append(time.perf_counter() - t0)
        if (i + 1 >= min_calls and time.perf_counter() > t_end) or time.perf_counter() > t_end + budget_s:
            break
    warm = times[max(1, len(times) // 10):] if len(times) > 3 else times
    return statistics.median(warm), len(times)


def cpu_baseline(tab, sel, w, budget_s=8.0):
    """The reference's CPU lane (ft_n135.h moe_forward4, built from the reference sources into oracle/_ref) on the same
    routes (sel / w: the routes of the bounded sample, the first tokens of the timed batch), driven as the reference's
    cpu_forward drives it (nv2_host.cpp:1974-2003): experts in RAM, routes given (no router), mode auto (I16 when an
    expert of the sample has a format other than K 3), the shared expert as a weight-1 job. Timed with one thread per
    physical core of the GPU's NUMA node (the reference's lane rule, cpus.py:50-65, capped at 16: the GPU's share of
    the host) and with one thread on one core; median of warm calls, whole-call wall time."""
    import numpy as np
    from oracle import oracle as O
    R = O.ref_lane()
    if R is None:
        return None
    node, node_cpus = gpu_numa_cpus()
    cpus = node_cpus[:16]
    E1 = tab.E + (1 if tab.has_shared else 0)
    sel = sel.cpu().numpy()
    w = w.float().cpu().numpy()
    T, k = sel.shape
    if tab.has_shared:
        sel = np.concatenate([sel, np.full((T, 1), tab.E, np.int64)], 1)
        w = np.concatenate([w, np.ones((T, 1), np.float32)], 1)
        k += 1
    tf = {0: 0, 1: 1, 2: 2}
    mode = -1
    proxy = False
    prng = np.random.default_rng(1)
    experts = {}
    for e in sorted(set(sel.ravel().tolist())):
        ex = tab.host_expert(e)
        if any(f not in tf for f in ex["fmt"]):
            # the lane has no K 4 (ft_n135.h:82): time K 3 experts of the same shapes, random codes, same scales
            proxy = True
            for m, (kin, nout) in enumerate(((tab.H, tab.I), (tab.H, tab.I), (tab.I, tab.H))):
                if ex["fmt"][m] not in tf:
                    ex["tr"][m] = prng.integers(0, 256, (kin // 16) * (nout // 16) * 96, dtype=np.uint8)
                    ex["fmt"][m] = 2
        if any(f != 2 for f in ex["fmt"]):
            # formats other than K 3 decode only in the I16 (p16 VBMI) kernel; the reference switches to it when the
            # first job's expert has one (ft_n135.h:933-936), a layer of mixed formats needs it for every call
            mode = 2
        experts[e] = ex
    x = np.random.default_rng(0).standard_normal((T, tab.H)).astype(np.float16).astype(np.float32)
    si = np.ascontiguousarray(sel.astype(np.int32))
    wf = np.ascontiguousarray(w)
    out = np.zeros((T, tab.H), np.float32)
    res = {}
    for label, use in (("node", cpus), ("one_core", cpus[:1])):
        arr = (ctypes.c_int * len(use))(*use)
        if R.ref_lane_create(tab.H, tab.I, E1, len(use), arr, 0.0) != 0:
            return None
        keep = []
        try:
            for e, ex in experts.items():
                sc = [ex["suh"][0], ex["svh"][0], ex["suh"][1], ex["svh"][1], ex["suh"][2], ex["svh"][2]]
                sc = [np.ascontiguousarray(a.view(np.uint16)) for a in sc]
                keep += ex["tr"] + sc
                R.ref_lane_set_expert(e, *[t.ctypes.data for t in ex["tr"]], *[a.ctypes.data for a in sc], *ex["fmt"])
            med, n = _lane_median(R, T, x, si, wf, k, out, mode, budget_s, 20 if label == "node" else 5)
        finally:
            R.ref_lane_destroy()
        res[label] = (med, n, len(use))
        log(f"bench: cpu baseline {label}: {len(use)} threads, {n} calls, median {med * 1e6:.0f} us")
    med, n, nt = res["node"]
    med1, n1, _ = res["one_core"]
    return {"value": T / med, "unit": "tokens/s", "cores": nt, "kind": "reference",
            "sample": f"one {T}-token layer call (the routes of the first {T} tokens of the timed batch, {k} jobs per "
                      f"token{' incl. the shared expert' if tab.has_shared else ''}); median wall time of {n} warm calls "
                      f"{med * 1e6:.0f} us with {nt} threads pinned one per physical core of the GPU's NUMA node {node}, "
                      f"{n1} calls {med1 * 1e6:.0f} us on one core; moe_forward4 mode {'I16' if mode == 2 else 'auto'}"
                      f"{'; K 3 proxy of the K 4 experts (the reference lane has no K 4)' if proxy else ''}",
            "one_core": {"value": T / med1, "unit": "tokens/s", "cores": 1},
            "cpu_model": cpu_model(), "numa_node": node, "node_physical_cores": len(node_cpus),
            "us_per_layer": med * 1e6, "us_per_layer_one_core": med1 * 1e6}


def bench_c4(args):
    """43 layers of the GLM-shaped layer in decode (batch 1) with the expert-slot table: routed experts at home in pinned
    host memory, a VRAM cache of 30 % of them warmed with each layer's most popular experts, Zipf(1.1) routing with a
    per-layer permutation over a cycle of synthetic tokens. A step is one token through the 43 layers: router, slot step
    (copies of admissions on a side stream), dispatch, gate / up of resident experts, gate / up of staged experts after
    their copies, epilogue, down of resident experts, down of staged experts after their copies, combine."""
    import numpy as np
    import torch
    import bmx
    from bmx import synth
    dev = torch.device("cuda:0")
    c = synth.CONFIGS["c4"]
    NL, E, H, I, topk = c["layers"], c["E"], c["H"], c["I"], c["topk"]
    NTOK = 64
    S = int(round(c["cache_frac"] * NL * E))
    log(f"bench c4: {NL} layers x {E} experts, homes in pinned host memory, {S} VRAM slots")
    layers, biases, lgs = [], [], []
    rng = np.random.default_rng(0)
    NH = 16      # distinct pinned home arenas (2 GB each); layer li reads the trellis bytes of layer li % NH
    for li in range(NL):
        if li < NH:
            t = bmx.ExpertTable.random(H, I, E, synth.formats("c4", E, True), shared=True, seed=1000 + li, device=dev,
                                       home="host")
        else:
            h = layers[li % NH]
            t = bmx.ExpertTable(H, I, h.arena, h.fmt, h.suh, h.svh, h.off_u, h.off_d, E, True)
        t.shared_to_device()
        layers.append(t)
        biases.append(torch.from_numpy((rng.standard_normal(E) * 0.1).astype(np.float32)).to(dev))
        lgs.append(synth.zipf_logits(NTOK, E, 1.1, seed=li, perm_seed=7919 * (li + 1)))
        if li % 8 == 0:
            log(f"bench c4: layer {li} built")
    lg_all = torch.from_numpy(np.stack(lgs)).to(dev)            # [NL, NTOK, E] fp16
    PF = args.prefetch
    AH = args.prefetch_ahead if args.copies == "dma" else 1
    if PF:
        # layer-ahead guesses: layer li routes its logits plus noise (a stand-in for its router on the previous layer's
        # MoE input); routed inside the timed region like the real picks
        noise = np.random.default_rng(99).standard_normal((NL, NTOK, E)).astype(np.float32) * args.guess_noise
        lg_guess = torch.from_numpy((np.stack(lgs).astype(np.float32) + noise).astype(np.float16)).to(dev)
        gsel = torch.empty((1, topk), dtype=torch.int64, device=dev)
        gw = torch.empty((1, topk), dtype=torch.float16, device=dev)
        pf_copied = [None, None]
        pf_admitted = [torch.cuda.Event() for _ in range(NL)]
    slots = bmx.ExpertSlots(layers, S, maxj=16, copies=args.copies)
    DMA = args.copies == "dma"
    CPUL = args.cpu_lane > 0 and DMA
    FUSED = not CPUL and not args.separate_route_step     # routing + slot step in one launch (bmx_route_slot_step)
    if CPUL:
        # planned steps: the agent's planner puts misses on the CPU lane (fast mode, args.cpu_lane worker threads, reading
        # its own huge-page copy of the homes) when its estimated finish is no later than the GPU's; the GPU costs are
        # measured per-expert times of this stack, the CPU's is measured (seeded when the lane is set up, then the
        # worker's running mean per pick)
        slots.cpu_lane(topk, threads=args.cpu_lane, copy=True)
        slots.plan(dict(cpu_on=1, max_cpu=args.cpu_max, cpu_fast=1, cpu_measured=1, gpu_base_us=50.0, gpu_hit_us=0.0,
                        gpu_admit_us=140.0, cpu_base_us=10.0, cpu_expert_us=args.cpu_expert_us, cpu_token_us=60.0))
    # warm: each layer's most popular experts (Zipf rank order of its permutation), S // NL per layer
    per = S // NL
    for li in range(NL):
        perm = np.random.default_rng(7919 * (li + 1)).permutation(E)
        slots.warm(li, [int(e) for e in perm[:per]])
    torch.cuda.synchronize()
    h0 = slots.stats()
    log(f"bench c4: warmed, stats {h0}")

    L = bmx.lib()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float16)).to(dev)
    descs = [slots.desc(li, topk) for li in range(NL)]
    sel = torch.empty((1, topk), dtype=torch.int64, device=dev)
    w = torch.empty((1, topk), dtype=torch.float16, device=dev)
    sel_g, w_g = torch.empty_like(sel), torch.empty_like(w)          # planned steps: the picks the GPU computes
    out = torch.empty((NL, H), dtype=torch.float32, device=dev)
    rpg = L.bmx_rows_per_group(1, topk, 1)
    routes = bmx.ops.RoutesBuf(1, topk, E, True, rpg, dev)
    dws_n = L.bmx_dispatch_workspace(1, topk, E)
    dws = torch.empty(max(dws_n, 1), dtype=torch.uint8, device=dev)
    ws_n = L.bmx_experts_workspace(ctypes.byref(descs[0]), 1, 1)
    ws = torch.zeros(ws_n, dtype=torch.uint8, device=dev)
    stepped = [torch.cuda.Event() for _ in range(NL)]
    copied_gu = [torch.cuda.Event() for _ in range(NL)]
    copied_dn = [torch.cuda.Event() for _ in range(NL)]
    side = slots.side
    tstruct = ctypes.byref(slots.struct)
    seq, pseq, seqs = ctypes.c_int64(), ctypes.c_int64(), [0] * NL

    # timeline phases of a layer call (the reference's per-layer split, engine/nv2.py:836-901): an event before each
    PHASES = ("route", "step", "dispatch", "moe_resident", "copy_wait_gate_up", "moe_staged_act_down_resident",
              "copy_wait_down", "down_staged_combine", "cpu_add")

    def token(tok, evs=None):
        s = torch.cuda.current_stream()
        sp = ctypes.c_void_p(s.cuda_stream)
        mark = (lambda li, k: evs[li][k].record(sp)) if evs is not None else (lambda li, k: None)
        for li in range(NL):
            mark(li, 0)
            lgp = ctypes.c_void_p(lg_all.data_ptr() + (li * NTOK + tok) * E * 2)
            if FUSED:
                # the routing and the step in one launch: the route phase holds both, the step phase reads ~0
                bmx._lib.check(L.bmx_route_slot_step(tstruct, slots.agent if DMA else None, li, lgp, P(biases[li]), E,
                                                     topk, 1, 1, c["score"], 1, c["scale"], 0, 1, P(sel), P(w),
                                                     ctypes.byref(seq), sp), "route + slot step")
                mark(li, 1)
                if DMA:
                    seqs[li] = seq.value
            else:
                bmx._lib.check(L.bmx_router_topk(lgp, P(biases[li]), 1, E, topk, 1, 1, c["score"], 1, c["scale"], 0,
                                                 P(sel), P(w), sp), "router")
                mark(li, 1)
            if FUSED and DMA:
                pass
            elif FUSED:
                stepped[li].record(s)
                side.wait_event(stepped[li])
                bmx._lib.check(L.bmx_slot_copy_mats(tstruct, li, 3, ctypes.c_void_p(side.cuda_stream)), "slot copy")
                copied_gu[li].record(side)
                bmx._lib.check(L.bmx_slot_copy_mats(tstruct, li, 4, ctypes.c_void_p(side.cuda_stream)), "slot copy")
                copied_dn[li].record(side)
            elif CPUL:
                bmx._lib.check(L.bmx_slot_step_planned(tstruct, slots.agent, li, P(sel), P(w), 1, topk, 0, 1, P(x),
                                                       P(sel_g), P(w_g), None, ctypes.byref(seq), sp), "planned step")
                seqs[li] = seq.value
            elif DMA:
                bmx._lib.check(L.bmx_slot_step_agent(tstruct, slots.agent, li, P(sel), topk, 0, 1, ctypes.byref(seq),
                                                     sp), "slot step")
                seqs[li] = seq.value
            else:
                bmx._lib.check(L.bmx_slot_step(tstruct, li, P(sel), topk, 0, 1, sp), "slot step")
                stepped[li].record(s)
                side.wait_event(stepped[li])
                bmx._lib.check(L.bmx_slot_copy_mats(tstruct, li, 3, ctypes.c_void_p(side.cuda_stream)), "slot copy")
                copied_gu[li].record(side)
                bmx._lib.check(L.bmx_slot_copy_mats(tstruct, li, 4, ctypes.c_void_p(side.cuda_stream)), "slot copy")
                copied_dn[li].record(side)
            if PF and li + AH < NL and DMA:
                lgq = ctypes.c_void_p(lg_guess.data_ptr() + ((li + AH) * NTOK + tok) * E * 2)
                bmx._lib.check(L.bmx_router_topk(lgq, P(biases[li + AH]), 1, E, topk, 1, 1, c["score"], 1, c["scale"],
                                                 0, P(gsel), P(gw), sp), "guess router")
                bmx._lib.check(L.bmx_slot_prefetch_agent(tstruct, slots.agent, li + AH, P(gsel), topk, 0, PF,
                                                         ctypes.byref(pseq), sp), "slot prefetch")
            elif PF and li + 1 < NL:
                b = li & 1
                lgq = ctypes.c_void_p(lg_guess.data_ptr() + ((li + 1) * NTOK + tok) * E * 2)
                bmx._lib.check(L.bmx_router_topk(lgq, P(biases[li + 1]), 1, E, topk, 1, 1, c["score"], 1, c["scale"], 0,
                                                 P(gsel), P(gw), sp), "guess router")
                if pf_copied[b] is not None:
                    s.wait_event(pf_copied[b])
                bmx._lib.check(L.bmx_slot_prefetch(tstruct, li + 1, P(gsel), topk, 0, PF, b, sp), "slot prefetch")
                pf_admitted[li].record(s)
                side.wait_event(pf_admitted[li])
                bmx._lib.check(L.bmx_slot_prefetch_copy(tstruct, li + 1, b, 7, ctypes.c_void_p(side.cuda_stream)),
                               "prefetch copy")
                ev = torch.cuda.Event()
                ev.record(side)
                pf_copied[b] = ev
            gs, gw_ = (sel_g, w_g) if CPUL else (sel, w)
            mark(li, 2)
            bmx._lib.check(L.bmx_dispatch(P(gs), 1, topk, E, 0, 1, rpg, ctypes.byref(routes.struct), P(dws), dws_n, sp),
                           "dispatch")
            d = ctypes.byref(descs[li])
            o = ctypes.c_void_p(out.data_ptr() + li * H * 4)
            for k, st in enumerate((bmx._lib.STAGE_GATE_UP_RESIDENT, "gu", bmx._lib.STAGE_GATE_UP_STAGED,
                                    bmx._lib.STAGE_ACT, bmx._lib.STAGE_DOWN_RESIDENT, "dn", bmx._lib.STAGE_DOWN_STAGED,
                                    bmx._lib.STAGE_COMBINE)):
                ph = (3, 4, 5, None, None, 6, 7, None)[k]
                if ph is not None:
                    mark(li, ph)
                if isinstance(st, str):
                    if DMA:
                        bmx._lib.check(L.bmx_copy_wait_layer(slots.agent, li, 0 if st == "gu" else 1, sp), "copy wait")
                    else:
                        s.wait_event(copied_gu[li] if st == "gu" else copied_dn[li])
                    continue
                bmx._lib.check(L.bmx_moe_stage(d, st, P(x), 1, ctypes.byref(routes.struct), None, None, P(gw_), o,
                                               P(ws), ws_n, 1, sp), "stage")
            mark(li, 8)
            if CPUL:
                bmx._lib.check(L.bmx_cpu_lane_add(slots.agent, seqs[li], o, 1, sp), "cpu lane add")
            mark(li, 9)

    steps, warmup = (args.steps, args.warmup) if args.config == "c4" else (args.c4_steps, min(args.warmup, 5))
    args = argparse.Namespace(**dict(vars(args), steps=steps, warmup=warmup))
    for i in range(args.warmup):
        token(i % NTOK)
    torch.cuda.synchronize()
    st0 = slots.stats()
    ps0 = slots.plan_stats() if CPUL else None
    t0 = time.perf_counter()
    for i in range(args.steps):
        token((args.warmup + i) % NTOK)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    st1 = slots.stats()
    ps1 = slots.plan_stats() if CPUL else None
    d = [b - a for a, b in zip(st0, st1)]
    exp_bytes = layers[0].expert_bytes(0)
    staged = (d[2] + d[5]) * exp_bytes
    # timeline: the same token loop once more with a timing event before each phase of every layer call (kept out of
    # the timed loop above, whose figure has no events in it)
    nt = max(1, args.timeline_steps)
    evs = [[[TimingEvent() for _ in range(len(PHASES) + 1)] for _ in range(NL)] for _ in range(nt)]
    for i in range(nt):
        token((args.warmup + args.steps + i) % NTOK, evs[i])
    torch.cuda.synchronize()
    parts = {ph: statistics.mean(evs[i][li][k].elapsed_time(evs[i][li][k + 1]) * 1e3 for i in range(nt)
                                 for li in range(NL)) for k, ph in enumerate(PHASES)}
    layer_us = [evs[i][li][0].elapsed_time(evs[i][li][-1]) * 1e3 for i in range(nt) for li in range(NL)]
    timeline = {"n": nt * NL, "tokens": nt, "us_layer_mean": round(sum(parts.values()), 1),
                "parts_us_mean": {k: round(v, 2) for k, v in parts.items()},
                "copy_wait_us_mean": round(parts["copy_wait_gate_up"] + parts["copy_wait_down"], 2),
                "compute_us_mean": round(sum(v for k, v in parts.items() if not k.startswith("copy_wait")), 2),
                "us_layer_p50": round(statistics.median(layer_us), 1) if layer_us else None,
                "timing": "timing-only events (no system-scope release) on the compute stream before each phase of every "
                          "layer call, in a separate loop of the same tokens; copy_wait_* is the time the stream spends "
                          "in the one-lane kernel waiting for the copies of the layer's admissions (the part of the copy "
                          "no compute hides)" + ("; the router and the slot step are one launch, timed as route (step "
                                                 "reads the events' own cost)" if FUSED else "")}
    log(f"bench c4: timeline {timeline['parts_us_mean']}")
    h2d = measure_h2d()
    link = staged / (ms * 1e-3 * args.steps) / 1e9
    roofline = {"kernel": "home -> slot copies of the misses (copy agent, SDMA engines)" if DMA else
                          "home -> slot copies of the misses (copy kernel on a side stream)",
                "bound": "pcie", "achieved": round(link, 2), "peak": round(h2d, 2), "unit": "GB/s",
                "frac": round(link / h2d, 4), "traffic": round(staged / args.steps),
                "peak_source": "one 1 GiB pinned host -> device hipMemcpyAsync timed in this run (PCIe Gen5 x16: 64 GB/s "
                               "per direction published)",
                "floor_us_per_token": round(staged / args.steps / (h2d * 1e9) * 1e6, 1),
                "achieved_source": "misses' expert bytes per token (admissions + prefetches x 7,077,888 B) over the timed "
                                   "loop's time per token"}
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(layers[0], sel.repeat(4, 1), w.repeat(4, 1),
                           budget_s=args.cpu_budget if args.config == "c4" else min(4.0, args.cpu_budget))
        if cpu:
            per_layer = cpu["us_per_layer"] / 4
            cpu = {"value": round(1e6 / (per_layer * NL), 3), "unit": "tokens/s", "cores": cpu["cores"], "kind": "reference",
                   "sample": f"one c4 layer's call on 4 tokens (routes of the last timed token), {cpu['sample']}; "
                             f"per token x {NL} layers"}
    res = {
        "metric": METRIC, "value": round(1e3 / ms, 3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16",
        "data": f"synthetic: random EXL3 3 bpw trellis codes, homes of routed experts in pinned host memory ({NH} distinct "
                f"2 GB arenas, layer li reading those of layer li % {NH}: the box pins about 55 GB), suh ~ U(0.5,1.5), "
                "svh ~ U(0.5,1.5)/sqrt(k), x ~ N(0,1) fp16, router logits = Zipf(1.1) log-popularity of a per-layer "
                f"permutation + Gumbel noise over a cycle of {NTOK} tokens, bias ~ N(0,0.1); seed 0",
        "config": {"workload": f"c4 decode stack: {NL} layers of {E} routed experts top-{topk} sigmoid+bias + 1 shared (in "
                               f"VRAM), H {H}, I {I}, EXL3 3 bpw; expert-slot table of {S} VRAM slots (30 %) warmed with each "
                               f"layer's top {per} experts by popularity", "tokens": 1, "layers": NL, "path": "decode",
                   "step": "per layer: router + slot step" + (" (one launch)" if FUSED else "") + " (copies "
                           + ("by the copy agent on the DMA engines" if DMA else "on a side stream") + ") + "
                           + (f"guess of layer li + {AH} (router on noisy logits) + slot prefetch of up to {PF} + "
                              if PF else "")
                           + "dispatch + gate/up (resident, then staged) + down (resident, then staged) + combine"},
        "us_per_token": round(ms * 1e3, 3), "us_per_layer": round(ms * 1e3 / NL, 3),
        "slot_stats_per_token": {"hits": d[0] / args.steps, "misses": d[1] / args.steps, "admitted": d[2] / args.steps,
                                 "no_victim": d[3] / args.steps, "evictions": d[4] / args.steps,
                                 "prefetched": d[5] / args.steps, "prefetch_used": d[6] / args.steps,
                                 "prefetch_wasted": d[7] / args.steps},
        "copies": args.copies,
        "cpu_lane": {"threads": args.cpu_lane, "max_cpu": args.cpu_max, "cpu_expert_us": args.cpu_expert_us,
                     "cpu_experts_per_token": (ps1[1] - ps0[1]) / args.steps,
                     "cpu_jobs_per_token": (ps1[2] - ps0[2]) / args.steps,
                     "cpu_job_us": round((ps1[3] - ps0[3]) / max(1, ps1[2] - ps0[2]), 1),
                     "cpu_pick_us_measured": round(ps1[4] / 1e3, 1)} if CPUL else None,
        "prefetch": {"limit": PF, "guess_noise": args.guess_noise, "ahead": AH,
                     "precision": round(d[6] / max(1, d[5]), 4)} if PF else None,
        "hit_rate": round(d[0] / max(1, d[0] + d[1]), 4),
        "staged_bytes_per_token": staged / args.steps,
        "staged_gbps": round(staged / (ms * 1e-3 * args.steps) / 1e9, 2),
        "timeline": timeline,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if DMA:
        log(f"bench c4: copy agent {slots.agent_status()}")
        slots.close()
    return res


def measure_h2d(nbytes=1 << 30, reps=3):
    """Pinned host -> device copy rate (GB/s, best of reps) of one nbytes hipMemcpyAsync on a side stream."""
    import torch
    src = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    side = torch.cuda.Stream()
    best = 0.0
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(side):
            a.record()
            dst.copy_(src, non_blocking=True)
            b.record()
        b.synchronize()
        best = max(best, nbytes / (a.elapsed_time(b) * 1e-3) / 1e9)
    del src, dst
    return best


def bench_staged(args, cpu=None):
    """Staged prefill of the DeepSeek-shaped layer with its experts at home in pinned host memory: NL layers (their homes
    in NH distinct arenas, layer li reading the bytes of arena li % NH), a VRAM slot table of 30 % of the experts warmed
    with each layer's most popular ones, Zipf(1.1) routing with a per-layer permutation, 8192-token chunks. A step is one
    chunk through the NL layers: per layer the router, the hits-only slot step with the staging of every non-resident
    expert one layer ahead (ExpertSlots.stage_prefill: copies into two staging arenas on a copy stream), the layer's
    products and combine, the table restore. Bound: the PCIe link (the non-resident experts' bytes cross it once)."""
    import numpy as np
    import torch
    import bmx
    from bmx import synth
    dev = torch.device("cuda:0")
    c = synth.CONFIGS["c3"]
    NL, NH, E, H, I, topk, T = args.staged_layers, min(4, args.staged_layers), c["E"], c["H"], c["I"], c["topk"], c["T"]
    S = int(round(0.30 * NL * E))
    log(f"bench prefill_staged: {NL} layers x {E} experts (homes: {NH} pinned arenas), {S} VRAM slots, {T} tokens")
    fm = synth.formats("c3", E, False)
    layers = []
    for li in range(NL):
        if li < NH:
            t = bmx.ExpertTable.random(H, I, E, fm, seed=3000 + li, device=dev, home="host")
        else:
            h = layers[li % NH]
            t = bmx.ExpertTable(H, I, h.arena, h.fmt, h.suh, h.svh, h.off_u, h.off_d, E, False)
        layers.append(t)
    slots = bmx.ExpertSlots(layers, S, maxj=16, copies="kernel")
    kw = dict(score=c["score"], renorm=c["renorm"], scale=c["scale"], n_group=c["n_group"], topk_group=c["topk_group"])
    mods = [bmx.MoELayer(layers[li], topk, slots=slots, li=li, **kw) for li in range(NL)]
    per = S // NL
    lgs = []
    for li in range(NL):
        perm = np.random.default_rng(7000 + li).permutation(E)
        slots.warm(li, [int(e) for e in perm[:per]])
        lgs.append(torch.from_numpy(synth.zipf_logits(T, E, 1.1, seed=7000 + li)).to(dev))
    x = torch.from_numpy(np.random.default_rng(0).standard_normal((T, H)).astype(np.float16)).to(dev)
    torch.cuda.synchronize()

    def forward():
        for li, m in enumerate(mods):
            sel, w = m.routing_fn(T, None, x, {"logits": lgs[li]})
            sel, w, _ = m.layer(li, sel, w, x, T)
            m.run_bszN(x, sel, w)

    steps, warmup = max(1, args.staged_steps), 1
    for _ in range(warmup):
        forward()
    torch.cuda.synchronize()
    st0 = dict(slots.st_stats)
    t0 = time.perf_counter()
    for _ in range(steps):
        forward()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    st1 = dict(slots.st_stats)
    staged_bytes = (st1["bytes"] - st0["bytes"]) / steps
    staged_experts = (st1["experts"] - st0["experts"]) / steps
    h2d = measure_h2d()
    link = staged_bytes / (ms * 1e-3) / 1e9
    us_layer = ms * 1e3 / NL
    res = {
        "workload": f"c3 staged prefill: {NL} layers of {E} routed experts top-{topk} group-limited (8 groups, top-4), "
                    f"H {H}, I {I}, EXL3 2/3 mixed, {T} tokens per chunk; routed experts at home in pinned host memory "
                    f"({NH} distinct arenas), a VRAM slot table of {S} slots (30 %) warmed with each layer's top {per} "
                    f"experts; every non-resident expert staged into one of two arenas one layer ahead",
        "T": T, "layers": NL, "steps": steps, "warmup": warmup, "path": "prefill (staged)",
        "value": round(T * 1e3 / (ms / NL), 2), "unit": "tokens/s",
        "us_per_layer": round(us_layer, 1), "ms_per_chunk": round(ms, 3),
        "staged_experts_per_layer": round(staged_experts / NL, 1),
        "staged_bytes_per_layer": round(staged_bytes / NL),
        "roofline": {"kernel": "home -> staging arena copies (hipMemcpyAsync on a copy stream, one layer ahead)",
                     "bound": "pcie", "achieved": round(link, 2), "peak": round(h2d, 2), "unit": "GB/s",
                     "frac": round(link / h2d, 4), "traffic": round(staged_bytes / NL),
                     "floor_us_per_layer": round(staged_bytes / NL / (h2d * 1e9) * 1e6, 1),
                     "peak_source": "one 1 GiB pinned host -> device hipMemcpyAsync timed in this run (PCIe Gen5 x16: 64 "
                                    "GB/s per direction published)",
                     "achieved_source": "bytes staged per chunk over the chunk's time (layers computing while the next "
                                        "layer's experts are copied)"},
        "cpu_baseline": cpu,
    }
    log(f"bench prefill_staged: {us_layer:.0f} us per layer, {link:.1f} GB/s staged of {h2d:.1f} GB/s measured H2D")
    slots.close()
    return res


# Legs of the default run: (config, tokens per step, input batches rotated over, distinct layer tables rotated over).
# Decode steps rotate over a pool of token batches (and, for the 151 MB c1 layer, over layer tables) so that the
# experts a step reads change from step to step and the weights do not stay in the 256 MB Infinity Cache: what a model's
# layer sees when the other layers run between two of its calls.
LEGS = {
    "decode": ("c2", 1, 64, 1),
    "prefill": ("c3", 8192, 1, 1),
    "decode_t8": ("c2", 8, 16, 1),
    "c1": ("c1", 1, 64, 32),
    "c5": ("c5", 16, 16, 1),
    "prefill_staged": None,       # bench_staged: the c3 layer stack with its experts in pinned host memory
    "c4": None,                   # bench_c4: the 43-layer decode stack with the expert-slot table
    "c4_cpu_lane": None,          # the same stack with the planner putting misses on a 12-thread CPU lane
}
HEADLINE_LEGS = ("decode", "prefill")


def bench_leg(leg, cfg, T, P, NT, args, with_cpu):
    """Times one workload: `steps` whole-layer calls (bmx_moe_layer: router + dispatch + expert products + combine),
    eager and as one replayed HIP graph, step i on input batch i % P and layer table i % NT; then the same steps one
    stage at a time with events between the stages (the stage times and the roofline)."""
    import numpy as np
    import torch
    import bmx
    from bmx import synth
    dev = torch.device("cuda:0")
    c = synth.CONFIGS[cfg]
    E, topk, H = c["E"], c["topk"], c["H"]
    log(f"bench {leg}: building {NT} x {cfg} table (E={E}, H={H}, I={c['I']}), {P} input batches of {T} tokens")
    tabs = [synth.table(cfg, seed=s, device=dev) for s in range(NT)]
    _, _, bias = synth.inputs(cfg, T=1, seed=0, device=dev)
    xs, lgs = [], []
    for p in range(P):
        x, lg, _ = synth.inputs(cfg, T=T, seed=p, device=dev)
        xs.append(x)
        lgs.append(lg)
    layers = [bmx.MoELayer(t, topk, score=c["score"], bias=bias, n_group=c["n_group"], topk_group=c["topk_group"],
                           renorm=c["renorm"], scale=c["scale"]) for t in tabs]
    torch.cuda.synchronize()
    L = bmx.lib()
    Pp = lambda t: ctypes.c_void_p(t.data_ptr())
    pa = {"auto": 0, "decode": 1, "prefill": 2, "mid": 3, "split": 4}[args.path]
    need = max(L.bmx_moe_layer_workspace(ctypes.byref(l.desc), T, pa) for l in layers)
    lws = torch.zeros(need, dtype=torch.uint8, device=dev)
    sel_b = torch.empty((T, topk), dtype=torch.int64, device=dev)
    w_b = torch.empty((T, topk), dtype=torch.float16, device=dev)
    out_b = torch.empty((T, H), dtype=torch.float32, device=dev)
    steps = args.steps if T < 512 else max(1, min(args.steps, args.prefill_steps))
    warmup = args.warmup if T < 512 else min(args.warmup, 3)

    def step(i):
        l = layers[i % NT]
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        bmx._lib.check(L.bmx_moe_layer(ctypes.byref(l.desc), ctypes.byref(l.router), Pp(xs[i % P]), Pp(lgs[i % P]), T,
                                       Pp(sel_b), Pp(w_b), Pp(out_b), Pp(lws), need, pa, s), "bmx_moe_layer")

    def timed(fn):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps

    def run_steps():
        for i in range(steps):
            step(i)

    for i in range(warmup):
        step(i)
    log(f"bench {leg}: timing {steps} steps (eager launches)")
    ms_eager = timed(run_steps)
    want = out_b.clone()
    # the same steps captured once into a HIP graph and replayed (no host launch cost per kernel)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(min(3, steps)):
            step(i)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_steps()
    graph.replay()
    log(f"bench {leg}: timing {steps} steps (graph replay)")
    ms_graph = timed(graph.replay)
    torch.cuda.synchronize()
    if not torch.equal(out_b, want):
        raise RuntimeError(f"{leg}: graph replay output differs from the eager call")
    del graph
    ms = min(ms_eager, ms_graph)

    # per-stage timing with events on the launch stream (torch's current stream): the same layer calls one stage set at
    # a time (bmx_moe_layer_stages), so each stage runs the kernels the one-call step runs
    topk = layers[0].num_experts_per_tok
    path = L.bmx_resolve_path(T, topk, pa)
    prefill, mid = path == bmx._lib.PATH_PREFILL, path == bmx._lib.PATH_MID
    split = path == bmx._lib.PATH_SPLIT
    rpg = L.bmx_rows_per_group(T, topk, pa)
    # a one-token decode call routes the token inside its gate / up GEMV (its route stage launches nothing)
    fused_route = T == 1 and path == bmx._lib.PATH_DECODE and rpg == 1 and os.environ.get("BMX_ROUTE_IN_GEMV") != "0"
    sels, ws_ = [], []
    for p in range(P):
        sp, wp = layers[0].routing_fn(T, None, xs[p], {"logits": lgs[p]})
        sels.append(sp)
        ws_.append(wp)
    routes = [bmx.ops.dispatch(sels[p], E, 0, tabs[0].has_shared, rpg) for p in range(P)]
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    stages = [("route", bmx._lib.STAGE_ROUTE)] + ([("prep", bmx._lib.STAGE_PREP)] if prefill or mid or split else []) + [
        ("gate_up", bmx._lib.STAGE_GATE_UP), ("act", bmx._lib.STAGE_ACT), ("down", bmx._lib.STAGE_DOWN),
        ("combine", bmx._lib.STAGE_COMBINE)]
    nst = steps
    evs = [[TimingEvent() for _ in range(len(stages) + 1)] for _ in range(nst)]

    def staged_step(i, e):
        l, p = layers[i % NT], i % P
        for j, (_, st) in enumerate(stages):
            if e: e[j].record(s)
            bmx._lib.check(L.bmx_moe_layer_stages(ctypes.byref(l.desc), ctypes.byref(l.router), Pp(xs[p]), Pp(lgs[p]), T,
                                                  Pp(sel_b), Pp(w_b), Pp(out_b), Pp(lws), need, pa, 1 << st, s),
                           "bmx_moe_layer_stages")
        if e: e[-1].record(s)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(warmup):
        staged_step(i, None)
    host_ms = (time.perf_counter() - t0) * 1e3 / max(1, warmup)      # host time to enqueue one staged step
    torch.cuda.synchronize()
    # Held-back timing: a bounded clock spin (torch.cuda._sleep) before each batch of steps keeps the stream busy while
    # the host enqueues the batch, so the stages run back to back and the events time the kernels, not the host's
    # launch gaps (the route stage of a one-token call launches nothing and reads as the event overhead)
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record()
    torch.cuda._sleep(1 << 21)
    c1.record()
    torch.cuda.synchronize()
    cyc_per_ms = (1 << 21) / max(c0.elapsed_time(c1), 1e-3)
    batch = 16
    hold_cycles = int(min(50.0, 2.0 * batch * host_ms + 0.2) * cyc_per_ms)
    for b0 in range(0, nst, batch):
        torch.cuda._sleep(hold_cycles)
        for i in range(b0, min(nst, b0 + batch)):
            staged_step(warmup + i, evs[i])
    torch.cuda.synchronize()
    stage_ms = {name: statistics.mean(e[j].elapsed_time(e[j + 1]) for e in evs) for j, (name, _) in enumerate(stages)}
    gu_sep_ms = None
    if fused_route:
        # the same steps with the routing in its own launch (BMX_ROUTE_IN_GEMV=0, read at each call): the gate / up GEMV
        # alone (k_gemv_part<1,2>, the plan's k-splits), for the roofline's view of the GEMV without the routing
        os.environ["BMX_ROUTE_IN_GEMV"] = "0"
        try:
            for i in range(warmup):
                staged_step(i, None)
            torch.cuda.synchronize()
            for b0 in range(0, nst, batch):
                torch.cuda._sleep(hold_cycles)
                for i in range(b0, min(nst, b0 + batch)):
                    staged_step(warmup + i, evs[i])
            torch.cuda.synchronize()
            j = [n for n, _ in stages].index("gate_up")
            gu_sep_ms = statistics.mean(e[j].elapsed_time(e[j + 1]) for e in evs)
        finally:
            del os.environ["BMX_ROUTE_IN_GEMV"]
    # algorithmic units of every timed step: trellis bytes of the unique experts touched, FLOPs of the routed rows
    gu_bytes = dn_bytes = 0
    rows_tot = 0
    sel_np = [x.cpu().numpy() for x in sels]
    for i in range(nst):
        t, p = tabs[i % NT], i % P
        ex = set(int(e) for e in sel_np[p].ravel() if 0 <= e < E)
        if t.has_shared:
            ex.add(E)
        gu_bytes += sum(t.mat_bytes(e, 0) + t.mat_bytes(e, 1) for e in ex)
        dn_bytes += sum(t.mat_bytes(e, 2) for e in ex)
        rows_tot += routes[p].rows()
    gu_bytes, dn_bytes, rows = gu_bytes / nst, dn_bytes / nst, rows_tot / nst
    q_bytes = gu_bytes + dn_bytes
    gu_ms = stage_ms["gate_up"]
    layer_flops = synth.flops(H, c["I"], rows)
    gu_flops = 4.0 * H * c["I"] * rows

    cpu = None
    if with_cpu and not args.no_cpu:
        n_cpu = T if T <= 64 else 64
        cpu = cpu_baseline(tabs[0], sels[0][:n_cpu], ws_[0][:n_cpu],
                           budget_s=args.cpu_budget if leg in HEADLINE_LEGS else min(4.0, args.cpu_budget))
    kind = "prefill" if prefill else "mid" if mid else "split" if split else "decode"
    traffic = traffic_src = prof_us = None
    tpath = os.path.join(REPO, "profiles", f"{kind}_{cfg}_t{T}.json")
    if os.path.exists(tpath):
        tr = json.load(open(tpath))
        traffic = tr["read_bytes"] + tr["write_bytes"]
        prof_us = tr.get("kernel_us_avg")
        traffic_src = (f"loaded from the committed profiles/{kind}_{cfg}_t{T}.json ({tr.get('measured', 'date not recorded')}"
                       f"; command in profiles/{kind}_{cfg}_t{T}.md): rocprofv3 FETCH_SIZE / WRITE_SIZE passes over the "
                       f"same workload, scaled by a plain copy's counters; not measured in this run")
    if prefill:
        ach = gu_flops / (gu_ms * 1e-3) / 1e12
        kern = "k_pf_gemm<false> (BMX_STAGE_GATE_UP: trellis decode + gate/up MFMA grouped GEMM, 128-row groups)"
        roofline = {"kernel": kern, "bound": "mfma", "achieved": round(ach, 1), "peak": MFMA_FP16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(ach / MFMA_FP16_PEAK_TFLOPS, 4), "traffic": traffic,
                    "algorithmic_flops": gu_flops, "kernel_us": round(gu_ms * 1e3, 3), "traffic_source": traffic_src,
                    "timing": "achieved uses the mean event-timed duration of the gate/up stage (one kernel launch) over "
                              "the timed steps, enqueued behind a clock spin so the stages run back to back between "
                              "timing-only events (no system-scope release); "
                              "kernel_us_rocprof is the committed trace's average for the same leg"}
        if prof_us:
            roofline.update(kernel_us_rocprof=prof_us,
                            frac_rocprof=round(gu_flops / (prof_us * 1e-6) / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4))
    else:
        gu_gbps = gu_bytes / (gu_ms * 1e-3) / 1e9
        kern = ("k_gemv_gu_route (BMX_STAGE_GATE_UP of the one-token layer call: routing + dispatch of the token, "
                "then trellis decode + gate/up split-K GEMV)" if fused_route
                else "k_mid_gemm<false> (BMX_STAGE_GATE_UP of the mid-size path: trellis decode + gate/up MFMA in 32-row "
                     "groups, k-split; a decode-size call, so the roofline is the quantized bytes against HBM)" if mid
                else "k_gemv_part<gate/up> + k_mid_gemm<false> (BMX_STAGE_GATE_UP of the split path: the GEMV over the "
                     "experts with few rows, then the MFMA kernel over those with many; the two launches timed as one "
                     "stage)" if split
                else "k_gemv_part<gate/up> (BMX_STAGE_GATE_UP: trellis decode + gate/up split-K GEMV)")
        roofline = {"kernel": kern,
                    "bound": "hbm", "achieved": round(gu_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": round(gu_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic, "algorithmic_bytes": round(gu_bytes),
                    "kernel_us": round(gu_ms * 1e3, 3), "traffic_source": traffic_src,
                    "timing": "achieved uses the mean event-timed duration of the gate/up stage (one kernel launch) over "
                              "the timed steps, each step on other experts, enqueued behind a clock spin so the stages run "
                              "back to back, between timing-only events (no system-scope release; an empty stage, the route "
                              "stage of a one-token call, reads as the events' own cost); kernel_us_rocprof is the committed trace's average for the same leg (no event "
                              "records around the kernel)"}
        if prof_us:
            roofline.update(kernel_us_rocprof=prof_us,
                            frac_rocprof=round(gu_bytes / (prof_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4))
        if mid:
            mf = gu_flops / (gu_ms * 1e-3) / 1e12
            roofline.update(mfma_view={"achieved": round(mf, 2), "peak": MFMA_FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                       "frac": round(mf / MFMA_FP16_PEAK_TFLOPS, 4), "algorithmic_flops": gu_flops})
        if gu_sep_ms:
            sep = gu_bytes / (gu_sep_ms * 1e-3) / 1e9
            roofline.update(gemv_without_routing={
                "kernel": "k_gemv_part<1,2> (the same steps with the routing in its own launch, BMX_ROUTE_IN_GEMV=0)",
                "kernel_us": round(gu_sep_ms * 1e3, 3), "achieved": round(sep, 1),
                "frac": round(sep / HBM_PEAK_GBPS, 4)})
    scores = {0: "softmax", 1: "sigmoid"}[c["score"]] + ("+bias" if c["bias"] else "")
    if c["n_group"] > 1:
        scores = f"group-limited ({c['n_group']} groups, top-{c['topk_group']}) {scores}"
    bpw = {"c1": "4", "c2": "3", "c3": "2/3 mixed", "c4": "3", "c5": "2/2.5 mixed"}[cfg]
    return {
        "leg": leg, "ms": ms, "T": T, "steps": steps, "warmup": warmup,
        "workload": f"{cfg} {kind} layer: {E} routed experts top-{topk} {scores}{' + 1 shared' if c['shared'] else ''}, "
                    f"H {H}, I {c['I']}, EXL3 {bpw} bpw, {T} token{'s' if T > 1 else ''} per step",
        "rotation": f"step i reads input batch i % {P} and layer table i % {NT}"
                    + ("" if P * NT > 1 else " (one batch: the layer's 2.4 GB of experts are read in full every step)"),
        "path": kind,
        "value": round(T * 1e3 / ms, 2), "unit": "tokens/s",
        "us_per_layer": round(ms * 1e3, 3), "us_per_token": round(ms * 1e3 / T, 3),
        "us_per_layer_eager": round(ms_eager * 1e3, 3), "us_per_layer_graph": round(ms_graph * 1e3, 3),
        "quantized_bytes_per_layer": round(q_bytes),
        "layer_hbm_gbps": round(q_bytes / (ms * 1e-3) / 1e9, 1),
        "layer_tflops": round(layer_flops / (ms * 1e-3) / 1e12, 1),
        "layer_mfma_frac": round(layer_flops / (ms * 1e-3) / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4),
        "stage_us": {k: round(v * 1e3, 3) for k, v in stage_ms.items()},
        "roofline": roofline,
        "cpu_baseline": ({k: (round(v, 3) if isinstance(v, float) else v) for k, v in cpu.items()} if cpu else None),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--prefill-steps", type=int, default=20, help="timed steps of the 8192-token prefill leg")
    ap.add_argument("--legs", default=",".join(LEGS),
                    help=f"comma-separated legs of the default run ({', '.join(LEGS)}); the first two are the metric")
    ap.add_argument("--tokens", type=int, default=None, help="with --config: tokens per step")
    ap.add_argument("--config", default=None, help="one workload instead of the legs (c1, c2, c3, c5; c4: the stack)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--path", choices=["auto", "decode", "mid", "prefill", "split"], default="auto",
                    help="expert-products path (auto: the library's choice for the batch)")
    ap.add_argument("--prefetch", type=int, default=0, metavar="N",
                    help="c4: layer-ahead prefetch of up to N guessed experts of the next layer per layer (0: off)")
    ap.add_argument("--prefetch-ahead", type=int, default=1, metavar="D",
                    help="c4 prefetch: layer li prefetches the guess of layer li + D")
    ap.add_argument("--copies", choices=["kernel", "dma"], default="dma",
                    help="c4: slot copies by a kernel on a side stream or by the copy agent on the DMA engines")
    ap.add_argument("--guess-noise", type=float, default=1.0, metavar="SIGMA",
                    help="c4 prefetch: the next layer's guess routes its own logits plus N(0, SIGMA) noise")
    ap.add_argument("--cpu-lane", type=int, default=0, metavar="THREADS",
                    help="c4: planned steps with the CPU lane (fast mode) on THREADS worker threads (0: off)")
    ap.add_argument("--cpu-max", type=int, default=2, help="c4 --cpu-lane: most misses a layer call puts on the CPU")
    ap.add_argument("--separate-route-step", action="store_true",
                    help="c4: the router and the slot step as two launches (default: one, bmx_route_slot_step)")
    ap.add_argument("--cpu-expert-us", type=float, default=125.0,
                    help="c4 --cpu-lane: the planner's CPU cost of one expert until the lane's first job is timed")
    ap.add_argument("--timeline-steps", type=int, default=10, help="c4: tokens of the per-layer timeline loop")
    ap.add_argument("--c4-steps", type=int, default=30, help="timed tokens of the c4 leg in the default run")
    ap.add_argument("--staged-layers", type=int, default=8, help="prefill_staged: layers of the stack")
    ap.add_argument("--staged-steps", type=int, default=3, help="prefill_staged: timed chunks through the stack")
    ap.add_argument("--cpu-budget", type=float, default=8.0,
                    help="seconds of CPU-lane calls per thread setting (headline legs; the others take at most 4)")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="run one plain device copy of MIB MiB first (scale reference for HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: measures one GPU; --gpus {args.gpus} is not supported (sharding the layer's experts across "
              f"GPUs is not implemented)", file=sys.stderr)
        sys.exit(2)
    if args.config == "c4":
        print(json.dumps(bench_c4(args)), flush=True)
        return
    import torch
    if args.calib_copy:
        src = torch.empty(args.calib_copy << 18, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.config:
        from bmx import synth
        c = synth.CONFIGS[args.config]
        T = args.tokens or c["T"]
        P = 1 if T * c["topk"] >= 512 else max(1, 64 // T)
        legs = [(args.config, args.config, T, P, 1)]
    else:
        legs = []
        for name in args.legs.split(","):
            if name not in LEGS:
                raise SystemExit(f"bench.py: unknown leg {name!r} (legs: {', '.join(LEGS)})")
            legs.append((name,) + (LEGS[name] or ()))
    results = []
    for leg in legs:
        name = leg[0]
        if name in ("c4", "c4_cpu_lane"):
            a4 = argparse.Namespace(**vars(args))
            if name == "c4_cpu_lane" and not a4.cpu_lane:
                a4.cpu_lane = 12
            r = bench_c4(a4)
            r = dict(r, leg=name, ms=r["ms_per_step"], T=1)
        elif name == "prefill_staged":
            pf = next((x for x in results if x["leg"] == "prefill"), None)
            cpu = None
            if pf is not None and pf.get("cpu_baseline"):
                cpu = dict(pf["cpu_baseline"], sample="the prefill leg's sample (the same layer shape, experts in RAM): "
                                                      + pf["cpu_baseline"]["sample"])
            r = bench_staged(args, cpu)
            r = dict(r, leg="prefill_staged", ms=r["ms_per_chunk"] / r["layers"])
        else:
            _, cfg, T, P, NT = leg
            r = bench_leg(name, cfg, T, P, NT, args, with_cpu=True)
        results.append(r)
        torch.cuda.empty_cache()
    head = results[0]
    if head["leg"] in ("c4", "c4_cpu_lane"):
        # The stack leg's result is already a whole line of its own.
        res = {k: v for k, v in head.items() if k not in ("leg", "ms", "T")}
    else:
        layer_call = "us_per_layer_graph" in head
        res = {
            "metric": METRIC,
            "value": head["value"],
            "unit": head["unit"],
            "n_gpus": 1,
            "steps": head["steps"],
            "warmup": head["warmup"],
            "ms_per_step": round(head["ms"], 6),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "fp16",
            "data": "synthetic: random EXL3 trellis codes, suh ~ U(0.5,1.5), svh ~ U(0.5,1.5)/sqrt(k), x ~ N(0,1) fp16 "
                    "(c5: 1 % of channels x20), router logits ~ N(0,1) fp16 (c3 / c5: Zipf(1.1) log-popularity + Gumbel "
                    "noise), bias ~ N(0,0.1); seeded; decode steps rotate over input batches (and c1 over layer tables) "
                    "so the experts read change every step (cold weights)",
            "config": {"workload": head["workload"], "tokens": head["T"], "path": head["path"]},
        }
        if layer_call:
            res["config"].update(rotation=head["rotation"],
                                 step="router + dispatch + gate/up + down + combine (one bmx_moe_layer call)")
            res["timing"] = "min of eager launches and HIP-graph replay of the same sequence of bmx_moe_layer calls"
        else:
            res["config"].update(layers=head["layers"], step="one chunk of tokens through every layer of the stack, "
                                                             "experts staged from host memory one layer ahead")
        for k in ("us_per_layer", "us_per_token", "us_per_layer_eager", "us_per_layer_graph", "quantized_bytes_per_layer",
                  "layer_hbm_gbps", "stage_us", "ms_per_chunk", "staged_experts_per_layer", "staged_bytes_per_layer",
                  "roofline", "cpu_baseline"):
            if k in head:
                res[k] = head[k]
    for r in results[1:]:
        r = dict(r)
        del r["ms"]
        res[r.pop("leg")] = r
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()

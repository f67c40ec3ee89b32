"""GPU expert-slot table against the oracle's CLOCK step (bit-exact state after every step), the staging copies (slot
bytes equal the home bytes), and the layer with experts staged from pinned host memory (bit-identical outputs to the
same layer with every expert resident)."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def small_layers(n_layers, E, H, I, seed, home, fmts=None):
    import bmx
    fm = fmts or (bmx.TF_K3,) * 3
    return [bmx.ExpertTable.random(H, I, E, fm, seed=seed + li, device="cuda", home=home) for li in range(n_layers)]


def tables_of(slots):
    """Host copies of every layer's bmx_expert tr pointers: [L, E, 3] uint64."""
    import bmx
    es = ctypes.sizeof(bmx._lib.Expert)
    out = []
    for t in slots.layers:
        raw = t.table().cpu().numpy().tobytes()
        arr = (bmx._lib.Expert * (t.E + (1 if t.has_shared else 0))).from_buffer_copy(raw)
        out.append([[arr[e].tr[m] for m in range(3)] for e in range(t.E)])
        assert len(raw) == es * (t.E + (1 if t.has_shared else 0))
    return np.array(out, dtype=np.uint64)


def check_state(slots, ref, fresh_want, step):
    torch.cuda.synchronize()
    S = slots.S
    assert np.array_equal(slots.slotof.cpu().numpy(), ref.slotof), step
    assert np.array_equal(slots.owner.cpu().numpy()[:S], ref.owner[:S]), step
    assert np.array_equal(slots.refb.cpu().numpy()[:S], ref.refb[:S]), step
    assert np.array_equal(slots.pin.cpu().numpy()[:S], ref.pin[:S]), step
    ctl = slots.ctl.cpu().numpy()
    assert ctl[0] == ref.hand and ctl[1] == ref.epoch, (step, ctl, ref.hand, ref.epoch)
    assert np.array_equal(slots.stats_t.cpu().numpy(), ref.stats), (step, slots.stats_t.cpu().numpy(), ref.stats)
    assert np.array_equal(slots.fresh.cpu().numpy(), fresh_want), step
    assert np.array_equal(slots.pfl.cpu().numpy()[:S], ref.pfl[:S]), step
    # every table entry points at its slot when resident, at its home otherwise
    tr = tables_of(slots)
    base = slots.arena.data_ptr()
    t0 = slots.layers[0]
    for li, t in enumerate(slots.layers):
        for e in range(t.E):
            s = int(ref.slotof[li * t.E + e])
            want = (t.addr[e] if s < 0 else (base + s * t0.rec, base + s * t0.rec + t0.off_u, base + s * t0.rec + t0.off_d))
            assert tuple(int(v) for v in tr[li, e]) == tuple(want), (step, li, e)


@pytest.mark.parametrize("S,maxj,disabled", [(10, 4, (3,)), (5, 8, ()), (0, 4, ())])
def test_slot_step_matches_oracle(cuda, oracle, S, maxj, disabled):
    import bmx
    Lyr, E = 3, 16
    layers = small_layers(Lyr, E, 256, 128, 10, "device")
    first = 7
    slots = bmx.ExpertSlots(layers, S, maxj=maxj, disabled=disabled, first=first)
    ref = oracle.SlotTable(Lyr, E, S)
    for s in disabled:
        ref.pin[s] = -1
    rng = np.random.default_rng(S * 100 + maxj)
    for step in range(40):
        li = int(rng.integers(0, Lyr))
        n = int(rng.integers(0, 12))
        sel = rng.integers(0, E + 3, n) + first - 1            # a few ids outside [first, first + E): dropped
        admit = bool(rng.random() < 0.85)
        say("slot step", step, "layer", li, "picks", n, "admit", admit)
        slots.step(li, torch.from_numpy(sel.astype(np.int64)).cuda(), admit)     # Pool.step(li, sel, admit)
        jobs, ev = ref.step(li, sel.astype(np.int64), first, admit, maxj)
        fresh_want = np.zeros(E, np.int32)
        fresh_want[jobs[:, 0]] = 1
        assert np.array_equal(ref.fresh, fresh_want)          # no prefetches here: fresh = the admissions
        check_state(slots, ref, fresh_want, step)
        nj = int(slots.ctl[2].item())
        assert nj == len(jobs)
        assert np.array_equal(slots.jobs.cpu().numpy()[:2 * nj].reshape(nj, 2), jobs)


@pytest.mark.parametrize("S,maxj", [(10, 4), (6, 8), (0, 2)])
def test_slot_prefetch_matches_oracle(cuda, oracle, S, maxj):
    """Steps and layer-ahead prefetches interleaved (guesses with duplicates, resident experts, ids out of range, limits):
    slot state, prefetch job buffers, fresh flags and counters bit-exact against the oracle after every call."""
    import bmx
    Lyr, E = 3, 20
    layers = small_layers(Lyr, E, 256, 128, 20, "device")
    first = 3
    slots = bmx.ExpertSlots(layers, S, maxj=maxj, disabled=(2,) if S else (), first=first)
    ref = oracle.SlotTable(Lyr, E, S)
    if S:
        ref.pin[2] = -1
    rng = np.random.default_rng(S * 10 + maxj)
    fresh_want = np.zeros(E, np.int32)
    for it in range(60):
        li = int(rng.integers(0, Lyr))
        if rng.random() < 0.5:
            sel = rng.integers(0, E + 2, int(rng.integers(0, 10))) + first - 1
            say("slot step", it, "layer", li, "picks", sel.size)
            slots.step(li, torch.from_numpy(sel.astype(np.int64)).cuda())
            jobs, _ = ref.step(li, sel.astype(np.int64), first, True, maxj)
            fresh_want = ref.fresh.copy()
        else:
            g = rng.integers(0, E + 2, int(rng.integers(0, 16))) + first - 1
            limit = int(rng.integers(0, 6))
            b = slots.pf_calls & 1
            say("slot prefetch", it, "layer", li, "guesses", g.size, "limit", limit, "buffer", b)
            slots.prefetch(li, torch.from_numpy(g.astype(np.int64)).cuda(), limit)
            jobs, _ = ref.prefetch(li, g.astype(np.int64), first, limit, maxj)
            torch.cuda.synchronize()
            pj = slots.pjobs.cpu().numpy()[b * (1 + 2 * maxj):]
            assert pj[0] == len(jobs) and np.array_equal(pj[1:1 + 2 * len(jobs)].reshape(-1, 2), jobs), it
        check_state(slots, ref, fresh_want, it)
    st = ref.stats
    say("oracle stats", st.tolist())
    if S:
        assert st[5] > 0 and st[6] > 0


def resident_bytes_match(slots, layers):
    """Every resident expert's slot holds its home record's gate / up / down bytes; returns how many were checked."""
    L, E = len(layers), layers[0].E
    slotof = slots.slotof.cpu().numpy().reshape(L, E)
    arena = slots.arena.cpu().numpy()
    t0 = layers[0]
    checked = 0
    for li in range(L):
        for e in range(E):
            s = slotof[li, e]
            if s < 0:
                continue
            rec = layers[li].arena[e].cpu().numpy()
            for m, off in enumerate((0, t0.off_u, t0.off_d)):
                nb = layers[li].mat_bytes(e, m)
                assert np.array_equal(arena[s, off:off + nb], rec[off:off + nb]), (li, e, m)
            checked += 1
    say("resident experts checked", checked)
    return checked


def test_agent_ring_wraps_without_waits(cuda):
    """Three times the agent's 64-record ring of steps and prefetches published back to back, no layer waiting in
    between: every record is handed over in order (a step only reuses a ring slot the agent has read), and the slots
    end up holding their homes' bytes."""
    import time
    import bmx
    layers = small_layers(2, 12, 256, 128, 40, "host", fmts=(bmx.TF_K3, bmx.TF_K2, bmx.TF_K4))
    slots = bmx.ExpertSlots(layers, 7, maxj=6, copies="dma")
    rng = np.random.default_rng(9)
    records = 0
    for step in range(96):
        li = step % 2
        slots.step(li, torch.from_numpy(rng.integers(0, 12, 5).astype(np.int64)).cuda())
        slots.prefetch(1 - li, torch.from_numpy(rng.permutation(12)[:3].astype(np.int64)).cuda(), limit=2)
        records += 2
    slots.wait_copies(0)
    slots.wait_copies(1)
    torch.cuda.synchronize()
    t0 = time.time()
    while slots.agent_status()[0] < records and time.time() - t0 < 2.0:
        time.sleep(0.001)
    rec, ncopies, nbytes, gu, dn, late = slots.agent_status()
    say("agent records", rec, "copies", ncopies, "bytes", nbytes, "flags", gu, dn, late)
    assert rec == records and late == 0
    t0 = time.time()
    while slots.agent_status()[4] < records and time.time() - t0 < 2.0:
        time.sleep(0.001)
    assert slots.agent_status()[3] == slots.agent_status()[4] == records
    torch.cuda.synchronize()
    assert resident_bytes_match(slots, layers) == 7
    slots.close()


@pytest.mark.parametrize("copies,home", [("kernel", "host"), ("dma", "host"), ("dma", "device")])
def test_slot_copies_deliver_home_bytes(cuda, copies, home):
    import bmx
    layers = small_layers(2, 12, 256, 128, 30, home, fmts=(bmx.TF_K2, bmx.TF_K25, bmx.TF_K4))
    slots = bmx.ExpertSlots(layers, 7, maxj=6, copies=copies)
    rng = np.random.default_rng(5)
    for step in range(12):
        li = step % 2
        sel = torch.from_numpy(rng.integers(0, 12, 5).astype(np.int64)).cuda()
        slots.step(li, sel)
    slots.wait_copies(0)
    slots.wait_copies(1)
    torch.cuda.synchronize()
    assert resident_bytes_match(slots, layers) == 7
    if copies == "dma":
        import time
        t0 = time.time()
        while slots.agent_status()[4] < 12 and time.time() - t0 < 2.0:   # a last step without admissions needs no wait
            time.sleep(0.001)
        rec, ncopies, nbytes, gu, dn, late = slots.agent_status()
        say("agent records", rec, "copies", ncopies, "bytes", nbytes)
        assert rec == 12 and gu == dn == 12 and late == 0 and ncopies == 2 * slots.stats()[2]
        slots.close()


@pytest.mark.parametrize("copies", ["kernel", "dma"])
def test_layer_with_staged_experts_matches_resident(cuda, copies):
    """The same layers computed with every expert resident in device memory and with homes in pinned host memory staged
    through a small slot table (hits, admissions copied on the side stream by a kernel or by the copy agent on the DMA
    engines, and misses left at home when maxj runs out): identical outputs, bit for bit, on the GEMV, mid-size and
    prefill paths. One-token calls route and step in one launch (MoELayer.route_layer)."""
    import bmx
    from bmx import synth
    Lyr, E, H, I, topk = 3, 24, 512, 256, 4
    dev_layers = small_layers(Lyr, E, H, I, 50, "device")
    host_layers = small_layers(Lyr, E, H, I, 50, "host")
    slots = bmx.ExpertSlots(host_layers, 9, maxj=3, copies=copies)
    kw = dict(score=bmx.SCORE_SIGMOID, renorm=True, scale=1.0)
    ref_layers = [bmx.MoELayer(dev_layers[li], topk, **kw) for li in range(Lyr)]
    st_layers = [bmx.MoELayer(host_layers[li], topk, slots=slots, li=li, **kw) for li in range(Lyr)]
    rng = np.random.default_rng(9)
    for step in range(9):
        li = step % Lyr
        T = (1, 3, 40)[step % 3]
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16)).cuda()
        lg = torch.from_numpy(synth.zipf_logits(T, E, 1.1, seed=step)).cuda()
        for path in (bmx.PATH_DECODE, bmx.PATH_MID, bmx.PATH_PREFILL):
            sel, w = ref_layers[li].routing_fn(T, None, x, {"logits": lg})
            want = ref_layers[li].run_bszN(x, sel, w, path)
            if T == 1:      # the routing and the step in one launch
                sel2, w2, _ = st_layers[li].route_layer(li, x, T, {"logits": lg})
            else:
                sel2, w2 = st_layers[li].routing_fn(T, None, x, {"logits": lg})
                st_layers[li].layer(li, sel2, w2, x, T)
            got = st_layers[li].run_bszN(x, sel2, w2, path)
            torch.cuda.synchronize()
            say("staged layer step", step, "layer", li, "T", T, "path", path, "stats", slots.stats())
            assert torch.equal(sel, sel2) and torch.equal(got, want)
    h, m, adm, novic, ev = slots.stats()[:5]
    assert m > 0 and adm > 0 and ev > 0 and m > adm      # misses, admissions, evictions and unadmitted misses all ran
    if copies == "dma":
        say("agent", slots.agent_status())
        slots.close()


@pytest.mark.parametrize("copies", ["kernel", "dma"])
def test_prefetch_keeps_outputs(cuda, copies):
    """A decode loop over a stack of layers with homes in pinned host memory, each layer's step followed by a prefetch
    of the next layer's guessed experts (its router on noisy logits: right and wrong guesses) before the layer's
    products: outputs identical, bit for bit, to the same layers with every expert resident; prefetched experts are
    used and some are evicted unused."""
    import bmx
    from bmx import synth
    Lyr, E, H, I, topk = 4, 24, 512, 256, 4
    dev_layers = small_layers(Lyr, E, H, I, 80, "device")
    host_layers = small_layers(Lyr, E, H, I, 80, "host")
    slots = bmx.ExpertSlots(host_layers, 10, maxj=3, copies=copies)
    kw = dict(score=bmx.SCORE_SIGMOID, renorm=True, scale=1.0)
    ref_layers = [bmx.MoELayer(dev_layers[li], topk, **kw) for li in range(Lyr)]
    st_layers = [bmx.MoELayer(host_layers[li], topk, slots=slots, li=li, **kw) for li in range(Lyr)]
    rng = np.random.default_rng(11)
    for tok in range(12):
        T = 1 if tok % 4 else 3
        lgs = [torch.from_numpy(synth.zipf_logits(T, E, 1.1, seed=100 * tok + li)).cuda() for li in range(Lyr)]
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16)).cuda()
        for li in range(Lyr):
            sel, w = ref_layers[li].routing_fn(T, None, x, {"logits": lgs[li]})
            want = ref_layers[li].run_bszN(x, sel, w)
            sel2, w2 = st_layers[li].routing_fn(T, None, x, {"logits": lgs[li]})
            st_layers[li].layer(li, sel2, w2, x, T)
            if li + 1 < Lyr:
                noisy = lgs[li + 1].float() + torch.randn(lgs[li + 1].shape, device="cuda") * 0.7
                guess, _ = st_layers[li + 1].routing_fn(T, None, x, {"logits": noisy.half()})
                slots.prefetch(li + 1, guess.view(-1), limit=4)
            got = st_layers[li].run_bszN(x, sel2, w2)
            torch.cuda.synchronize()
            assert torch.equal(got, want), (tok, li)
        say("prefetch token", tok, "stats", slots.stats())
    h, m, adm, novic, ev, pfa, pfu, pfw = slots.stats()
    assert pfa > 0 and pfu > 0 and pfw > 0
    if copies == "dma":
        say("agent", slots.agent_status())
        slots.close()


def test_stage_async_copies(cuda):
    import bmx
    layers = small_layers(1, 4, 256, 128, 70, "host")
    slots = bmx.ExpertSlots(layers, 4, maxj=2)
    t = layers[0]
    src = [t.addr[e][0] for e in range(4)]
    dst = [slots.arena.data_ptr() + s * t.rec for s in range(4)]
    slots.stage_async(src, dst, [t.rec] * 4)
    torch.cuda.synchronize()
    assert torch.equal(slots.arena.cpu(), t.arena.clone())


def test_agent_failure_is_reported(cuda):
    """A copy wait that runs out of time, forced from the host (the agent's thread holds back from reading records, the
    wait limit is 20 ms; every kernel still ends by itself): a step queued behind the failed wait admits nothing, so its
    experts run from their homes, and the host calls after it raise instead of handing out results computed on slots
    whose copies never ran."""
    import bmx
    layers = small_layers(1, 12, 256, 128, 90, "host")
    slots = bmx.ExpertSlots(layers, 6, maxj=4, copies="dma")
    lib = bmx.lib()
    bmx._lib.check(lib.bmx_copy_agent_control(slots.agent, 1, 20000), "bmx_copy_agent_control")
    # picks made before the first launch: a host-to-device copy made later would wait for the 20 ms wait
    p01, p23, p4 = (torch.tensor(e, dtype=torch.int64, device="cuda") for e in ((0, 1), (2, 3), (4,)))
    torch.cuda.synchronize()
    say("agent failure: step admitting 0, 1 with the agent held")
    slots.step(0, p01)                              # admitted and published, never copied
    slots.wait_copies(0, part="gate_up")           # gives up on the device after 20 ms
    slots.step(0, p23)                              # launched before the wait gave up
    torch.cuda.synchronize()
    say("agent failure: stats", slots.stats(), "ctl", slots.ctl.tolist())
    assert int(slots.ctl[2].item()) == 0
    assert int(slots.slotof[2].item()) == -1 and int(slots.slotof[3].item()) == -1
    assert int(slots.slotof[0].item()) >= 0 and int(slots.slotof[1].item()) >= 0
    with pytest.raises(bmx.BmxError, match="ran out of time"):
        slots.check()
    with pytest.raises(bmx.BmxError, match="ran out of time"):
        slots.step(0, p4)
    with pytest.raises(bmx.BmxError, match="ran out of time"):
        slots.wait_copies(0)
    bmx._lib.check(lib.bmx_copy_agent_control(slots.agent, 0, 0), "bmx_copy_agent_control")
    slots.close()


@pytest.mark.parametrize("E,copies", [(40, "kernel"), (288, "dma")])
def test_route_slot_step_matches_separate(cuda, E, copies):
    """bmx_route_slot_step (one token's routing and the step in one launch) against bmx_router_topk followed by the step
    on a twin table: the same picks and weights, and the same slot state, fresh flags, counters and jobs after every
    call; the admitted experts' slots then hold their homes' bytes."""
    import bmx
    Lyr, S, topk = 3, 20, 8
    a_layers = small_layers(Lyr, E, 256, 128, 60, "host")
    b_layers = small_layers(Lyr, E, 256, 128, 60, "host")
    sa = bmx.ExpertSlots(a_layers, S, maxj=4, copies=copies)
    sb = bmx.ExpertSlots(b_layers, S, maxj=4, copies=copies)
    g = torch.Generator(device=cuda)
    g.manual_seed(61)
    bias = (torch.randn(E, generator=g, device=cuda) * 0.1).float()
    rng = np.random.default_rng(62)
    for step in range(24):
        li = int(rng.integers(0, Lyr))
        admit = bool(rng.random() < 0.85)
        lg = torch.randn((1, E), generator=g, device=cuda).half()
        say("route step", step, "layer", li, "admit", admit)
        sel, w = bmx.ops.router_topk(lg, topk, bias, 1, 1, bmx.SCORE_SIGMOID, True, 2.5)
        sa.step(li, sel.view(-1), admit)
        sel_b, w_b = sb.route_step(li, lg, topk, bias, 1, 1, bmx.SCORE_SIGMOID, True, 2.5, admit)
        torch.cuda.synchronize()
        assert torch.equal(sel, sel_b) and torch.equal(w, w_b), step
        for name in ("slotof", "owner", "refb", "pin", "ctl", "stats_t", "fresh", "pfl"):
            assert torch.equal(getattr(sa, name), getattr(sb, name)), (step, name)
        nj = int(sa.ctl[2].item())
        assert torch.equal(sa.jobs[:2 * nj], sb.jobs[:2 * nj]), step
    for li in range(Lyr):
        sa.wait_copies(li)
        sb.wait_copies(li)
    torch.cuda.synchronize()
    assert resident_bytes_match(sb, b_layers) == resident_bytes_match(sa, a_layers) > 0
    sa.close()
    sb.close()

"""The residency plan's request / reply on the GPU: planned steps against the oracle's planner and CLOCK step (lanes,
masked selection and slot-table state bit-exact after every step), the CPU lane's partial added to a layer call (bit
for bit the GPU rows summed in the documented order), and the bounded wait for a reply that never comes."""
import numpy as np
import pytest
import torch

from test_gpu_slots import check_state, small_layers

pytestmark = pytest.mark.gpu

MIXED = dict(cpu_on=1, max_cpu=2, home_single=1, gpu_base_us=10.0, gpu_hit_us=1.0, gpu_home_us=2.0, gpu_admit_us=6.0,
             cpu_base_us=5.0, cpu_expert_us=4.0, cpu_token_us=2.0)


def say(*a):
    print(*a, flush=True)


def picks(rng, T, topk, E, first):
    """T tokens' distinct picks, a few of them outside [first, first + E)"""
    return np.stack([rng.choice(E + 2, topk, replace=False) for _ in range(T)]).astype(np.int64) + first - 1


@pytest.mark.parametrize("policy", ["default", "mixed"])
def test_planned_steps_match_oracle(cuda, oracle, policy):
    import bmx
    Lyr, E, H, I, S, maxj, topk, first = 2, 20, 256, 128, 8, 4, 4, 5
    layers = small_layers(Lyr, E, H, I, 120, "host")
    slots = bmx.ExpertSlots(layers, S, maxj=maxj, copies="dma", first=first)
    pol = None if policy == "default" else MIXED
    cpu = pol is not None
    if cpu:
        slots.cpu_lane(topk, threads=4)
    slots.plan(pol)
    ref = oracle.SlotTable(Lyr, E, S)
    rng = np.random.default_rng(7 if cpu else 3)
    seen = set()
    for step in range(36):
        li = int(rng.integers(0, Lyr))
        T = int(rng.integers(1, 4))
        sel = picks(rng, T, topk, E, first)
        w = (rng.random((T, topk)) * 2).astype(np.float16)
        x = rng.standard_normal((T, H)).astype(np.float16)
        ex, res, cnt = ref.request(li, sel, first)
        lanes = oracle.plan_lanes(ex, res, cnt, T, sel.size, True, pol, cpu_ready=cpu)
        el = oracle.expert_lanes(E, ex, lanes)
        sg, wg, ln = oracle.planned_selection(sel, w, first, el)
        say("planned step", step, "layer", li, "T", T, "lanes", lanes.tolist())
        got = slots.step_planned(li, torch.from_numpy(sel).cuda(), torch.from_numpy(w).cuda(),
                                 torch.from_numpy(x).cuda())
        ref.step(li, sel.ravel(), first, True, maxj, elane=el)
        check_state(slots, ref, ref.fresh, step)
        assert np.array_equal(got[2].cpu().numpy(), ln), step
        assert np.array_equal(got[0].cpu().numpy(), sg), step
        assert np.array_equal(got[1].cpu().numpy().view(np.uint16), wg.view(np.uint16)), step
        seen.update(int(v) for v in lanes)
    say("lanes seen", sorted(seen), "stats", slots.stats(), "agent", slots.agent_status())
    want = {0, 1, 2, 3} if cpu else {0, 1}
    assert want <= seen
    slots.close()


def test_cpu_lane_partial_added(cuda, oracle):
    """Layer calls through MoELayer with a planned slot table whose planner puts two of each call's missing experts on
    the CPU lane: out = the GPU's combine of the masked selection (slot order) + the CPU lane's partial (w * y in pick
    order), bit for bit, with every y row the GPU's own (the CPU lane is exact)."""
    import bmx
    from bmx import synth
    Lyr, E, H, I, topk, first = 2, 16, 256, 128, 4, 0
    dev_layers = small_layers(Lyr, E, H, I, 140, "device")
    host_layers = small_layers(Lyr, E, H, I, 140, "host")
    slots = bmx.ExpertSlots(host_layers, 6, maxj=2, copies="dma")
    slots.cpu_lane(topk, threads=4)
    slots.plan(dict(cpu_on=1, max_cpu=2, gpu_base_us=1.0, gpu_admit_us=1.0))      # a free CPU lane: it takes two
    kw = dict(score=bmx.SCORE_SIGMOID, renorm=True, scale=1.0)
    ref_layers = [bmx.MoELayer(dev_layers[li], topk, **kw) for li in range(Lyr)]
    st_layers = [bmx.MoELayer(host_layers[li], topk, slots=slots, li=li, **kw) for li in range(Lyr)]
    rng = np.random.default_rng(21)
    ncpu = 0
    for step in range(10):
        li = step % Lyr
        T = 1 + step % 3
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16)).cuda()
        lg = torch.from_numpy(synth.zipf_logits(T, E, 1.1, seed=300 + step)).cuda()
        m = st_layers[li]
        sel, w = m.routing_fn(T, None, x, {"logits": lg})
        sel_g, w_g, flag = m.layer(li, sel, w, x, T)
        assert flag
        out = m.cpu_split_combine(m.combine(m.run_bszN(x, sel_g, w_g, bmx.PATH_DECODE)), None, False, None)
        # the GPU rows of every pick, from the resident twin
        routes = bmx.ops.dispatch(sel, E, first, False, bmx.lib().bmx_rows_per_group(T, topk, bmx.PATH_DECODE))
        y, _ = bmx.ops.moe_experts(ref_layers[li].desc, x, routes, bmx.PATH_DECODE)
        torch.cuda.synchronize()
        y, inv = y.cpu().numpy(), routes.inv.cpu().numpy()
        s, sg = sel.cpu().numpy().ravel(), sel_g.cpu().numpy().ravel()
        wv, wgv = w.cpu().numpy().ravel().astype(np.float32), w_g.cpu().numpy().ravel().astype(np.float32)
        want = np.zeros((T, H), np.float32)
        for t in range(T):
            o = np.zeros(H, np.float32)
            for k in range(topk):
                i = t * topk + k
                if sg[i] < 0 or wgv[i] == 0 or inv[i] < 0:
                    continue
                o = o + np.float32(wgv[i]) * y[inv[i]]
            part, any_cpu = np.zeros(H, np.float32), False
            for k in range(topk):
                i = t * topk + k
                if sg[i] == -1 and s[i] != -1:
                    part = part + np.float32(wv[i]) * y[inv[i]]
                    any_cpu = True
                    ncpu += 1
            want[t] = o + part if any_cpu else o
        got = out.cpu().numpy()
        say("cpu lane step", step, "layer", li, "T", T, "cpu picks", int(np.sum((sg == -1) & (s != -1))),
            "max diff", float(np.abs(got - want).max()))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), step
    assert ncpu > 0
    say("agent", slots.agent_status())
    slots.close()


def test_plan_reply_timeout_is_reported(cuda):
    """The agent's thread held back (forced from the host; the wait limit 20 ms; every kernel ends by itself): the
    planned step's bounded wait for its reply runs out, the step admits nothing and masks nothing (its misses run from
    their homes), and the agent reports the failure."""
    import bmx
    E, topk = 12, 3
    layers = small_layers(1, E, 256, 128, 160, "host")
    slots = bmx.ExpertSlots(layers, 6, maxj=4, copies="dma")
    slots.plan(None)
    lib = bmx.lib()
    bmx._lib.check(lib.bmx_copy_agent_control(slots.agent, 1, 20000), "bmx_copy_agent_control")
    sel = torch.tensor([[0, 4, 7]], dtype=torch.int64, device="cuda")
    w = torch.ones((1, topk), dtype=torch.float16, device="cuda")
    torch.cuda.synchronize()
    say("plan timeout: planned step with the agent held")
    sg, wg, ln, _ = slots.step_planned(0, sel, w)
    torch.cuda.synchronize()
    assert torch.equal(sg, sel.view(-1)) and torch.equal(wg, w.view(-1))
    assert ln.tolist() == [bmx.LANE_HOME] * 3
    assert int(slots.ctl[2].item()) == 0 and int((slots.slotof >= 0).sum().item()) == 0
    with pytest.raises(bmx.BmxError, match="ran out of time"):
        slots.check()
    bmx._lib.check(lib.bmx_copy_agent_control(slots.agent, 0, 0), "bmx_copy_agent_control")
    slots.close()


@pytest.mark.parametrize("copy", [False, True])
def test_cpu_lane_fast_partial_added(cuda, oracle, copy):
    """The same layer calls with the CPU lane in its fast mode (policy cpu_fast): out = the GPU's combine of the masked
    selection + the fast lane's partial, within the layer tolerance of the all-GPU rows' combine (the fast mode keeps the
    exact weights but not the device's summation order). copy: the lane reads its own copy of the homes."""
    import bmx
    from bmx import synth
    Lyr, E, H, I, topk, first = 2, 16, 256, 128, 4, 0
    dev_layers = small_layers(Lyr, E, H, I, 150, "device")
    host_layers = small_layers(Lyr, E, H, I, 150, "host")
    slots = bmx.ExpertSlots(host_layers, 6, maxj=2, copies="dma")
    slots.cpu_lane(topk, threads=4, copy=copy)
    slots.plan(dict(cpu_on=1, max_cpu=2, cpu_fast=1, gpu_base_us=1.0, gpu_admit_us=1.0))
    kw = dict(score=bmx.SCORE_SIGMOID, renorm=True, scale=1.0)
    ref_layers = [bmx.MoELayer(dev_layers[li], topk, **kw) for li in range(Lyr)]
    st_layers = [bmx.MoELayer(host_layers[li], topk, slots=slots, li=li, **kw) for li in range(Lyr)]
    rng = np.random.default_rng(31)
    ncpu = 0
    for step in range(8):
        li = step % Lyr
        T = 1 + step % 3
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16)).cuda()
        lg = torch.from_numpy(synth.zipf_logits(T, E, 1.1, seed=500 + step)).cuda()
        m = st_layers[li]
        sel, w = m.routing_fn(T, None, x, {"logits": lg})
        sel_g, w_g, flag = m.layer(li, sel, w, x, T)
        assert flag
        out = m.cpu_split_combine(m.combine(m.run_bszN(x, sel_g, w_g, bmx.PATH_DECODE)), None, False, None)
        want = ref_layers[li].run_bszN(x, sel, w, bmx.PATH_DECODE)
        torch.cuda.synchronize()
        got, want = out.cpu().numpy(), want.cpu().numpy()
        s, sg = sel.cpu().numpy().ravel(), sel_g.cpu().numpy().ravel()
        n = int(np.sum((sg == -1) & (s != -1)))
        ncpu += len(set(s[(sg == -1) & (s != -1)].tolist()))       # the planner counts experts, not picks
        err = float(np.sqrt(np.mean((got - want) ** 2)) / np.sqrt(np.mean(want ** 2)))
        say("fast cpu lane step", step, "layer", li, "T", T, "cpu picks", n, "max diff", float(np.abs(got - want).max()),
            "rel rms", err)
        assert np.abs(got - want).max() < 1e-2 and err < 1e-3, step
    assert ncpu > 0
    st = slots.plan_stats()
    say("plan stats", st)
    assert st[1] == ncpu and st[2] >= 1
    slots.close()


def test_plan_measured_cpu_cost(cuda, oracle):
    """Policy cpu_measured: the fast mode's mean is seeded when the lane is set up; the exact mode's starts empty, so with
    every cost 0 the first call's misses go to the CPU lane (its finish is then no later); once its job has run the
    planner prices a CPU expert at the worker's measured time per pick, which no longer ties with a GPU costing 0, so
    later calls put nothing there. The outputs stay the all-GPU rows' within the layer tolerance throughout."""
    import bmx
    from bmx import synth
    Lyr, E, H, I, topk = 2, 16, 256, 128, 4
    dev_layers = small_layers(Lyr, E, H, I, 160, "device")
    host_layers = small_layers(Lyr, E, H, I, 160, "host")
    slots = bmx.ExpertSlots(host_layers, 6, maxj=2, copies="dma")
    slots.cpu_lane(topk, threads=2)
    slots.plan(dict(cpu_on=1, max_cpu=2, cpu_fast=1, cpu_measured=1))
    assert slots.plan_stats()[4] > 0                                   # the fast mode's seed
    slots.plan(dict(cpu_on=1, max_cpu=2, cpu_fast=0, cpu_measured=1))
    assert slots.plan_stats()[4] == 0                                  # no exact-mode job yet
    kw = dict(score=bmx.SCORE_SIGMOID, renorm=True, scale=1.0)
    ref_layers = [bmx.MoELayer(dev_layers[li], topk, **kw) for li in range(Lyr)]
    st_layers = [bmx.MoELayer(host_layers[li], topk, slots=slots, li=li, **kw) for li in range(Lyr)]
    rng = np.random.default_rng(37)
    seen = []
    for step in range(6):
        li = step % Lyr
        x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float16)).cuda()
        lg = torch.from_numpy(synth.zipf_logits(1, E, 1.1, seed=700 + step)).cuda()
        m = st_layers[li]
        sel, w = m.routing_fn(1, None, x, {"logits": lg})
        sel_g, w_g, flag = m.layer(li, sel, w, x, 1)
        assert flag
        out = m.cpu_split_combine(m.combine(m.run_bszN(x, sel_g, w_g, bmx.PATH_DECODE)), None, False, None)
        want = ref_layers[li].run_bszN(x, sel, w, bmx.PATH_DECODE)
        torch.cuda.synchronize()
        got, want = out.cpu().numpy(), want.cpu().numpy()
        err = float(np.sqrt(np.mean((got - want) ** 2)) / np.sqrt(np.mean(want ** 2)))
        st = slots.plan_stats()
        seen.append(st)
        say("measured-cost step", step, "plan stats", st, "rel rms", err)
        assert np.abs(got - want).max() < 1e-2 and err < 1e-3, step
    assert seen[0][1] == 2 and seen[0][2] >= 1 and seen[0][4] > 0      # the first call's two misses ran on the CPU
    assert all(s[1] == seen[0][1] for s in seen[1:])                   # and, priced as measured, nothing after it
    slots.close()

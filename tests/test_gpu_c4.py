"""The 43-layer decode stack's slot-table workload at its real layer shape, on the GPU: GLM-shaped layers (288 routed
experts top-8 sigmoid + bias, one shared expert kept in VRAM, H 4096, I 1536, EXL3 3 bpw) whose routed experts live in
pinned host memory, a VRAM slot table holding 30 % of them (warmed with each layer's most popular experts), Zipf(1.1)
routing with a per-layer permutation, and the copy agent staging misses on the DMA engines. Eight layers (16 GB of
pinned homes) stand in for the 43: every layer of the stack runs the same code on its own table rows.

Checks, for every token: each layer's output is bit-identical to the same layer with every expert resident in device
memory, and the slot table's state (slot of every expert, owners, reference bits, pins, CLOCK hand, step counter,
counters, fresh flags, every expert-table pointer) is bit-exact against the oracle's CLOCK table replaying the same picks
(the reference's Pool.step / ec_step_k semantics, engine/tiers.py:360-373 and engine/ec.py:16-105). The planned variant
runs every step as a request answered by the copy agent's planner (its default policy: every miss admitted), the
reference's publish / reply protocol (engine/kernels/nv2/nv2_dev.cu:221-367, nv2_host.cpp:947-1133), with the same
checks."""
import numpy as np
import pytest
import torch

from test_gpu_slots import check_state

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("planned", [False, True])
def test_c4_stack_staged_matches_resident(cuda, oracle, planned):
    import bmx
    from bmx import synth
    c = synth.CONFIGS["c4"]
    NL, E, H, I, topk = 8, c["E"], c["H"], c["I"], c["topk"]
    S = int(round(c["cache_frac"] * NL * E))
    maxj, NTOK = 16, 48
    fm = (bmx.TF_K3,) * 3
    say(f"c4 stack: {NL} layers x {E} experts, H {H}, I {I}, {S} slots; building pinned homes and device twins")
    host_layers, dev_layers = [], []
    for li in range(NL):
        t = bmx.ExpertTable.random(H, I, E, fm, shared=True, seed=500 + li, device=cuda, home="host")
        t.shared_to_device()
        host_layers.append(t)
        dev_layers.append(bmx.ExpertTable.random(H, I, E, fm, shared=True, seed=500 + li, device=cuda))
        say("c4 stack: layer", li, "built")
    rng = np.random.default_rng(43)
    biases = [torch.from_numpy((rng.standard_normal(E) * 0.1).astype(np.float32)).to(cuda) for _ in range(NL)]
    kw = dict(score=c["score"], renorm=c["renorm"], scale=c["scale"])
    slots = bmx.ExpertSlots(host_layers, S, maxj=maxj, copies="dma")
    st = [bmx.MoELayer(host_layers[li], topk, bias=biases[li], slots=slots, li=li, **kw) for li in range(NL)]
    rf = [bmx.MoELayer(dev_layers[li], topk, bias=biases[li], **kw) for li in range(NL)]
    ref = oracle.SlotTable(NL, E, S)
    # warm: each layer's S // NL most popular experts (the Zipf ranks of its permutation), maxj per step, as the stack's
    # bench warms it; the oracle replays the same steps
    per = S // NL
    for li in range(NL):
        perm = np.random.default_rng(7919 * (li + 1)).permutation(E)
        top = [int(e) for e in perm[:per]]
        slots.warm(li, top)
        for i in range(0, len(top), maxj):
            ref.step(li, np.array(top[i:i + maxj], np.int64), 0, True, maxj)
    check_state(slots, ref, ref.fresh.copy(), "warm")
    say("c4 stack: warmed, stats", slots.stats(), "planned" if planned else "")
    if planned:
        slots.plan(None)
    lgs = [synth.zipf_logits(NTOK, E, 1.1, seed=li, perm_seed=7919 * (li + 1)) for li in range(NL)]
    for tok in range(NTOK):
        for li in range(NL):
            x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float16)).to(cuda)
            lg = torch.from_numpy(lgs[li][tok:tok + 1]).to(cuda)
            sel, w = rf[li].routing_fn(1, None, x, {"logits": lg})
            want = rf[li].run_bszN(x, sel, w)
            sel2, w2 = st[li].routing_fn(1, None, x, {"logits": lg})
            sel3, w3, _ = st[li].layer(li, sel2, w2, x, 1)
            got = st[li].combine(st[li].run_bszN(x, sel3, w3))
            ref.step(li, sel2.cpu().numpy(), 0, True, maxj)
            torch.cuda.synchronize()
            assert torch.equal(sel, sel2) and torch.equal(w, w2), (tok, li)
            assert torch.equal(sel3, sel2) and torch.equal(w3, w2), (tok, li)
            assert torch.equal(got, want), (tok, li)
        check_state(slots, ref, ref.fresh.copy(), f"token {tok}")
        if tok % 12 == 11:
            say("c4 stack: token", tok, "stats", slots.stats(), "agent", slots.agent_status())
    h, m, adm, novic, ev = slots.stats()[:5]
    say("c4 stack: hits", h, "misses", m, "admissions", adm, "evictions", ev)
    assert m > 0 and adm > 0 and ev > 0 and h > m
    slots.close()

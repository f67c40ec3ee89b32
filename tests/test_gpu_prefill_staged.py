"""Staged prefill through the expert-slot table, on the GPU: a stack of DeepSeek-shaped layers (384 routed experts,
group-limited top-6, H 4096, I 2048, EXL3 K 2 / K 3) whose experts live in pinned host memory, a VRAM slot table holding
30 % of them (each layer's most popular experts), and 8192-token prefill chunks with Zipf(1.1) routing.

A prefill-size call (at least stage_min picks) admits nothing: the step marks hits only, every expert of the layer that
is not resident is copied into one of two staging arenas one layer ahead, the layer's table points there for its
products and back afterwards (the reference's staged prefill: engine/nv2.py:378-386, engine/tiers.py:395-463,
engine/kernels/nv2/nv2_host.cpp:1512-1593, nv_restore_k engine/kernels/nv2/nv2_dev.cu:554-566).

Checks: every layer's output is bit-identical to the same layer with all experts resident in device memory; while a
layer computes, its table points each non-resident expert at its staging record; after each forward the slot table's
state (slots, owners, reference bits, pins, hand, step counter, counters, fresh flags, every table pointer) is
bit-exact against the oracle's CLOCK table replaying hits-only steps of the same picks."""
import numpy as np
import pytest
import torch

from test_gpu_slots import check_state, tables_of

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("copies", ["kernel", "dma"])
def test_c3_stack_staged_prefill_matches_resident(cuda, oracle, copies):
    import bmx
    from bmx import synth
    c = synth.CONFIGS["c3"]
    NL, E, H, I, topk, T = 3, c["E"], c["H"], c["I"], c["topk"], c["T"]
    S = int(round(0.30 * NL * E))
    maxj = 16
    fm = synth.formats("c3", E, False)
    say(f"staged prefill ({copies}): {NL} layers x {E} experts, H {H}, I {I}, {S} slots; building homes and twins")
    host_layers, dev_layers = [], []
    for li in range(NL):
        host_layers.append(bmx.ExpertTable.random(H, I, E, fm, seed=900 + li, device=cuda, home="host"))
        dev_layers.append(bmx.ExpertTable.random(H, I, E, fm, seed=900 + li, device=cuda))
        say("staged prefill: layer", li, "built")
    kw = dict(score=c["score"], renorm=c["renorm"], scale=c["scale"], n_group=c["n_group"], topk_group=c["topk_group"])
    slots = bmx.ExpertSlots(host_layers, S, maxj=maxj, copies=copies)
    st = [bmx.MoELayer(host_layers[li], topk, slots=slots, li=li, **kw) for li in range(NL)]
    rf = [bmx.MoELayer(dev_layers[li], topk, **kw) for li in range(NL)]
    ref = oracle.SlotTable(NL, E, S)
    per = S // NL
    for li in range(NL):
        perm = np.random.default_rng(40 + li).permutation(E)        # the permutation of layer li's Zipf routing
        top = [int(e) for e in perm[:per]]
        slots.warm(li, top)
        for i in range(0, len(top), maxj):
            ref.step(li, np.array(top[i:i + maxj], np.int64), 0, True, maxj)
    check_state(slots, ref, ref.fresh.copy(), "warm")
    rec = host_layers[0].rec
    for fwd in range(2):
        for li in range(NL):
            x, lg, _ = synth.inputs("c3", T=T, seed=40 + li, device=cuda)
            if fwd:
                x = (x.float() * 0.5).half()
            m = st[li]
            sel, w = m.routing_fn(T, None, x, {"logits": lg})
            say(f"staged prefill ({copies}): forward {fwd} layer {li}: layer call")
            sg, wg, flag = m.layer(li, sel, w, x, T)
            assert sg is sel and wg is w and not flag and m._staged == li
            if fwd == 0 and li == 1:
                # while the layer computes, its non-resident experts point at their staging records, in order
                ex = slots.st_layers[li][0]
                b = slots.st_buf[li % 2].data_ptr()
                tr = tables_of(slots)[li]
                assert len(ex) == E - per
                for j, e in enumerate(ex.tolist()):
                    assert tuple(int(v) for v in tr[e]) == (b + j * rec, b + j * rec + host_layers[0].off_u,
                                                            b + j * rec + host_layers[0].off_d), (li, j, e)
            out = m.run_bszN(x, sg, wg)
            want = rf[li].run_bszN(x, sel, w)
            torch.cuda.synchronize()
            same = torch.equal(out.view(torch.int32), want.view(torch.int32))
            say(f"staged prefill ({copies}): forward {fwd} layer {li}: bit-identical {same}, "
                f"max diff {float((out - want).abs().max())}")
            assert same, (fwd, li)
            ref.step(li, sel.cpu().numpy().ravel(), 0, False, maxj)
        check_state(slots, ref, np.zeros(E, np.int32), f"forward {fwd}")
        say(f"staged prefill ({copies}): forward {fwd} stats {slots.st_stats}")
    assert slots.st_stats["forwards"] == 2 and slots.st_stats["layers"] == 2 * NL
    assert slots.st_stats["experts"] == 2 * NL * (E - per)
    slots.close()

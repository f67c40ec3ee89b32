"""CPU expert lane against the device, bit for bit: the host emulation of v_dot2_f32_f16 against the instruction over
random, cancelling, accumulator-dominated, subnormal and carry / borrow operands; expert y rows from the lane against
the GPU decode path's for several batch sizes, formats and activations; and a layer whose chosen experts come from the
lane, combined on the GPU, against the all-GPU layer."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def f16_bits(rng, n, lo, hi):
    e = rng.integers(lo, hi + 1, n).astype(np.uint16)
    return (rng.integers(0, 2, n).astype(np.uint16) << 15) | (e << 10) | rng.integers(0, 1024, n).astype(np.uint16)


def dot2_cases(n=200_000, seed=7):
    rng = np.random.default_rng(seed)
    A, B, C = [], [], []
    h = lambda x: x.view(np.float16).astype(np.float64)
    for kind in range(6):
        a = f16_bits(rng, 2 * n, 4 if kind != 3 else 0, 26 if kind != 3 else 4).reshape(-1, 2)
        b = f16_bits(rng, 2 * n, 4 if kind != 3 else 0, 26 if kind != 3 else 9).reshape(-1, 2)
        S = h(a[:, 0]) * h(b[:, 0]) + h(a[:, 1]) * h(b[:, 1])
        es = np.floor(np.log2(np.maximum(np.abs(S), 1e-30)))
        if kind == 0:      # c of the products' size
            c = S * rng.uniform(-2, 2, n)
        elif kind == 1:    # cancelling products
            a[:, 1] = a[:, 0] ^ 0x8000
            b[:, 1] = b[:, 0] ^ rng.integers(0, 4, n).astype(np.uint16)
            c = rng.standard_normal(n) * 2.0 ** rng.integers(-20, 0, n)
        elif kind == 2:    # c far above the products
            c = rng.choice([-1.0, 1.0], n) * 2.0 ** np.clip(es + rng.integers(3, 40, n), -120, 120) * rng.uniform(1, 2, n)
        elif kind == 3:    # subnormal operands, tiny c
            c = rng.standard_normal(n) * 2.0 ** rng.integers(-149, -100, n)
        elif kind == 4:    # c just below a power of two, same sign as the products: the sum carries
            k = np.clip(es + rng.integers(-2, 31, n), -120, 120)
            c = np.sign(S) * 2.0 ** k * (1 - rng.uniform(0, 2.0 ** -rng.integers(1, 24, n)))
        else:              # c just above a power of two, opposite sign: the sum borrows
            k = np.clip(es + rng.integers(-2, 31, n), -120, 120)
            c = -np.sign(S) * 2.0 ** k * (1 + rng.uniform(0, 2.0 ** -rng.integers(1, 24, n)))
        A.append(a); B.append(b); C.append(c.astype(np.float32))
    pack = lambda x: (x[:, 0].astype(np.uint32) | (x[:, 1].astype(np.uint32) << 16))
    return pack(np.concatenate(A)), pack(np.concatenate(B)), np.concatenate(C)


def test_dot2_emulation_matches_device(cuda):
    import bmx
    from bmx import cpu_lane
    a, b, c = dot2_cases()
    n = c.size
    say("dot2 cases", n)
    ta, tb = torch.from_numpy(a.view(np.int32)).cuda(), torch.from_numpy(b.view(np.int32)).cuda()
    tc, to = torch.from_numpy(c).cuda(), torch.empty(n, dtype=torch.float32, device="cuda")
    assert ta.numel() == tb.numel() == tc.numel() == to.numel() == n
    bmx._lib.check(bmx.lib().bmx_dot2_f32_f16(ta.data_ptr(), tb.data_ptr(), tc.data_ptr(), to.data_ptr(), n,
                                              torch.cuda.current_stream().cuda_stream), "bmx_dot2_f32_f16")
    dev = to.cpu().numpy()
    emu = cpu_lane.dot2(a, b, c)
    bad = np.flatnonzero(dev.view(np.uint32) != emu.view(np.uint32))
    say("dot2 mismatches", bad.size)
    assert bad.size == 0, (bad[:5], dev[bad[:5]], emu[bad[:5]])


CASES = [
    # T, formats, act, gated, limit, shared
    (1, ((2, 0, 3), (1, 1, 1), (3, 3, 3), (2, 2, 2)), 0, True, 0.0, True),
    (4, ((2, 2, 2),), 2, True, 0.0, False),
    (9, ((3, 1, 0), (2, 2, 2)), 3, True, 7.0, True),
    (3, ((1, 2, 3),), 1, True, 0.0, False),
    (2, ((2, 2, 2),), 0, False, 0.0, True),
]


@pytest.mark.parametrize("T,fmts,act,gated,limit,shared", CASES)
def test_cpu_lane_rows_bitexact(cuda, T, fmts, act, gated, limit, shared):
    import bmx
    from bmx import cpu_lane
    H, I, E, topk = 512, 256, 8, 3
    fm = [fmts[e % len(fmts)] for e in range(E + (1 if shared else 0))]
    tab = bmx.ExpertTable.random(H, I, E, fm, shared=shared, seed=T * 13 + act, device=cuda)
    rng = np.random.default_rng(T)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16)).to(cuda)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16)).to(cuda)
    sel, w = bmx.ops.router_topk(lg, topk, None, 1, 1, bmx.SCORE_SIGMOID, True, 1.0)
    desc = tab.desc(topk, act=act, gated=gated, act_limit=limit)
    routes = bmx.ops.dispatch(sel, E, 0, shared, bmx.lib().bmx_rows_per_group(T, topk, bmx.PATH_DECODE))
    y, _ = bmx.ops.moe_experts(desc, x, routes, path=bmx.PATH_DECODE)
    torch.cuda.synchronize()
    ks_gu, ks_dn, grouped = cpu_lane.decode_splits(desc, T)
    say("case T", T, "act", act, "splits", ks_gu, ks_dn, "grouped", grouped)
    y = y.cpu().numpy()
    rt = routes.row_token.cpu().numpy()
    offs = routes.offsets.cpu().numpy()
    xs = x.cpu().numpy()
    nrows = int(offs[E + (1 if shared else 0)])
    checked = 0
    for e in range(E + (1 if shared else 0)):
        r0, r1 = int(offs[e]), int(offs[e + 1])
        if r1 <= r0:
            continue
        yc = cpu_lane.expert_rows(tab.host_expert(e), H, I, xs[rt[r0:r1]], ks_gu, ks_dn, grouped, act, gated, limit)
        eq = yc.view(np.uint32) == y[r0:r1].view(np.uint32)
        assert eq.all(), (e, float(eq.mean()), np.abs(yc - y[r0:r1]).max())
        checked += r1 - r0
    assert checked == nrows
    say("rows bit-identical", checked)


def test_layer_with_cpu_experts_bitexact(cuda):
    """One token through a layer: the experts of two of its picks computed by the CPU lane, their y rows put in place of
    the GPU's, combined in slot order on the GPU: the all-GPU layer output, bit for bit."""
    import bmx
    from bmx import cpu_lane
    H, I, E, topk, T = 512, 256, 16, 4, 1
    tab = bmx.ExpertTable.random(H, I, E, (bmx.TF_K3,) * 3, shared=True, seed=3, device=cuda)
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16)).to(cuda)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16)).to(cuda)
    sel, w = bmx.ops.router_topk(lg, topk, None, 1, 1, bmx.SCORE_SIGMOID, True, 1.0)
    desc = tab.desc(topk)
    want = bmx.ops.moe_forward(desc, x, sel, w, bmx.PATH_DECODE)
    routes = bmx.ops.dispatch(sel, E, 0, True, bmx.lib().bmx_rows_per_group(T, topk, bmx.PATH_DECODE))
    y, _ = bmx.ops.moe_experts(desc, x, routes, path=bmx.PATH_DECODE)
    ks_gu, ks_dn, grouped = cpu_lane.decode_splits(desc, T)
    offs = routes.offsets.cpu().numpy()
    picks = sel.cpu().numpy().ravel()[:2]
    yh = y.cpu().numpy()
    for e in picks:
        r0, r1 = int(offs[e]), int(offs[e + 1])
        yh[r0:r1] = cpu_lane.expert_rows(tab.host_expert(int(e)), H, I, x.cpu().numpy(), ks_gu, ks_dn, grouped)
    got = bmx.ops.combine(torch.from_numpy(yh).to(cuda), routes, w, H)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_cpu_lane_rows_bitexact_sequential_splits(cuda):
    """A launch large enough that the gate / up epilogue sums the k-splits in sequence (not in four groups): rows of
    two experts from the lane against the GPU's, bit for bit."""
    import bmx
    from bmx import cpu_lane
    H, I, E, topk, T = 256, 4096, 8, 3, 171
    tab = bmx.ExpertTable.random(H, I, E, [(2, 0, 3), (1, 1, 1)] * 4, seed=11, device=cuda)
    rng = np.random.default_rng(11)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16)).to(cuda)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16)).to(cuda)
    sel, w = bmx.ops.router_topk(lg, topk, None, 1, 1, bmx.SCORE_SIGMOID, True, 1.0)
    desc = tab.desc(topk)
    routes = bmx.ops.dispatch(sel, E, 0, False, bmx.lib().bmx_rows_per_group(T, topk, bmx.PATH_DECODE))
    y, _ = bmx.ops.moe_experts(desc, x, routes, path=bmx.PATH_DECODE)
    torch.cuda.synchronize()
    ks_gu, ks_dn, grouped = cpu_lane.decode_splits(desc, T)
    say("sequential case splits", ks_gu, ks_dn, "grouped", grouped)
    assert grouped == 0
    y = y.cpu().numpy()
    rt = routes.row_token.cpu().numpy()
    offs = routes.offsets.cpu().numpy()
    xs = x.cpu().numpy()
    for e in (0, 1):
        r0, r1 = int(offs[e]), int(offs[e + 1])
        r1 = min(r1, r0 + 24)
        yc = cpu_lane.expert_rows(tab.host_expert(e), H, I, xs[rt[r0:r1]], ks_gu, ks_dn, grouped, threads=16)
        assert (yc.view(np.uint32) == y[r0:r1].view(np.uint32)).all(), e
        say("expert", e, "rows bit-identical", r1 - r0)


def test_cpu_lane_time_c2_expert(cuda):
    """Reported, not asserted: one C2-shaped expert (H 4096, I 1536, K 3) for one token on the host's cores, the exact
    lane once, the fast mode warm (one expert again and again) and cold (32 experts in turn, 227 MB)."""
    import time
    import os
    import bmx
    from bmx import cpu_lane
    H, I = 4096, 1536
    tab = bmx.ExpertTable.random(H, I, 32, (bmx.TF_K3,) * 3, seed=2, device=cuda)
    exs = [tab.host_expert(e) for e in range(32)]
    x = np.random.default_rng(2).standard_normal((1, H)).astype(np.float16)
    th = min(16, os.cpu_count() or 1)
    t0 = time.perf_counter()
    cpu_lane.expert_rows(exs[0], H, I, x, 16, 4, 1, threads=th)
    say(f"cpu lane: one C2 expert, one token, {th} threads: {(time.perf_counter() - t0) * 1e3:.1f} ms")
    cpu_lane.expert_rows_fast(exs[0], H, I, x, threads=th)
    warm, cold = [], []
    for _ in range(10):
        t0 = time.perf_counter()
        cpu_lane.expert_rows_fast(exs[0], H, I, x, threads=th)
        warm.append(time.perf_counter() - t0)
    for e in range(1, 32):
        t0 = time.perf_counter()
        cpu_lane.expert_rows_fast(exs[e], H, I, x, threads=th)
        cold.append(time.perf_counter() - t0)
    say(f"cpu lane fast mode: one C2 expert, one token, {th} threads: warm {np.median(warm) * 1e6:.0f} us, "
        f"cold {np.median(cold) * 1e6:.0f} us (medians)")


def test_layer_verify_on_cpu_finds_a_flipped_bit(cuda):
    """MoELayer.verify_on_cpu: the GPU's expert rows agree with the exact CPU lane; one flipped low bit in a copy of the
    GPU's rows (planted on the host) is reported at its row."""
    import bmx
    H, I, E, topk, T = 512, 256, 12, 4, 3
    tab = bmx.ExpertTable.random(H, I, E, (bmx.TF_K3, bmx.TF_K2, bmx.TF_K4), shared=True, seed=21, device=cuda)
    layer = bmx.MoELayer(tab, topk, score=bmx.SCORE_SIGMOID, renorm=True, scale=1.0, act=bmx.ACT_GELU)
    rng = np.random.default_rng(21)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16)).to(cuda)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16)).to(cuda)
    sel, w = layer.routing_fn(T, None, x, {"logits": lg})
    assert layer.verify_on_cpu(x, sel, w) == []
    routes = bmx.ops.dispatch(sel, E, 0, True, bmx.lib().bmx_rows_per_group(T, topk, bmx.PATH_DECODE))
    y, _ = bmx.ops.moe_experts(layer.desc, x, routes, path=bmx.PATH_DECODE)
    yb = y.cpu().numpy().copy()
    r = 5
    yb.view(np.uint32)[r, 100] ^= 1
    bad = layer.verify_on_cpu(x, sel, w, y_rows=torch.from_numpy(yb))
    assert [b[0] for b in bad] == [r]

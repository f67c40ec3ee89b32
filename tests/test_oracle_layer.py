"""Pins the oracle's expert and layer forward: against an fp64 model built from the mathematics (dense Hadamard
matrices, exact products), against the reference's CPU lane (moe_forward4, golden outputs and the live library), and
against the reference's own routing-post-process known answers (dropped picks)."""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _hm():
    from scipy.linalg import hadamard
    return hadamard(128).astype(np.float64) / np.sqrt(128)


def make_expert(oracle, rng, H, I, fmts=(2, 2, 2)):
    ex = {"tr": [], "suh": [], "svh": [], "fmt": list(fmts)}
    for m, (k, n) in enumerate(((H, I), (H, I), (I, H))):
        ex["tr"].append(rng.integers(0, 256, (k // 16) * (n // 16) * oracle.TF_TB[fmts[m]], dtype=np.uint8))
        ex["suh"].append(rng.uniform(0.5, 1.5, k).astype(np.float16))
        ex["svh"].append((rng.uniform(0.5, 1.5, n) / np.sqrt(k)).astype(np.float16))
    return ex


def expert64(oracle, ex, H, I, x):
    """fp64 reference: y = svh_d * Hd(Wd^T Hd(suh_d * a)) with a = silu(g) * u, g / u the same for gate / up."""
    Hm = _hm()

    def blk(v):
        return (v.reshape(-1, 128) @ Hm).reshape(-1)

    def lin(m, v):
        k, n = ((H, I), (H, I), (I, H))[m]
        W = oracle.np_dequant(ex["tr"][m], ex["fmt"][m], k, n).astype(np.float64)
        return blk(blk(v * ex["suh"][m].astype(np.float64)) @ W) * ex["svh"][m].astype(np.float64)
    g = lin(0, x)
    u = lin(1, x)
    return lin(2, g / (1 + np.exp(-g)) * u)


def rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("fmts", [(2, 2, 2), (0, 1, 3), (3, 3, 0)])
def test_expert_vs_fp64_model(oracle, fmts):
    rng = np.random.default_rng(sum(fmts))
    H, I = 512, 256
    ex = make_expert(oracle, rng, H, I, fmts)
    x = rng.standard_normal(H).astype(np.float16)
    y, g, u, a = oracle.expert_forward(ex, H, I, x)
    want = expert64(oracle, ex, H, I, x.astype(np.float64))
    assert rel(y, want) < 2e-3                  # fp16 storage of xt, gate, up, act: ~5e-4 each
    assert np.abs(y - want).max() < 1e-2
    # a wrong sign, index or transposition in any stage moves the result by O(1)
    ex2 = dict(ex, suh=[ex["suh"][0], ex["suh"][1], ex["suh"][2][::-1].copy()])
    y2, *_ = oracle.expert_forward(ex2, H, I, x)
    assert rel(y2, want) > 0.1


def test_expert_intermediates(oracle):
    """gate / up are RN16 of xt . W; act is the rotated fp16 down input."""
    rng = np.random.default_rng(5)
    H, I = 256, 128
    ex = make_expert(oracle, rng, H, I)
    x = rng.standard_normal(H).astype(np.float16)
    y, g, u, a = oracle.expert_forward(ex, H, I, x)
    xt = oracle.prep(x, ex["suh"][0]).astype(np.float64)
    Wg = oracle.dequant(ex["tr"][0], 2, H, I).astype(np.float64)
    assert np.array_equal(g, (xt @ Wg).astype(np.float32).astype(np.float16))


def test_layer_matches_reference_lane_golden(oracle):
    z = np.load(os.path.join(GOLD, "lane.npz"))
    H, I, E = int(z["H"]), int(z["I"]), int(z["E"])
    exps = []
    for e in range(E):
        exps.append({"tr": [z["trellis"][3 * e + m] for m in range(3)],
                     "suh": [z["suh"][sum((H, H, I)[:m]) + e * (2 * H + I): sum((H, H, I)[:m]) + e * (2 * H + I) + (H, H, I)[m]] for m in range(3)],
                     "svh": [z["svh"][sum((I, I, H)[:m]) + e * (2 * I + H): sum((I, I, H)[:m]) + e * (2 * I + H) + (I, I, H)[m]] for m in range(3)],
                     "fmt": [2, 2, 2]})
    out = oracle.moe_forward(exps, 0, None, H, I, z["x"], z["sel"].astype(np.int64), z["w"])
    # the reference lane rounds at different points (fp16 after svh, fp16 activation) and EXACT sums in fp32:
    # distance of the same order as the GPU-vs-CPU figures it documents (~8e-4, docs/x16.md:62-68)
    assert rel(z["exact"], out) < 2e-3
    assert rel(z["affine"], out) < 3e-3
    assert rel(z["i16"], out) < 3e-3


def test_layer_matches_live_reference_lane(oracle, ref):
    import ctypes
    rng = np.random.default_rng(9)
    H, I, E, T, topk = 512, 256, 6, 4, 3
    exps = [make_expert(oracle, rng, H, I) for _ in range(E)]
    x = rng.standard_normal((T, H)).astype(np.float16)
    sel = np.array([[0, 2, 5], [1, 2, 3], [5, 4, 0], [3, 1, 2]], np.int64)
    w = rng.uniform(0.1, 0.5, (T, topk)).astype(np.float16)
    cpus = (ctypes.c_int * 2)(0, 1)
    assert ref.ref_lane_create(H, I, E, 2, cpus, 0.0) == 0
    try:
        keep = []
        for e, ex in enumerate(exps):
            sc = [ex["suh"][0], ex["svh"][0], ex["suh"][1], ex["svh"][1], ex["suh"][2], ex["svh"][2]]
            sc = [np.ascontiguousarray(a.view(np.uint16)) for a in sc]
            keep += sc
            ref.ref_lane_set_expert(e, *[t.ctypes.data for t in ex["tr"]], *[a.ctypes.data for a in sc], 2, 2, 2)
        lane = np.zeros((T, H), np.float32)
        xf, si, wf = x.astype(np.float32), sel.astype(np.int32), w.astype(np.float32)
        ref.ref_lane_forward(xf.ctypes.data, T, si.ctypes.data, wf.ctypes.data, topk, lane.ctypes.data, 1)
    finally:
        ref.ref_lane_destroy()
    out = oracle.moe_forward(exps, 0, None, H, I, x, sel, w)
    assert rel(lane, out) < 2e-3


def test_layer_is_weighted_sum_of_experts_plus_shared(oracle):
    rng = np.random.default_rng(21)
    H, I, E = 256, 128, 3
    exps = [make_expert(oracle, rng, H, I) for _ in range(E)]
    sh = make_expert(oracle, rng, H, I)
    x = rng.standard_normal((2, H)).astype(np.float16)
    sel = np.array([[2, 0], [1, 2]], np.int64)
    w = np.array([[0.75, 0.25], [0.5, 0.125]], np.float16)
    out = oracle.moe_forward(exps, 0, sh, H, I, x, sel, w)
    for t in range(2):
        want = sum(np.float32(w[t, k]) * oracle.expert_forward(exps[sel[t, k]], H, I, x[t])[0] for k in range(2))
        want = want + oracle.expert_forward(sh, H, I, x[t])[0]
        assert np.allclose(out[t], want, rtol=1e-6, atol=1e-6)
    # rows subset: same values
    sub = oracle.moe_forward(exps, 0, sh, H, I, x, sel, w, rows=np.array([1], np.int32))
    assert np.array_equal(sub[0], out[1])


def test_dropped_picks_reference_known_answer(oracle):
    """tests/test_warm_prefill.py:36-46 of the reference: cold expert 1 of E = 4 dropped -> sentinel id first + E and
    weight 0, renormalised to [[0.8, 0], [0.5, 0.5], [0, 0]]. A dropped pick contributes nothing."""
    rng = np.random.default_rng(4)
    H, I, E = 256, 128, 4
    exps = [make_expert(oracle, rng, H, I) for _ in range(E)]
    x = rng.standard_normal((3, H)).astype(np.float16)
    sel = np.array([[0, 4], [2, 3], [4, 4]], np.int64)
    w = np.array([[0.8, 0.0], [0.5, 0.5], [0.0, 0.0]], np.float16)
    out = oracle.moe_forward(exps, 0, None, H, I, x, sel, w)
    y0 = oracle.expert_forward(exps[0], H, I, x[0])[0]
    assert np.array_equal(out[0], np.float32(np.float16(0.8)) * y0)
    assert np.all(out[2] == 0)
    # first offset: ids 7.. with the sentinel first + E = 11
    out7 = oracle.moe_forward(exps, 7, None, H, I, x, sel + 7, w)
    assert np.array_equal(out7, out)


def test_activations_closed_forms(oracle):
    """act_gate (x16_dev.cu:68-112) against closed forms evaluated by scipy: SiLU = g * expit(g); the tanh GELU within its
    published distance of the exact GELU g * Phi(g) (< 1e-3 here; dropping the cubic term costs ~2e-2); ReLU^2; the
    gpt-oss SwiGLU (u + 1) * g * expit(1.702 g), whose glu is within 2.1e-2 of the exact GELU (1.0 instead of 1.702 is
    off by > 0.1); the non-gated relu(u) * u; the clamps of limit (g from above only, u on both sides)."""
    from scipy.special import expit, ndtr
    rng = np.random.default_rng(17)
    g = np.concatenate([rng.uniform(-6, 6, 400), [0.0, -0.0, 1e-3, -1e-3, 5.5]]).astype(np.float32)
    u = rng.uniform(-3, 3, g.size).astype(np.float32)
    A = lambda a, gd, lim=0.0: np.array([oracle.act(a, gd, gi, ui, lim) for gi, ui in zip(g, u)], np.float64)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    assert np.allclose(A(oracle.ACT_SILU, 1), g64 * expit(g64) * u64, rtol=1e-6, atol=1e-7)
    gelu_exact = g64 * ndtr(g64)
    assert np.abs(A(oracle.ACT_GELU, 1) / np.where(u64 == 0, 1, u64) - gelu_exact).max() < 1e-3
    assert np.allclose(A(oracle.ACT_RELU2, 1), np.maximum(g64, 0) ** 2 * u64, rtol=1e-6, atol=1e-7)
    oai = A(oracle.ACT_SILU_OAI, 1)
    assert np.allclose(oai, (u64 + 1) * g64 * expit(1.702 * g64), rtol=1e-6, atol=1e-7)
    assert np.abs(oai / (u64 + 1) - gelu_exact).max() < 2.1e-2
    assert oracle.act(oracle.ACT_SILU_OAI, 1, 2.0, -1.0) == 0.0
    assert np.allclose(A(oracle.ACT_SILU, 0), np.maximum(u64, 0) * u64, rtol=1e-6, atol=1e-7)
    lim = 1.5
    gc, uc = np.minimum(g64, lim), np.clip(u64, -lim, lim)
    assert np.allclose(A(oracle.ACT_SILU_OAI, 1, lim), (uc + 1) * gc * expit(1.702 * gc), rtol=1e-6, atol=1e-7)
    assert np.allclose(A(oracle.ACT_SILU, 1, lim), np.minimum(g64 * expit(g64), lim) * uc, rtol=1e-6, atol=1e-7)
    assert np.allclose(A(oracle.ACT_RELU2, 1, lim), np.minimum(np.maximum(g64, 0) ** 2, lim) * uc, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("act,gated,limit", [(1, 1, 0.0), (2, 1, 0.0), (3, 1, 0.0), (3, 1, 7.0), (0, 1, 2.0), (0, 0, 0.0)])
def test_expert_activation_vs_fp64_model(oracle, act, gated, limit):
    """The whole expert with each activation against the fp64 model of the mathematics (activation from scipy)."""
    from scipy.special import expit
    rng = np.random.default_rng(31 + act)
    H, I = 256, 128
    ex = make_expert(oracle, rng, H, I)
    x = rng.standard_normal(H).astype(np.float16)
    y, g, u, a = oracle.expert_forward(ex, H, I, x, act=act, gated=bool(gated), limit=limit)
    Hm = _hm()
    blk = lambda v: (v.reshape(-1, 128) @ Hm).reshape(-1)

    def lin(m, v):
        k, n = ((H, I), (H, I), (I, H))[m]
        W = oracle.np_dequant(ex["tr"][m], ex["fmt"][m], k, n).astype(np.float64)
        return blk(blk(v * ex["suh"][m].astype(np.float64)) @ W) * ex["svh"][m].astype(np.float64)
    g64, u64 = lin(0, x.astype(np.float64)), lin(1, x.astype(np.float64))
    if act == 3:
        if limit:
            g64, u64 = np.minimum(g64, limit), np.clip(u64, -limit, limit)
        av = (u64 + 1) * g64 * expit(1.702 * g64)
    else:
        if not gated:
            xv = np.maximum(u64, 0)
        elif act == 0:
            xv = g64 * expit(g64)
        elif act == 1:
            xv = 0.5 * g64 * (1 + np.tanh(0.797884560803 * (g64 + 0.044715 * g64 ** 3)))
        else:
            xv = np.maximum(g64, 0) ** 2
        if limit:
            u64, xv = np.clip(u64, -limit, limit), np.minimum(xv, limit)
        av = xv * u64
    want = lin(2, av)
    assert rel(y, want) < 3e-3 and np.abs(y - want).max() < 2e-2

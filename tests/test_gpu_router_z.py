"""GPU parity of the router from hidden states and of the shared expert's gate, through the C ABI, and the drop-in call
sequence of the reference's hooks (engine/tiers.py:707-739):

  sel, w = m.routing_fn(bsz, cfg, z, params)          routing from z: the router projection (bmx_router_logits) + top-k
  sel, w, cpu = nv.layer(li, sel, w, z, bsz)          residency step (none here)
  out = m.bc.run_bszN(z, sel, rw)                     expert products + combine
  fhs = m.cpu_split_combine(Nv2.combine(fhs), partial, pending, shape)

Projection: the GPU's fp16 logits equal RN16 of the exact float64 product except within fp32 accumulation error of a
rounding boundary (one fp16 ulp at most). Selection and weights: bit-exact against the oracle's router applied to the
GPU's logits (softmax, sigmoid + bias, sqrt-softplus + bias, group-limited). Layer outputs with a gated shared expert:
within 1e-2 max-abs / 1e-3 relative RMS of the oracle's layer."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

MAX_ABS, REL_RMS = 1e-2, 1e-3


def say(*a):
    print(*a, flush=True)


def rel_rms(a, b):
    return float(np.sqrt(np.mean((a.astype(np.float64) - b) ** 2)) / np.sqrt(np.mean(b.astype(np.float64) ** 2)))


def check_logits(got, z, W, oracle):
    """got = RN16(an fp32 accumulation of z W^T): within half an fp16 ulp of the exact value plus the accumulation's
    error, bounded by 64 fp32 ulps of sum |z_h W_eh| (recursive fp32 summation of 4096 terms stays far inside it)."""
    exact = oracle.router_logits(z, W)
    g = got.astype(np.float64)
    acc_err = 64 * 2.0 ** -24 * (np.abs(z.astype(np.float64)) @ np.abs(W.astype(np.float64)).T)
    half_ulp = 0.5 * np.spacing(np.maximum(np.abs(g), np.abs(exact)).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(g - exact) <= half_ulp + acc_err)
    return float((got != exact.astype(np.float16)).mean())


@pytest.mark.parametrize("T,E,H", [(1, 288, 4096), (5, 64, 2048), (33, 384, 4096), (513, 1000, 1024), (7, 256, 5120),
                                   # H = 64 mod 128: the projection's half-block tail
                                   (3, 64, 576), (40, 288, 2112), (1, 96, 64)])
def test_router_logits_projection(cuda, oracle, T, E, H):
    import bmx
    rng = np.random.default_rng(T * 7 + E)
    z = rng.standard_normal((T, H)).astype(np.float16)
    W = (rng.standard_normal((E, H)) / np.sqrt(H)).astype(np.float16)
    say("router logits", T, E, H)
    got = bmx.ops.router_logits(torch.from_numpy(z).to(cuda), torch.from_numpy(W).to(cuda)).cpu().numpy()
    frac = check_logits(got, z, W, oracle)
    say("fraction off RN16(exact):", frac)
    assert frac < 0.01


def test_router_logits_prefill_rows(cuda, oracle):
    """The 8192-token DeepSeek-shaped chunk: every row projected (E 384, H 4096), a sample of rows checked."""
    import bmx
    rng = np.random.default_rng(11)
    T, E, H = 8192, 384, 4096
    z = torch.randn((T, H), device=cuda).half()
    W = (torch.randn((E, H), device=cuda) / 64.0).half()
    got = bmx.ops.router_logits(z, W)
    rows = np.sort(rng.choice(T, 96, replace=False))
    check_logits(got[rows].cpu().numpy(), z[rows].cpu().numpy(), W.cpu().numpy(), oracle)
    assert torch.isfinite(got.float()).all()


SCORES = [("softmax", 0, False, 1, 1), ("sigmoid+bias", 1, True, 1, 1), ("sqrtsp+bias", 2, True, 1, 1),
          ("sqrtsp groups", 2, True, 8, 4), ("sigmoid groups", 1, True, 8, 4)]


@pytest.mark.parametrize("name,score,use_bias,G,TG", SCORES)
@pytest.mark.parametrize("T", [1, 8, 513])
def test_routing_fn_from_z(cuda, oracle, name, score, use_bias, G, TG, T):
    """routing_fn(bsz, cfg, z, params) with no logits in params: projection on the GPU, then top-k; bit-exact against
    the oracle's router on the GPU's logits."""
    import bmx
    E, H, topk = 384, 2048, 6
    rng = np.random.default_rng(T + 100 * score + G)
    tab = bmx.ExpertTable.random(H, 256, E, (bmx.TF_K2,) * 3, seed=1, device=cuda)
    W = torch.from_numpy((rng.standard_normal((E, H)) * 2.0 / np.sqrt(H)).astype(np.float16)).to(cuda)
    bias = torch.from_numpy((rng.standard_normal(E) * 0.05).astype(np.float32)).to(cuda) if use_bias else None
    layer = bmx.MoELayer(tab, topk, first=3, score=score, bias=bias, n_group=G, topk_group=TG, renorm=True, scale=2.0,
                         router_weight=W)
    z = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16)).to(cuda)
    say("routing from z:", name, "T", T)
    sel, w = layer.routing_fn(T, None, z, {})
    lg = layer.router_logits(z)
    torch.cuda.synchronize()
    osel, ow = oracle.router(lg.cpu().numpy(), topk, bias.cpu().numpy() if bias is not None else None, G, TG, score,
                             True, 2.0, first=3)
    assert np.array_equal(sel.cpu().numpy(), osel)
    assert np.array_equal(w.cpu().numpy().view(np.uint16), ow.view(np.uint16))
    check_logits(lg.cpu().numpy(), z.cpu().numpy(), W.cpu().numpy(), oracle)


@pytest.mark.parametrize("T", [1, 3, 64])
def test_sqrtsp_router_bitexact(cuda, oracle, T):
    """bmx_router_topk with the sqrt-softplus score on fp16 logits against the oracle, including renorm off."""
    import bmx
    rng = np.random.default_rng(T)
    E, k = 256, 8
    lg = (rng.standard_normal((T, E)) * 3).astype(np.float16)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    for renorm in (True, False):
        sel, w = bmx.ops.router_topk(torch.from_numpy(lg).to(cuda), k, torch.from_numpy(bias).to(cuda), 1, 1,
                                     bmx.SCORE_SQRTSP, renorm, 1.5, 0)
        osel, ow = oracle.router(lg, k, bias, 1, 1, oracle.SCORE_SQRTSP, renorm, 1.5)
        assert np.array_equal(sel.cpu().numpy(), osel)
        assert np.array_equal(w.cpu().numpy().view(np.uint16), ow.view(np.uint16))


@pytest.mark.parametrize("T,path", [(1, 1), (8, 1), (16, 3), (600, 2)])
def test_shared_gate_layer(cuda, oracle, T, path):
    """A layer whose shared expert is gated by sigmoid(x . g): outputs against the oracle (small launches combine in
    k_dn_combine_par, the 600-token prefill call in k_dn_combine); a gate vector of zeros halves the shared expert."""
    import bmx
    E, H, I, topk = 16, 4096 if T == 600 else 1024, 256, 4
    rng = np.random.default_rng(T)
    tab = bmx.ExpertTable.random(H, I, E, (bmx.TF_K3,) * 3, shared=True, seed=T, device=cuda)
    g = torch.from_numpy((rng.standard_normal(H) * 0.03).astype(np.float16)).to(cuda)
    layer = bmx.MoELayer(tab, topk, score=bmx.SCORE_SIGMOID, renorm=True, scale=1.0, shared_gate=g)
    plain = bmx.MoELayer(tab, topk, score=bmx.SCORE_SIGMOID, renorm=True, scale=1.0)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16)).to(cuda)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16)).to(cuda)
    sel, w = layer.routing_fn(T, None, x, {"logits": lg})
    say("shared gate layer T", T, "path", path)
    got = layer.run_bszN(x, sel, w, path).cpu().numpy()
    ungated = plain.run_bszN(x, sel, w, path).cpu().numpy()
    rows = np.arange(T) if T <= 16 else np.sort(rng.choice(T, 12, replace=False))
    exps = [tab.host_expert(e) for e in range(E)]
    want = oracle.moe_forward(exps, 0, tab.host_expert(E), H, I, x.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy(),
                              rows=rows, sh_gate=g.cpu().numpy())
    err, rr = float(np.abs(got[rows] - want).max()), rel_rms(got[rows], want)
    say("max_abs", err, "rel_rms", rr)
    assert err < MAX_ABS and rr < REL_RMS
    assert not np.array_equal(got, ungated)
    # the same GPU rows with the gate's value applied by hand: routed part = ungated minus the shared row
    gvals = [float(oracle.shared_gate(x[t].cpu().numpy(), g.cpu().numpy())) for t in rows]
    z = torch.zeros(H, dtype=torch.float16, device=cuda)
    half = bmx.MoELayer(tab, topk, score=bmx.SCORE_SIGMOID, renorm=True, scale=1.0, shared_gate=z)
    h = half.run_bszN(x, sel, w, path).cpu().numpy()
    routed = 2.0 * h[rows] - ungated[rows]                # h = routed + sh / 2, ungated = routed + sh
    sh = ungated[rows] - routed
    for i, t in enumerate(rows):
        assert np.allclose(got[t], routed[i] + gvals[i] * sh[i], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("T", [1, 8, 40])
def test_reference_hook_sequence(cuda, oracle, T):
    """The reference's per-layer hooks in order, on a GLM-shaped layer (sigmoid + bias, scale 2.5, one gated shared
    expert) with routing from z: routing_fn -> layer -> run_bszN -> combine -> cpu_split_combine (with and without a
    CPU partial); against the oracle, and bit-identical to the one-call MoELayer.forward(z)."""
    import bmx
    E, H, I, topk = 64, 2048, 512, 8
    rng = np.random.default_rng(40 + T)
    tab = bmx.ExpertTable.random(H, I, E, (bmx.TF_K3,) * 3, shared=True, seed=7, device=cuda)
    W = torch.from_numpy((rng.standard_normal((E, H)) * 2.0 / np.sqrt(H)).astype(np.float16)).to(cuda)
    bias = torch.from_numpy((rng.standard_normal(E) * 0.1).astype(np.float32)).to(cuda)
    g = torch.from_numpy((rng.standard_normal(H) * 0.03).astype(np.float16)).to(cuda)
    m = bmx.MoELayer(tab, topk, first=0, score=bmx.SCORE_SIGMOID, bias=bias, renorm=True, scale=2.5, router_weight=W,
                     shared_gate=g)
    z = torch.from_numpy(rng.standard_normal((1, T, H)).astype(np.float16)).to(cuda)      # [bsz, seq, H] view
    bsz = T
    sel, w = m.routing_fn(bsz, None, z, {})
    sel, w, cpu = m.layer(0, sel, w, z, bsz)
    assert cpu is False
    fhs = m.run_bszN(z, sel, w)
    out = m.cpu_split_combine(m.combine(fhs), None, False, z.shape)
    partial = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(cuda)
    out2 = m.cpu_split_combine(m.combine(fhs), partial, True, None)
    one = m.forward(z)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (1, T, H)
    assert torch.equal(out.view(T, H), fhs) and torch.equal(out2, fhs + partial)
    assert torch.equal(one, fhs)
    lg = m.router_logits(z).cpu().numpy()
    osel, ow = oracle.router(lg, topk, bias.cpu().numpy(), 1, 1, oracle.SCORE_SIGMOID, True, 2.5)
    assert np.array_equal(sel.cpu().numpy(), osel) and np.array_equal(w.cpu().numpy().view(np.uint16), ow.view(np.uint16))
    rows = np.arange(T) if T <= 8 else np.sort(rng.choice(T, 8, replace=False))
    want = oracle.moe_forward([tab.host_expert(e) for e in range(E)], 0, tab.host_expert(E), H, I,
                              z.view(T, H).cpu().numpy(), osel, ow, rows=rows, sh_gate=g.cpu().numpy())
    got = fhs.cpu().numpy()[rows]
    err, rr = float(np.abs(got - want).max()), rel_rms(got, want)
    say("hook sequence T", T, "max_abs", err, "rel_rms", rr)
    assert err < MAX_ABS and rr < REL_RMS

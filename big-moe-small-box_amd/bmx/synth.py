"""Synthetic workloads of the MoE layer (seeded; random-init weights of the named shapes, no checkpoints).

  c1  64 routed experts, top-8 softmax, H 2048, I 768, EXL3 4 bpw, 1 decode token
  c2  288 routed experts, top-8 sigmoid + bias ~N(0, 0.1) (renormalised, x2.5), 1 shared expert, H 4096, I 1536, 3 bpw;
      decode batches of 1 and 8 tokens
  c3  384 routed experts, group-limited top-6 (8 groups, top-4 groups; sigmoid, renormalised, x2.5), H 4096, I 2048,
      mixed 2 / 3 bpw (K 2 for even experts, K 3 for odd), 8192-token chunk, logits with Zipf(1.1) expert popularity
  c4  43 layers of c2 shape in decode (batch 1), Zipf-skewed routing with a per-layer permutation
  c5  c3 shape with 16 speculative-verify tokens, K 2 / 2.5 alternating (2.25 average), 1 % of activation channels x20,
      shared-context routing (base logits + small per-token noise)
Trellis bytes are uniform random (every bit string is a valid code); suh ~ U(0.5, 1.5); svh ~ U(0.5, 1.5) / sqrt(k)
so every linear keeps its input's norm and the layer output is O(1)."""
import math

import numpy as np
import torch

from . import _lib as L
from .experts import ExpertTable

CONFIGS = {
    "c1": dict(E=64, topk=8, H=2048, I=768, score=L.SCORE_SOFTMAX, renorm=True, scale=1.0, n_group=1, topk_group=1,
               shared=False, bias=False, T=1),
    "c2": dict(E=288, topk=8, H=4096, I=1536, score=L.SCORE_SIGMOID, renorm=True, scale=2.5, n_group=1, topk_group=1,
               shared=True, bias=True, T=1),
    "c3": dict(E=384, topk=6, H=4096, I=2048, score=L.SCORE_SIGMOID, renorm=True, scale=2.5, n_group=8, topk_group=4,
               shared=False, bias=False, T=8192),
    "c4": dict(E=288, topk=8, H=4096, I=1536, score=L.SCORE_SIGMOID, renorm=True, scale=2.5, n_group=1, topk_group=1,
               shared=True, bias=True, T=1, layers=43, cache_frac=0.30),
    "c5": dict(E=384, topk=6, H=4096, I=2048, score=L.SCORE_SIGMOID, renorm=True, scale=2.5, n_group=8, topk_group=4,
               shared=False, bias=False, T=16),
}


def formats(name, E, shared):
    n = E + (1 if shared else 0)
    if name == "c1":
        return [(L.TF_K4,) * 3] * n
    if name in ("c2", "c4"):
        return [(L.TF_K3,) * 3] * n
    if name == "c3":
        return [((L.TF_K2,) * 3 if e % 2 == 0 else (L.TF_K3,) * 3) for e in range(n)]
    if name == "c5":
        return [((L.TF_K2,) * 3 if e % 2 == 0 else (L.TF_K25,) * 3) for e in range(n)]
    raise KeyError(name)


def table(name, seed=0, device="cuda", E=None, H=None, I=None):
    c = CONFIGS[name]
    E = E or c["E"]
    return ExpertTable.random(H or c["H"], I or c["I"], E, formats(name, E, c["shared"]), shared=c["shared"], seed=seed,
                              device=device)


def zipf_logits(T, E, s=1.1, seed=0, perm_seed=None):
    """logits = log p_pi(e) + Gumbel noise: top-k of it samples k experts without replacement proportionally to the
    Zipf(s) popularity p_r ~ r^-s of a seeded permutation pi of the experts."""
    rng = np.random.default_rng(seed)
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    perm = np.random.default_rng(seed if perm_seed is None else perm_seed).permutation(E)
    logp = np.empty(E)
    logp[perm] = np.log(p)
    g = -np.log(-np.log(rng.uniform(1e-12, 1.0, (T, E))))
    return (logp[None, :] + g).astype(np.float16)


def inputs(name, T=None, seed=0, device="cuda"):
    """(x fp16 [T, H], logits fp16 [T, E], bias fp32 [E] or None) for a config."""
    c = CONFIGS[name]
    T = T or c["T"]
    H, E = c["H"], c["E"]
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    if name == "c5":
        ch = rng.choice(H, max(1, H // 100), replace=False)
        x[:, ch] *= 20.0
    if name in ("c3", "c4"):
        lg = zipf_logits(T, E, 1.1, seed)
    elif name == "c5":
        base = zipf_logits(1, E, 1.1, seed)[0].astype(np.float32)
        lg = (base[None, :] + 0.3 * rng.standard_normal((T, E))).astype(np.float16)
    else:
        lg = rng.standard_normal((T, E)).astype(np.float16)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if c["bias"] else None
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    return t(x.astype(np.float16)), t(lg), (t(bias) if bias is not None else None)


def quantized_bytes(tab, experts):
    """Algorithmic HBM bytes of a decode layer call: the trellis bytes of every distinct expert it touches."""
    return sum(tab.expert_bytes(int(e)) for e in set(int(e) for e in experts))


def flops(H, I, picks):
    return 6.0 * H * I * picks

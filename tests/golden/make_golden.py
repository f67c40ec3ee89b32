"""Writes the golden fixtures under tests/golden/ from the reference's own CPU code (oracle/_ref/libreflane.so, built by
`make -C oracle ref` from the reference tree) and the reference test's ring definition:

  codebook_w_gpu.npy   fp16 bits of ft_core.h w_gpu(state) for all 65536 states            (ft_core.h:76-84)
  perm.npy             ft_core.h PERM (init_perm)                                            (ft_core.h:49-62)
  ring_ends.npy        n135::tf_s(f, i) for TF_K2 / TF_K25 / TF_K3, i < 256                 (ft_n135.h:84-89)
  k3_tiles.npz         random K 3 trellis (64 x 96 matrix) and ft_core.h dense_weights of it (ft_core.h:1007-1022)
  ring_tiles.npz       random tiles per format and their states by the ring closed form of the reference's
                       tests/gpu_dsv41_vbmi_tables.py:67-81 (ring_states), restated below bit by bit
  prep.npz             x, suh and ft_core.h prep_block / ft_n135.h prep_block_v outputs     (ft_core.h:97-103)
  lane.npz             a 4-expert K 3 layer (H 256, I 256), 3 tokens, and moe_forward4 outputs in EXACT mode

Run from the repository root: python tests/golden/make_golden.py
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as O  # noqa: E402


def ring_states(tile, ka, mask):
    """16-bit window [S(i) - 16, S(i)) of the MSB-first 32-bit-word ring (the reference test's definition)."""
    words = np.frombuffer(bytes(tile), dtype="<u4")
    R = len(words) * 32
    bits = [(int(words[p >> 5]) >> (31 - (p & 31))) & 1 for p in range(R)]
    out = np.zeros(256, np.uint16)
    for i in range(256):
        s = (i >> 4) * (16 * ka + bin(mask).count("1"))
        for j in range((i & 15) + 1):
            s += ka + ((mask >> j) & 1)
        v = 0
        for p in range(s - 16, s):
            v = (v << 1) | bits[p % R]
        out[i] = v
    return out


def main():
    R = O.ref_lane()
    assert R is not None, "build oracle/_ref/libreflane.so first (make -C oracle ref)"
    rng = np.random.default_rng(20260)
    cb = np.array([R.ref_w_gpu(s) for s in range(65536)], np.float32).astype(np.float16).view(np.uint16)
    np.save(os.path.join(HERE, "codebook_w_gpu.npy"), cb)
    np.save(os.path.join(HERE, "perm.npy"), np.array([R.ref_perm(i) for i in range(256)], np.int32))
    np.save(os.path.join(HERE, "ring_ends.npy"), np.array([[R.ref_tf_s(f, i) for i in range(256)] for f in range(3)], np.int32))

    k, n = 64, 96
    tr = rng.integers(0, 256, (k // 16) * (n // 16) * 96, dtype=np.uint8)
    W = np.zeros((k, n), np.float32)
    R.ref_dense_weights_k3(tr.ctypes.data, k, n, W.ctypes.data)
    np.savez_compressed(os.path.join(HERE, "k3_tiles.npz"), trellis=tr, k=k, n=n, w=W.astype(np.float16))

    out = {}
    for name, (fmt, ka, mask) in {"k2": (O.TF_K2, 2, 0), "k25": (O.TF_K25, 2, 0xAAAA), "k3": (O.TF_K3, 3, 0),
                                  "k4": (O.TF_K4, 4, 0)}.items():
        tiles = rng.integers(0, 256, (4, O.TF_TB[fmt]), dtype=np.uint8)
        out[name + "_tiles"] = tiles
        out[name + "_states"] = np.stack([ring_states(t, ka, mask) for t in tiles])
    np.savez_compressed(os.path.join(HERE, "ring_tiles.npz"), **out)

    x = rng.standard_normal((4, 128)).astype(np.float16)
    suh = rng.uniform(0.5, 1.5, (4, 128)).astype(np.float16)
    xt = np.zeros((4, 128), np.float32)
    xv = np.zeros((4, 128), np.float32)
    for i in range(4):
        xf = x[i].astype(np.float32)
        s = np.ascontiguousarray(suh[i].view(np.uint16))
        R.ref_prep_block(xf.ctypes.data, s.ctypes.data, xt[i].ctypes.data)
        R.ref_prep_block_v(xf.ctypes.data, s.ctypes.data, xv[i].ctypes.data)
    np.savez_compressed(os.path.join(HERE, "prep.npz"), x=x, suh=suh, xt=xt.astype(np.float16), xt_v=xv.astype(np.float16))

    H, I, E, T, topk = 256, 256, 4, 3, 2
    trs, suhs, svhs = [], [], []
    for e in range(E):
        for (kk, nn) in ((H, I), (H, I), (I, H)):
            trs.append(rng.integers(0, 256, (kk // 16) * (nn // 16) * 96, dtype=np.uint8))
            suhs.append(rng.uniform(0.5, 1.5, kk).astype(np.float16))
            svhs.append((rng.uniform(0.5, 1.5, nn) / np.sqrt(kk)).astype(np.float16))
    xs = rng.standard_normal((T, H)).astype(np.float16)
    sel = np.array([[0, 1], [2, 3], [3, 1]], np.int32)
    w = np.array([[0.625, 0.375], [0.5, 0.5], [0.25, 0.75]], np.float16)
    cpus = (ctypes.c_int * 1)(0)
    assert R.ref_lane_create(H, I, E, 1, cpus, 0.0) == 0
    keep = []
    for e in range(E):
        t3 = trs[3 * e:3 * e + 3]
        sc = [suhs[3 * e], svhs[3 * e], suhs[3 * e + 1], svhs[3 * e + 1], suhs[3 * e + 2], svhs[3 * e + 2]]
        sc = [np.ascontiguousarray(a.view(np.uint16)) for a in sc]
        keep += sc
        R.ref_lane_set_expert(e, *[t.ctypes.data for t in t3], *[a.ctypes.data for a in sc], 2, 2, 2)
    lane_out = {}
    xf = xs.astype(np.float32)
    wf = w.astype(np.float32)
    for mode, name in ((1, "exact"), (0, "affine"), (2, "i16")):
        o = np.zeros((T, H), np.float32)
        R.ref_lane_forward(xf.ctypes.data, T, sel.ctypes.data, wf.ctypes.data, topk, o.ctypes.data, mode)
        lane_out[name] = o
    R.ref_lane_destroy()
    np.savez_compressed(os.path.join(HERE, "lane.npz"), H=H, I=I, E=E, x=xs, sel=sel, w=w,
                        trellis=np.stack(trs), suh=np.concatenate(suhs), svh=np.concatenate(svhs), **lane_out)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()

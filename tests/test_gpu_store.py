"""Layers served from a packed expert store: the ExpertTable read from the store (device arena, and pinned host homes
behind an expert-slot table) computes the same outputs, bit for bit, as a table built directly from the checkpoint's
tensors, and matches the oracle."""
import numpy as np
import pytest
import torch

from test_store import E, exl3_checkpoint, tensor_bytes

pytestmark = pytest.mark.gpu

H, I, TOPK = 256, 384, 3


def say(*a):
    print(*a, flush=True)


def direct_table(tensors, l, H, I, cuda):
    """ExpertTable of model layer l built from the checkpoint tensors (gate | up | down per expert row)."""
    import bmx
    mats = ("gate_proj", "up_proj", "down_proj")
    rows, suh, svh = [], [[], [], []], [[], [], []]
    for e in range(E):
        parts = [tensor_bytes(tensors[f"model.layers.{l}.mlp.experts.{e}.{m}.trellis"]) for m in mats]
        rows.append(np.frombuffer(b"".join(parts), np.uint8))
        for i, m in enumerate(mats):
            suh[i].append(tensors[f"model.layers.{l}.mlp.experts.{e}.{m}.suh"])
            svh[i].append(tensors[f"model.layers.{l}.mlp.experts.{e}.{m}.svh"])
    n0 = tensors[f"model.layers.{l}.mlp.experts.0.gate_proj.trellis"].nbytes
    n1 = tensors[f"model.layers.{l}.mlp.experts.0.up_proj.trellis"].nbytes
    arena = torch.from_numpy(np.stack(rows)).to(cuda)
    tb = n0 // ((H // 16) * (I // 16))
    fmt = {64: 0, 80: 1, 96: 2, 128: 3}[tb]
    return bmx.ExpertTable(H, I, arena, torch.tensor([(fmt,) * 3] * E, dtype=torch.int32),
                           [torch.from_numpy(np.stack(s)).to(cuda) for s in suh],
                           [torch.from_numpy(np.stack(s)).to(cuda) for s in svh], n0, n0 + n1, E, False)


@pytest.mark.parametrize("version", [1, 2])
def test_store_layers_match_checkpoint_tables(cuda, oracle, tmp_path, version):
    import bmx
    from bmx import store
    ck = tmp_path / "ckpt"
    tensors = exl3_checkpoint(ck, (0, 1), H, I, (96, 96), seed=version)
    out = tmp_path / "out"
    out.mkdir()
    store.pack(ck, out, "s", version=version)
    st = store.ExpertStore(out, "s")
    assert st.verify() == []
    kw = dict(score=bmx.SCORE_SIGMOID, renorm=True, scale=1.0)
    dev = [st.table(li, cuda) for li in range(2)]
    host = [st.table(li, cuda, home="host") for li in range(2)]
    slots = bmx.ExpertSlots(host, 3, maxj=2)
    ref = [bmx.MoELayer(direct_table(tensors, li, H, I, cuda), TOPK, **kw) for li in range(2)]
    from_store = [bmx.MoELayer(dev[li], TOPK, **kw) for li in range(2)]
    from_host = [bmx.MoELayer(host[li], TOPK, **kw) for li in range(2)]
    staged = [bmx.MoELayer(host[li], TOPK, slots=slots, li=li, **kw) for li in range(2)]
    rng = np.random.default_rng(3)
    for step in range(6):
        li, T = step % 2, (1, 5, 40)[step % 3]
        say("store layer step", step, "layer", li, "T", T)
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16)).to(cuda)
        lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16)).to(cuda)
        sel, w = ref[li].routing_fn(T, None, x, {"logits": lg})
        want = ref[li].run_bszN(x, sel, w)
        for lay in (from_store[li], from_host[li]):
            assert torch.equal(lay.run_bszN(x, sel, w), want)
        sel2, w2 = staged[li].routing_fn(T, None, x, {"logits": lg})
        staged[li].layer(li, sel2, w2, x, T)
        assert torch.equal(staged[li].run_bszN(x, sel2, w2), want)
        if step == 0:
            used = sorted(set(int(e) for e in sel.cpu().numpy().ravel()))
            exps = [dev[li].host_expert(e) if e in used else None for e in range(E)]
            o = oracle.moe_forward(exps, 0, None, H, I, x.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy())
            got = want.cpu().numpy()
            err = float(np.sqrt(np.mean((got - o) ** 2)) / np.sqrt(np.mean(o ** 2)))
            say("vs oracle rel_rms", err, "max_abs", float(np.abs(got - o).max()))
            assert err < 1e-3 and np.abs(got - o).max() < 1e-2


def test_unmarked_store_needs_consent(cuda, tmp_path):
    from bmx import store
    ck = tmp_path / "ckpt"
    exl3_checkpoint(ck, (0,), 256, 128, (64,), mul1=False)
    (tmp_path / "o").mkdir()
    store.pack(ck, tmp_path / "o", "u")
    st = store.ExpertStore(tmp_path / "o", "u")
    with pytest.raises(ValueError, match="mul1"):
        st.table(0, cuda)
    t = st.table(0, cuda, allow_unmarked=True)
    assert (t.H, t.I, t.E) == (256, 128, E) and int(t.fmt[0, 0]) == 0

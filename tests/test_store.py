"""Expert store (bmx.store): pack from a safetensors checkpoint, manifest layout, verify, read back. CPU only.

The v1 layout's known answers are the reference's own (tests/test_store.py:12-49 of the reference: two MoE layers of
4 experts, 4096-byte trellis tensors, 64 / 32-value scales -> trellis part 12288, record 16384, slot offsets 4096 /
8192, a corrupted byte found in record 5)."""
import itertools
import json

import numpy as np
import pytest

LAYERS, E = (3, 4), 4
GLM = ("gate_proj", "up_proj", "down_proj")


def save_checkpoint(directory, tensors, shards=1):
    """A sharded safetensors checkpoint written by the safetensors library: tensors {key: numpy array} dealt over the
    shards in sorted key order, and the model.safetensors.index.json weight map."""
    from safetensors.numpy import save_file
    directory.mkdir()
    keys = sorted(tensors)
    weight_map = {}
    for i in range(shards):
        fn = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        part = {k: np.ascontiguousarray(tensors[k]) for k in keys[i::shards]}
        save_file(part, str(directory / fn))
        weight_map.update(dict.fromkeys(part, fn))
    (directory / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))


def pattern_checkpoint(directory):
    """Two MoE layers (model layers 3 and 4) of 4 experts, the sizes of the reference's store test: int16 trellis
    tensors of 4096 bytes, fp16 suh of 64 and svh of 32 values, an int32 .mul1 marker (7) per matrix, and one
    attention tensor per layer that the store must skip. Every tensor holds its own ramp of values, so a record can be
    checked byte by byte."""
    t = {}
    tag = itertools.count(1)
    for layer in LAYERS:
        t[f"model.layers.{layer}.self_attn.q_proj.weight"] = np.full(64, layer, np.float16)
        for e in range(E):
            for m in GLM:
                k = f"model.layers.{layer}.mlp.experts.{e}.{m}"
                n = next(tag)
                t[k + ".trellis"] = (np.arange(2048, dtype=np.int32) * 7 + n * 1000).astype(np.int16)
                t[k + ".suh"] = (np.arange(64) / 64 + n).astype(np.float16)
                t[k + ".svh"] = (np.arange(32) / 32 - n).astype(np.float16)
                t[k + ".mul1"] = np.array(7, np.int32)
    save_checkpoint(directory, t, shards=2)
    return t


def exl3_checkpoint(d, layers, H, I, tile_bytes, seed=0, naming=GLM, mul1=True):
    """Random EXL3-shaped experts: trellis int16 [k/16, n/16, 8 * TB / 16], suh fp16 [k], svh fp16 [n]; tile_bytes
    per layer (64 / 80 / 96 / 128 for K 2 / 2.5 / 3 / 4). Returns {key: numpy array}."""
    rng = np.random.default_rng(seed)
    t = {}
    for l, tb in zip(layers, tile_bytes):
        for e in range(E):
            for m, (k, n) in zip(naming, ((H, I), (H, I), (I, H))):
                key = f"model.layers.{l}.mlp.experts.{e}.{m}"
                tr = rng.integers(0, 256, (k // 16) * (n // 16) * tb, dtype=np.uint8)
                t[key + ".trellis"] = tr.view(np.int16).reshape(k // 16, n // 16, tb // 2)
                t[key + ".suh"] = (rng.random(k) + 0.5).astype(np.float16)
                t[key + ".svh"] = ((rng.random(n) + 0.5) / np.sqrt(k)).astype(np.float16)
                if mul1:
                    t[key + ".mul1"] = np.array(0x83DCD12D, np.uint32).view(np.int32)
    save_checkpoint(d, t)
    return t


def tensor_bytes(a):
    return np.ascontiguousarray(a).tobytes()


def test_v1_layout_known_answers(tmp_path):
    from bmx import store
    ck = tmp_path / "ckpt"
    tensors = pattern_checkpoint(ck)
    out = tmp_path / "out"
    out.mkdir()
    store.pack(ck, out, "x", version=1, threads=2)
    raw = json.load(open(out / "x.json"))
    assert raw["format"] == "exl3-expert-store-v1"
    assert raw["n_layers"] == 2 and raw["experts_per_layer"] == E and raw["trellis_bytes"] == 3 * 4096
    assert raw["record_bytes"] == 4096 * 4 and raw["vram_slot"] == {"off_u": 4096, "off_d": 8192, "slot_bytes": 12288}
    assert [L["model_layer"] for L in raw["layers"]] == list(LAYERS)
    assert raw["mul1_markers_hex"] == [np.array(7, "<i4").tobytes().hex()]
    assert store.verify(out, "x", threads=2) == []
    # every record is its tensors in field order, then zeros
    blob = open(out / "x.bin", "rb").read()
    for li, l in enumerate(LAYERS):
        for e in range(E):
            rec = blob[(li * E + e) * 16384:(li * E + e + 1) * 16384]
            want = b"".join(tensor_bytes(tensors[f"model.layers.{l}.mlp.experts.{e}.{m}.trellis"]) for m in GLM)
            want += b"".join(tensor_bytes(tensors[f"model.layers.{l}.mlp.experts.{e}.{m}.{s}"]) for m in GLM for s in ("suh", "svh"))
            assert rec == want + bytes(16384 - len(want))
    with open(out / "x.bin", "r+b") as f:              # corrupt one byte of record 5 (layer 1, expert 1)
        f.seek(5 * 16384 + 100)
        f.write(b"\xff")
    assert store.verify(out, "x", threads=2) == [(1, 1)]
    assert store.verify(out, "x", sample=0) == []       # only the first / last expert of each layer


def test_v2_per_layer_records_and_classes(tmp_path):
    from bmx import store
    ck = tmp_path / "ckpt"
    tensors = exl3_checkpoint(ck, (0, 1, 2), 256, 128, (96, 64, 96))
    out = tmp_path / "out"
    out.mkdir()
    store.pack(ck, out, "y", version=2, threads=3)
    m = store.manifest(out, "y")
    assert m["format"] == "exl3-expert-store-v2" and m["mats"] == ["gate_proj", "up_proj", "down_proj"]
    k3, k2 = 2 * 256 // 16 * 128 // 16 * 96, 2 * 256 // 16 * 128 // 16 * 64   # gate + up trellis bytes
    recs = [L["rec_bytes"] for L in m["layers"]]
    assert [L["trellis_bytes"] for L in m["layers"]] == [k3 * 3 // 2, k2 * 3 // 2, k3 * 3 // 2]
    assert all(r % 4096 == 0 for r in recs) and m["layers"][1]["base"] == E * recs[0]
    assert m["layers"][2]["base"] == E * (recs[0] + recs[1])
    raw = json.load(open(out / "y.json"))
    assert [c["layers"] for c in raw["classes"]] == [[0, 2], [1]]
    st = store.ExpertStore(out, "y")
    assert st.size_classes() == [[0, 2], [1]]
    for li in range(3):
        H, I, fmts, off_u, off_d, tb = st.geometry(li)
        assert (H, I) == (256, 128) and fmts == ((2, 2, 2) if li != 1 else (0, 0, 0))
        for e in range(E):
            for m_ in ("gate_proj", "up_proj", "down_proj"):
                tr = tensor_bytes(tensors[f"model.layers.{li}.mlp.experts.{e}.{m_}.trellis"])
                assert bytes(st.field(li, f"{m_}.trellis")[e]) == tr
                suh = tensors[f"model.layers.{li}.mlp.experts.{e}.{m_}.suh"]
                assert np.array_equal(st.field(li, f"{m_}.suh")[e], suh)
            img = bytes(st.records(li)[e, :tb])
            assert img[off_u:off_u + 10] == tensor_bytes(tensors[f"model.layers.{li}.mlp.experts.{e}.up_proj.trellis"])[:10]
    assert st.verify() == []


def test_v1_refuses_mixed_layers_and_reads_deepseek_names(tmp_path):
    from bmx import store
    ck = tmp_path / "ckpt"
    exl3_checkpoint(ck, (0, 1), 256, 128, (96, 64))
    (tmp_path / "o").mkdir()
    with pytest.raises(ValueError, match="version 1"):
        store.pack(ck, tmp_path / "o", "z", version=1)
    ck2 = tmp_path / "ckpt2"
    exl3_checkpoint(ck2, (5,), 128, 256, (128,), naming=("w1", "w3", "w2"))
    store.pack(ck2, tmp_path / "o", "w", version=1, naming="deepseek")
    st = store.ExpertStore(tmp_path / "o", "w")
    assert st.man["mats"] == ["w1", "w3", "w2"] and st.geometry(0)[:3] == (128, 256, (3, 3, 3))


def test_geometry_rejects_non_exl3_shapes(tmp_path):
    from bmx import store
    ck = tmp_path / "ckpt"
    pattern_checkpoint(ck)
    (tmp_path / "o").mkdir()
    store.pack(ck, tmp_path / "o", "x", version=1)
    with pytest.raises(ValueError, match="trellis"):
        store.ExpertStore(tmp_path / "o", "x").geometry(0)

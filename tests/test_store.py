"""The on-disk int4 format (lowbit.store) and model.save_int4, on the CPU: bytes and scales round-trip unchanged,
the metadata round-trips, malformed files and entries are refused with clear errors, and a model's projections are
saved under their qualified module names."""
import json

import numpy as np
import pytest
import torch

from lowbit import decode, model as lbmodel, quant, store
from oracle import quant_ref as R


def _entries(seed=0):
    rng = np.random.default_rng(seed)
    out = {}
    for name, (n, k) in {"a.q_proj": (48, 256), "b.down_proj": (17, 384), "c": (1, 128)}.items():
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        out[name] = R.quantize_w4(w, 128)
    return out


def test_round_trip_is_bit_exact(tmp_path):
    ents = _entries()
    path = tmp_path / "w.safetensors"
    store.save_w4(path, ents, 128, clip_grid=(1.0, 0.975, 0.95))
    meta = store.read_meta(path)
    assert meta["group"] == 128 and meta["clip_grid"] == (1.0, 0.975, 0.95)
    assert meta["names"] == sorted(ents)
    got, group = store.load_w4(path)
    assert group == 128 and sorted(got) == sorted(ents)
    for name, (p, s) in ents.items():
        gp, gs = got[name]
        assert gp.dtype == torch.uint8 and gs.dtype == torch.float16
        assert np.array_equal(gp.numpy(), p) and np.array_equal(gs.numpy().view(np.uint16), s.view(np.uint16)), name
        # the loaded bytes dequantize to the oracle's fp16 weights
        assert np.array_equal(R.dequantize_w4_f16(gp.numpy(), gs.numpy(), 128), R.dequantize_w4_f16(p, s, 128))
    sub, _ = store.load_w4(path, names=["c"])
    assert list(sub) == ["c"]
    with pytest.raises(KeyError, match="no entry"):
        store.load_w4(path, names=["missing"])


def test_group_64_and_tensor_inputs(tmp_path):
    w = (np.random.default_rng(1).standard_normal((32, 192)) * 0.1).astype(np.float32)
    p, s = R.quantize_w4(w, 64)
    path = tmp_path / "g64.safetensors"
    store.save_w4(path, {"x": (torch.from_numpy(p), torch.from_numpy(s))}, 64)
    got, group = store.load_w4(path)
    assert group == 64 and np.array_equal(got["x"][0].numpy(), p) and store.read_meta(path)["clip_grid"] is None


def test_save_refuses_malformed_entries(tmp_path):
    p, s = _entries()["a.q_proj"]
    path = tmp_path / "bad.safetensors"
    with pytest.raises(ValueError, match="multiple of 32"):
        store.save_w4(path, {"x": (p, s)}, 48)
    with pytest.raises(ValueError, match="scales are"):
        store.save_w4(path, {"x": (p, s[:, :1])}, 128)
    with pytest.raises(ValueError, match="multiple of the group size"):
        store.save_w4(path, {"x": (p[:, :96], s)}, 128)
    with pytest.raises(ValueError, match="expected torch.float16"):
        store.save_w4(path, {"x": (p, s.astype(np.float32))}, 128)
    with pytest.raises(ValueError, match="expected torch.uint8"):
        store.save_w4(path, {"x": (p.astype(np.int8), s)}, 128)
    with pytest.raises(ValueError, match="reserved suffix"):
        store.save_w4(path, {"x.scales": (p, s)}, 128)
    assert not path.exists()                    # nothing is written when an entry is refused


def test_load_refuses_foreign_or_broken_files(tmp_path):
    from safetensors.torch import save_file
    p, s = (torch.from_numpy(a) for a in _entries()["a.q_proj"])
    good = {"format": "lowbit-w4", "version": "1", "group": "128", "layout": "canonical"}
    cases = [
        ({"x.packed": p, "x.scales": s}, {}, "not a lowbit int4 file"),
        ({"x.packed": p, "x.scales": s}, {**good, "version": "9"}, "unsupported format version"),
        ({"x.packed": p, "x.scales": s}, {**good, "layout": "mma"}, "unsupported layout"),
        ({"x.packed": p}, good, "lacks its packed bytes or its scales"),
        ({"x.packed": p, "x.scales": s, "extra": s.clone()}, good, "unexpected tensor"),
    ]
    for i, (tensors, meta, msg) in enumerate(cases):
        path = tmp_path / f"f{i}.safetensors"
        save_file(tensors, str(path), metadata=meta or None)
        with pytest.raises(ValueError, match=msg):
            store.load_w4(path)
    path = tmp_path / "shape.safetensors"
    save_file({"x.packed": p, "x.scales": s[:, :1].contiguous()}, str(path), metadata=good)
    with pytest.raises(ValueError, match="has scales"):
        store.load_w4(path)
    path = tmp_path / "dtype.safetensors"
    save_file({"x.packed": p, "x.scales": s.float()}, str(path), metadata=good)
    with pytest.raises(ValueError, match="wrong dtype"):
        store.load_w4(path)


def test_save_int4_names_every_projection(tmp_path):
    m = decode.random_model("tiny", seed=4, device="cpu").float()
    layers = []
    for parent, name, lin in lbmodel._projections(m):
        packed, scales = quant.quantize_w4(lin.weight.detach().numpy(), 128)
        layers.append((parent, name, lin, torch.from_numpy(packed), torch.from_numpy(scales)))
    path = tmp_path / "tiny.safetensors"
    lbmodel.save_int4(m, layers, path, 128, clip_grid=None)
    meta = store.read_meta(path)
    want = sorted(f"model.layers.{i}.{sub}.{t}" for i in range(2) for t in lbmodel.TARGETS
                  for sub in (["self_attn"] if t in ("q_proj", "k_proj", "v_proj", "o_proj") else ["mlp"]))
    assert meta["names"] == want
    got, _ = store.load_w4(path)
    names = {id(mod): n for n, mod in m.named_modules()}
    for _, _, lin, packed, scales in layers:
        gp, gs = got[names[id(lin)]]
        assert torch.equal(gp, packed) and torch.equal(gs, scales)
    other = decode.random_model("tiny", seed=5, device="cpu")
    with pytest.raises(ValueError, match="not a module of this model"):
        lbmodel.save_int4(other, layers, tmp_path / "x.safetensors")
    # the header is plain JSON with the format's metadata
    raw = path.read_bytes()
    header = json.loads(raw[8:8 + int.from_bytes(raw[:8], "little")])
    assert header["__metadata__"]["format"] == "lowbit-w4"

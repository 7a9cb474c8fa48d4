"""W4Linear inside a Hugging Face Qwen2 decoder on the GPU (a two-layer model with Qwen2.5 head geometry): the GPU
quantizer gives the oracle's bits for every projection, INT4 logits match fake-quant logits (same quantized weights,
PyTorch arithmetic) on identical inputs, graph replay equals eager execution, and feeding 16 or 48 tokens per step
(MFMA kernel) agrees with feeding one (GEMV)."""
import numpy as np
import pytest
import torch

from lowbit import decode, model as lbmodel
from oracle import quant_ref as R

pytestmark = pytest.mark.gpu

CLIP = tuple(round(1.0 - 0.025 * i, 3) for i in range(11))


def rel_max(a, b):
    return float((a.float() - b.float()).abs().max() / b.float().pow(2).mean().sqrt())


@pytest.fixture(scope="module")
def models():
    torch.cuda.set_device(0)
    m = decode.random_model("tiny", seed=11)
    weights = [lin.weight.detach().float().cpu().numpy() for _, _, lin in lbmodel._projections(m)]
    layers = lbmodel.quantize_layers(m, 128)
    for (_, name, _, packed, scales), w in zip(layers, weights):
        p_ref, s_ref = R.quantize_w4(w, 128)
        assert np.array_equal(packed.cpu().numpy(), p_ref) and np.array_equal(scales.cpu().numpy(), s_ref), name
    lbmodel.apply_fake_quant(layers)
    fake = decode.random_model("tiny", seed=11)
    fake.load_state_dict(m.state_dict())
    replaced, nbytes = lbmodel.apply_int4(layers)
    assert replaced == 14 and nbytes > 0
    assert all(isinstance(layer.self_attn.q_proj, lbmodel.W4Linear) and isinstance(layer.mlp.down_proj, lbmodel.W4Linear)
               for layer in m.model.layers)
    return m, fake


def feed_logits(model, prompt, feed, chunk, graph=True):
    dec = decode.GraphDecoder(model, prompt.shape[1] + feed.numel() + 16, chunk)
    dec.prefill(prompt)
    if graph:
        dec.capture()
        rows = [dec.step(feed[i:i + chunk]).clone() for i in range(0, feed.numel(), chunk)]
    else:                                        # the same forward, eagerly
        rows = []
        for i in range(0, feed.numel(), chunk):
            dec.tokens.copy_(feed[i:i + chunk].view(1, chunk))
            dec.positions.copy_(dec.offsets + dec.pos)
            with torch.inference_mode():
                rows.append(dec._forward().clone())
            dec.pos += chunk
    return torch.cat(rows)


def test_int4_matches_fake_quant_and_graph_matches_eager(cuda, models):
    m, fake = models
    gen = torch.Generator(device="cuda").manual_seed(7)
    prompt = torch.randint(0, 1024, (1, 40), generator=gen, device="cuda")
    feed = torch.randint(0, 1024, (48,), generator=gen, device="cuda")
    ref = feed_logits(fake, prompt, feed, 1, graph=False)
    g1 = feed_logits(m, prompt, feed, 1)
    assert torch.equal(g1, feed_logits(m, prompt, feed, 1, graph=False))          # replay == eager, bit for bit
    assert rel_max(g1, ref) < 2e-2
    assert float((g1.argmax(-1) == ref.argmax(-1)).float().mean()) >= 0.9
    for chunk in (16, 48):                                                         # MFMA path vs GEMV path
        gc = feed_logits(m, prompt, feed, chunk)
        assert rel_max(gc, g1) < 2e-2, chunk
        assert rel_max(gc, ref) < 2e-2, chunk


def test_greedy_graph_decode_runs_on_device(cuda, models):
    m, _ = models
    prompt = torch.randint(0, 1024, (1, 24), generator=torch.Generator(device="cuda").manual_seed(3), device="cuda")
    dec = decode.GraphDecoder(m, 24 + 40, 1)
    first = dec.prefill(prompt).argmax(-1)
    dec.capture()
    toks = dec.greedy(first, 32)
    dec2 = decode.GraphDecoder(m, 24 + 40, 1)                                      # eager greedy, step by step
    nxt = dec2.prefill(prompt).argmax(-1)
    eager = [int(nxt)]
    for _ in range(31):
        dec2.tokens.fill_(eager[-1])
        dec2.positions.copy_(dec2.offsets + dec2.pos)
        with torch.inference_mode():
            eager.append(int(dec2._forward()[-1].argmax(-1)))
        dec2.pos += 1
    assert toks.tolist() == eager


def test_saved_int4_loads_to_the_same_model(cuda, tmp_path):
    """quantize once, save_int4, load_int4 into a fresh copy of the model: the same W4Linear weights and bit-identical
    logits, with no quantizer call; a file whose shapes do not fit the model is refused."""
    from lowbit import store
    a = decode.random_model("tiny", seed=12)
    b = decode.random_model("tiny", seed=12)
    layers = lbmodel.quantize_layers(a, 128, CLIP)
    path = tmp_path / "tiny_int4.safetensors"
    lbmodel.save_int4(a, layers, path, 128, CLIP)
    assert store.read_meta(path)["clip_grid"] == CLIP
    ra, na = lbmodel.apply_int4(layers)
    rb, nb = lbmodel.load_int4(b, path)
    assert (ra, na) == (rb, nb) == (14, na)
    for la, lb in zip(a.model.layers, b.model.layers):
        for qa, qb in ((la.self_attn.q_proj, lb.self_attn.q_proj), (la.mlp.down_proj, lb.mlp.down_proj)):
            assert torch.equal(qa.wq.packed_mma, qb.wq.packed_mma) and torch.equal(qa.wq.scales, qb.wq.scales)
    ids = torch.randint(0, 1024, (1, 37), generator=torch.Generator(device="cuda").manual_seed(3), device="cuda")
    with torch.inference_mode():
        assert torch.equal(a(ids).logits, b(ids).logits)
    # a file from a model of another shape: same names, other widths
    ents, g = store.load_w4(path)
    name = "model.layers.0.mlp.up_proj"
    p, s = ents[name]
    ents[name] = (p[:256].contiguous(), s[:256].contiguous())
    bad = tmp_path / "bad.safetensors"
    store.save_w4(bad, ents, g)
    c = decode.random_model("tiny", seed=12)
    with pytest.raises(ValueError, match="saved weight is 256 x 256"):
        lbmodel.load_int4(c, bad)
    assert not any(isinstance(mod, lbmodel.W4Linear) for mod in c.modules())      # nothing was swapped
    del ents[name]
    store.save_w4(bad, ents, g)
    with pytest.raises(KeyError, match="no entry"):
        lbmodel.load_int4(decode.random_model("tiny", seed=12), bad)

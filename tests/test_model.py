"""The model-level surface on the CPU: the random-init Qwen2.5 geometry of the benchmark, the projections
quantize_layers finds, and fake-quant weights equal (bit for bit) to the oracle's dequantized values."""
import numpy as np
import torch

from lowbit import decode, model as lbmodel
from oracle import quant_ref as R


def test_qwen25_geometry():
    for name, (hidden, inter, layers, heads, kv) in decode.QWEN25.items():
        cfg = decode.qwen25_config(name)
        assert (cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers) == (hidden, inter, layers)
        assert (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim) == (heads, kv, 128)
        assert cfg.rope_parameters["rope_theta"] == 1e6 and cfg.rms_norm_eps == 1e-6
    assert decode.qwen25_config("3b").vocab_size == 151936 and decode.qwen25_config("3b").tie_word_embeddings


def test_projections_and_fake_quant_on_cpu():
    """quantize_layers visits the seven TARGETS of every layer in order; apply_fake_quant writes exactly the oracle's
    dequantized fp16 values (packed here by the host quantizer, lowbit.quant)."""
    from lowbit import quant
    m = decode.random_model("tiny", seed=3, device="cpu").float()
    found = list(lbmodel._projections(m))
    assert [name for _, name, _ in found] == list(lbmodel.TARGETS) * 2
    layers = []
    for parent, name, lin in found:
        packed, scales = quant.quantize_w4(lin.weight.detach().numpy(), 128)
        layers.append((parent, name, lin, torch.from_numpy(packed), torch.from_numpy(scales)))
    before = [lin.weight.detach().clone() for _, _, lin, _, _ in layers]
    lbmodel.apply_fake_quant(layers)
    for (_, name, lin, packed, scales), w0 in zip(layers, before):
        p_ref, s_ref = R.quantize_w4(w0.numpy(), 128)
        assert np.array_equal(packed.numpy(), p_ref) and np.array_equal(scales.numpy(), s_ref), name
        assert np.array_equal(lin.weight.detach().half().numpy(), R.dequantize_w4_f16(p_ref, s_ref, 128)), name


def test_random_model_is_seeded_and_scaled():
    a = decode.random_model("tiny", seed=5, device="cpu")
    b = decode.random_model("tiny", seed=5, device="cpu")
    wa = a.model.layers[0].mlp.down_proj.weight.float()
    assert torch.equal(wa, b.model.layers[0].mlp.down_proj.weight.float())
    assert abs(float(wa.std()) - 0.02) < 2e-3 and float(a.model.layers[0].self_attn.q_proj.bias.abs().max()) == 0.0


def test_rope_permutation_pairs_rotation_partners_in_one_tile():
    """Row 16 (d / 8) + d % 8 of each head holds dim d < 64 and the row 8 below it holds d + 64 (the kernels'
    rope_row), and the permutation is a bijection of every head's 128 rows."""
    from lowbit import fused
    heads = 5
    perm = fused.rope_permutation(heads).tolist()
    assert sorted(perm) == list(range(heads * 128))
    for h in range(heads):
        for d in range(64):
            row = 16 * (d // 8) + d % 8
            assert perm[h * 128 + row] == h * 128 + d and perm[h * 128 + row + 8] == h * 128 + d + 64

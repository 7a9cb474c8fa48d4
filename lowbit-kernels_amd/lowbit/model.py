"""INT4 weight-only projections for Hugging Face decoders: the reference's lowbit/model.py surface (W4Linear, TARGETS,
quantize_layers, apply_fake_quant, apply_int4; lowbit/model.py:12-57) on the gfx950 library.

A model is quantized once (quantize_layers). The same packed values can then back a "fake-quant" model (its own
nn.Linear layers holding the dequantized fp16 weights, so PyTorch does the arithmetic) or the INT4 kernels (W4Linear).
Equal results from the two isolate kernel error from quantization error.
"""
import torch
from torch import nn

from . import ops

# the seven projections of a Qwen2 / Llama decoder layer; embeddings and the (tied) head stay fp16
TARGETS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


class W4Linear(nn.Module):
    """nn.Linear replacement holding an ops.W4Weight. forward flattens the leading dimensions, runs ops.linear in fp16
    (GEMV / MFMA / dequantize + BLAS by row count, or a fixed `gemv_version`) and adds the bias in place."""

    def __init__(self, wq, bias, in_features, out_features, gemv_version=0):
        super().__init__()
        self.wq = wq
        self.in_features, self.out_features, self.gemv_version = in_features, out_features, gemv_version
        if bias is None:
            self.bias = None
        else:
            self.bias = nn.Parameter(bias.detach().to(torch.float16), requires_grad=False)

    def forward(self, x):
        lead = x.shape[:-1]
        y = ops.linear(x.reshape(-1, self.in_features).to(torch.float16), self.wq, version=self.gemv_version)
        if self.bias is not None:
            y.add_(self.bias)
        return y.view(*lead, self.out_features)

    def extra_repr(self):
        return f"in_features={self.in_features}, out_features={self.out_features}, group={self.wq.group}"


def _projections(model):
    """(parent module, attribute name, nn.Linear) for every TARGETS projection, in module order."""
    for parent in model.modules():
        for name in TARGETS:
            child = getattr(parent, name, None)
            if isinstance(child, nn.Linear):
                yield parent, name, child


def quantize_layers(model, group=128, clip_grid=None):
    """Quantize every projection with the GPU quantizer (absmax, or the clip search over `clip_grid`).
    Returns a list of (parent, name, linear, packed, scales)."""
    return [(parent, name, lin, *ops.quantize_w4_gpu(lin.weight, group, clip_grid))
            for parent, name, lin in list(_projections(model))]


@torch.no_grad()
def apply_fake_quant(layers, group=128):
    """Overwrite each projection's weight with its dequantized fp16 value: exactly what the kernels multiply by."""
    for _, _, lin, packed, scales in layers:
        lin.weight.copy_(ops.dequantize_w4_gpu(packed, scales, group))


def apply_int4(layers, group=128, gemv_version=0, layouts=("mma",)):
    """Swap every quantized projection for a W4Linear on the same packed values (device layouts built on the GPU).
    Returns (layers replaced, INT4 bytes). Consumes `layers`, so the fp16 weights can be freed."""
    replaced, nbytes = 0, 0
    while layers:
        parent, name, lin, packed, scales = layers.pop(0)
        wq = ops.W4Weight(packed, scales, group, layouts, device=packed.device)
        setattr(parent, name, W4Linear(wq, lin.bias, lin.in_features, lin.out_features, gemv_version))
        replaced, nbytes = replaced + 1, nbytes + wq.nbytes()
    torch.cuda.empty_cache()
    return replaced, nbytes

"""INT4 weight-only projections for Hugging Face decoders: the reference's lowbit/model.py surface (W4Linear, TARGETS,
quantize_layers, apply_fake_quant, apply_int4; lowbit/model.py:12-57) on the gfx950 library, plus save_int4 /
load_int4, which keep the quantized projections on disk (lowbit.store) so a model is quantized once.

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
    """nn.Linear replacement holding an ops.W4Weight. forward flattens the leading dimensions and runs ops.linear in
    fp16 (GEMV / MFMA / dequantize + BLAS by row count, or a fixed `gemv_version`) with the bias, which the INT4
    kernels add in their store (reference lowbit/model.py:25-26 adds it as a separate op; same rounding)."""

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
        y = ops.linear(x.reshape(-1, self.in_features).to(torch.float16), self.wq, version=self.gemv_version,
                       bias=self.bias)
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


def _names(model):
    """id(module) -> its qualified name in `model` (e.g. "model.layers.0.self_attn.q_proj")."""
    return {id(mod): name for name, mod in model.named_modules()}


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


def save_int4(model, layers, path, group=128, clip_grid=None):
    """Write the quantized projections of quantize_layers(model, group, clip_grid) to `path` (lowbit.store format,
    keyed by each projection's qualified module name), so later runs can load_int4 instead of quantizing again."""
    from . import store
    names = _names(model)
    entries = {}
    for _, _, lin, packed, scales in layers:
        if id(lin) not in names:
            raise ValueError("a quantized layer is not a module of this model")
        entries[names[id(lin)]] = (packed, scales)
    store.save_w4(path, entries, group, clip_grid)


def load_int4(model, path, gemv_version=0, layouts=("mma",)):
    """Swap every TARGETS projection of `model` for a W4Linear on the packed weights saved at `path` (no
    quantization). Every projection must be in the file with its shape; biases come from the model's own layers.
    Returns (layers replaced, INT4 bytes), like apply_int4."""
    from . import store
    meta = store.read_meta(path)
    names = _names(model)
    todo = [(parent, attr, lin, names[id(lin)]) for parent, attr, lin in list(_projections(model))]
    missing = [q for *_, q in todo if q not in meta["names"]]
    if missing:
        raise KeyError(f"{path} has no entry {missing[0]!r}")
    dev = next(model.parameters()).device
    if dev.type != "cuda":
        dev = torch.device("cuda", torch.cuda.current_device())
    entries, group = store.load_w4(path, names=[q for *_, q in todo])
    for _, _, lin, q in todo:                         # every shape is checked before any layer is swapped
        packed = entries[q][0]
        if tuple(packed.shape) != (lin.out_features, lin.in_features // 2):
            raise ValueError(f"{q}: saved weight is {packed.shape[0]} x {packed.shape[1] * 2}, the layer is "
                             f"{lin.out_features} x {lin.in_features}")
    replaced, nbytes = 0, 0
    for parent, attr, lin, q in todo:
        packed, scales = entries.pop(q)
        wq = ops.W4Weight(packed, scales, group, layouts, device=dev)
        setattr(parent, attr, W4Linear(wq, lin.bias, lin.in_features, lin.out_features, gemv_version))
        replaced, nbytes = replaced + 1, nbytes + wq.nbytes()
    torch.cuda.empty_cache()
    return replaced, nbytes

"""lowbit: W4A16 (int4 weights, fp16 activations) kernels for AMD Instinct MI355X (gfx950).

Modules: quant (format, host side), ops (GPU weights, kernel dispatch), model (W4Linear for Hugging Face Qwen2, and
save_int4 / load_int4), store (the on-disk packed format), decode (graph decoding of a transformers model, random-init
Qwen2.5 shapes), fused (a Qwen2 decoder layer from the library's kernels).
The kernels live in liblowbit_w4.so (C ABI: include/lowbit_w4.h), built by lowbit-kernels_amd/build.py.
"""

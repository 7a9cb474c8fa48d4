"""A Qwen2 decoder forward assembled from the library's kernels, for batch-1 decoding with graph capture.

The stock transformers modules issue about fifty launches per decoder layer and token on ROCm (RMSNorm as five
elementwise ops, RoPE as six, bias and residual adds, cache index copies, mask construction); on MI355X, where a
small launch costs ~3 us, that overhead, not the projections, dominates a decode step. FusedQwen2 runs one layer as

    rmsnorm -> qkv projection (+bias) -> rope + cache write -> attention -> o projection (+residual, in place)
    -> rmsnorm -> gate|up projection (silu(gate) * up) -> down projection (+residual, in place)

(for one token with W4A16 projections the two RMSNorms run inside the q|k|v and gate|up GEMVs' prologues and RoPE +
cache write inside the q|k|v store, whose rows are permuted per head so that rotation partners share a tile: 6
launches, the attention's partition merge included)

with its own KV cache. The projections are either W4A16 (lowbit_w4_linear_fused: GEMV / MFMA kernels with the
consumer fused into the store, for up to 64 rows; dequantize + hipBLASLt beyond) or fp16 (hipBLASLt through torch,
bias and residual folded into addmm, silu * up as two torch ops), so the two variants share every other kernel and
differ only in the projections. Weights come from a transformers Qwen2ForCausalLM; q|k|v are merged into one
projection and gate|up into another, their rows interleaved 8 gate / 8 up per 16-row tile for the silu epilogue.
"""
import math

import torch
import torch.nn.functional as F

from . import _native, ops

EPI_STORE, EPI_BIAS, EPI_RESIDUAL, EPI_SILU_MUL = (_native.EPI_STORE, _native.EPI_BIAS, _native.EPI_RESIDUAL,
                                                   _native.EPI_SILU_MUL)


def interleave_gate_up(gate, up):
    """Rows [g0..g7, u0..u7, g8..g15, u8..u15, ...] of two [I, ...] tensors (I % 8 == 0)."""
    i = gate.shape[0]
    if i % 8 or up.shape[0] != i:
        raise ValueError("gate and up need the same row count, a multiple of 8")
    rest = gate.shape[1:]
    return torch.stack([gate.reshape(i // 8, 8, *rest), up.reshape(i // 8, 8, *rest)], 1).reshape(2 * i, *rest)


def rope_permutation(heads, head_dim=128):
    """Row order of a q|k|v projection for the fused RoPE: within each head, 16-row tile t holds dims 8 t .. 8 t + 7
    then their rotation partners head_dim / 2 + 8 t .. (row 16 (d / 8) + d % 8 holds dim d < head_dim / 2)."""
    half = head_dim // 2
    within = []
    for t in range(half // 8):
        within += [8 * t + r for r in range(8)] + [half + 8 * t + r for r in range(8)]
    return torch.tensor([h * head_dim + d for h in range(heads) for d in within], dtype=torch.long)


# Rows up to which a projection takes its input norm fused (norm_weight of lowbit_w4_linear_fused and
# lowbit_w4_qkv_rope_rows) rather than after a separate lowbit_rmsnorm launch. Every workgroup of the MFMA GEMM reads
# the rows whole for their statistics: up to 16 rows that costs less than the launch it saves, beyond it more (MI355X,
# graph-timed, cold weights: 3B gate|up 11.0 us fused against 11.3 for rmsnorm + GEMM at 16 rows, 16.9 against 14.5 at
# 48; 3B decode feeding 16 tokens a step 7980 -> 8250 tokens/s, 48 a step 19170 -> 18350 had it been fused there too).
FUSED_NORM_ROWS = 16


class _W4:
    """A merged W4A16 projection: W4Weight on the MFMA layout plus its bias."""

    def __init__(self, packed, scales, group, bias=None):
        self.wq = ops.W4Weight(packed, scales, group, ("mma",), device=packed.device)
        self.bias = bias

    def __call__(self, x, epilogue, aux=None, out=None, norm=None):
        wq = self.wq
        if x.shape[0] <= 64:                                 # the GEMV / MFMA GEMM, the input norm in its prologue
            if norm is not None and (x.shape[0] > FUSED_NORM_ROWS or x.shape[1] > (16384 if x.shape[0] == 1 else 8192)):
                x, norm = _normed(x, norm), None
            return ops.ext().w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, epilogue, aux, out, norm)
        x = _normed(x, norm)
        if ops.prefill_path(x.shape[0], wq):                 # the int4 prefill GEMM, epilogue fused
            return ops.ext().w4_gemm_prefill(x, wq.packed_mma, wq.scales, wq.group, epilogue, aux, out)
        w = ops.dequant(wq)                                  # prefill: dequantize + hipBLASLt, epilogue in torch
        return _torch_epilogue(x, w, epilogue, aux, out, round_first=True)


class _F16:
    """A merged fp16 projection (hipBLASLt through torch)."""

    def __init__(self, weight, bias=None):
        self.w, self.bias = weight, bias

    def __call__(self, x, epilogue, aux=None, out=None, norm=None):
        return _torch_epilogue(_normed(x, norm), self.w, epilogue, aux, out)


class _F16GEMV:
    """A merged fp16 projection through the library's fp16-weight GEMV for one row (lowbit_f16_linear_fused: the W4A16
    GEMV's structure, epilogues and fused input norm over fp16 weight bytes), hipBLASLt through torch for more rows."""

    def __init__(self, weight, bias=None):
        self.w, self.bias = weight, bias

    def __call__(self, x, epilogue, aux=None, out=None, norm=None):
        if x.shape[0] == 1 and self.w.shape[1] <= 16384:
            return ops.ext().f16_linear_fused(x, self.w, epilogue, aux, out, norm)
        return _torch_epilogue(_normed(x, norm), self.w, epilogue, aux, out)


def _normed(x, norm):
    """x, or lowbit_rmsnorm(x) * weight for norm = (weight, eps), for the routes without a fused input norm."""
    return x if norm is None else ops.ext().rmsnorm(x, norm[0], norm[1])


def _torch_epilogue(x, w, epilogue, aux, out, round_first=False):
    """The epilogues through torch. round_first: round the product to fp16, then add the bias or residual in fp16
    (the int4 kernels' rounding, so a W4A16 layer rounds alike on every route); otherwise fold the addend into addmm
    (one rounding, as nn.Linear with a bias does), which the fp16 projections use."""
    if round_first and epilogue in (EPI_BIAS, EPI_RESIDUAL):
        y = F.linear(x, w)
        if epilogue == EPI_BIAS:
            return torch.add(y, aux, out=out) if out is not None else y.add_(aux)
        return out.add_(y) if out is not None and out.data_ptr() == aux.data_ptr() else torch.add(aux, y, out=out)
    if epilogue == EPI_BIAS:
        return torch.addmm(aux, x, w.t(), out=out) if out is not None else torch.addmm(aux, x, w.t())
    if epilogue == EPI_RESIDUAL:
        if out is not None and out.data_ptr() == aux.data_ptr():
            return out.addmm_(x, w.t())
        return torch.addmm(aux, x, w.t(), out=out) if out is not None else torch.addmm(aux, x, w.t())
    y = F.linear(x, w)
    if epilogue == EPI_SILU_MUL:
        m = y.shape[0]
        gu = y.view(m, -1, 2, 8)
        r = (F.silu(gu[:, :, 0]) * gu[:, :, 1]).reshape(m, -1)
        return out.copy_(r) if out is not None else r
    return out.copy_(y) if out is not None else y


class FusedQwen2:
    """Batch-1 Qwen2 forward from the library's kernels (see the module docstring).

    build(model, max_len, quant, group, clip_grid): quant = "int4" quantizes every projection with the GPU quantizer
    (the same bits as lowbit.model.quantize_layers) and keeps only the packed weights; quant = "fp16" keeps fp16
    copies of the merged weights (hipBLASLt projections); quant = "fp16_gemv" keeps them too, in the int4 variant's
    row order, and runs one-token steps through the library's fp16-weight GEMV with the int4 variant's fusions (the
    same launches, only the weight bytes differ). forward(tokens [M], positions [M]) -> logits [M, vocab]; the KV cache rows at
    `positions` are written, rows 0..position are attended.
    """

    def __init__(self, model, max_len, quant="int4", group=128, clip_grid=None):
        cfg = model.config
        self.hidden, self.hq, self.hkv = cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads
        self.head_dim = getattr(cfg, "head_dim", None) or self.hidden // self.hq
        if self.head_dim != 128:
            raise ValueError("the fused attention kernels take head_dim 128")
        self.eps, self.max_len, self.quant = cfg.rms_norm_eps, max_len, quant
        dev = model.model.embed_tokens.weight.device
        self.embed = model.model.embed_tokens.weight.detach()
        self.head = model.lm_head.weight.detach()
        self.final_norm = model.model.norm.weight.detach()
        self.inv_freq = model.model.rotary_emb.inv_freq.detach().float().contiguous()
        self.scale = 1.0 / math.sqrt(self.head_dim)
        self.layers = []
        for layer in model.model.layers:
            att, mlp = layer.self_attn, layer.mlp
            qkv_w = torch.cat([att.q_proj.weight, att.k_proj.weight, att.v_proj.weight]).detach()
            qkv_b = torch.cat([att.q_proj.bias, att.k_proj.bias, att.v_proj.bias]).detach().half().contiguous()
            if quant in ("int4", "fp16_gemv"):               # rows in the fused RoPE's order (rope_permutation)
                perm = rope_permutation(self.hq + 2 * self.hkv, self.head_dim).to(qkv_w.device)
                qkv_w, qkv_b = qkv_w[perm], qkv_b[perm].contiguous()
            gu_w = interleave_gate_up(mlp.gate_proj.weight.detach(), mlp.up_proj.weight.detach())
            ws = {"qkv": qkv_w, "o": att.o_proj.weight.detach(), "gu": gu_w, "down": mlp.down_proj.weight.detach()}
            if quant == "int4":
                proj = {}
                for name, w in ws.items():
                    packed, scales = ops.quantize_w4_gpu(w, group, clip_grid)
                    proj[name] = _W4(packed, scales, group)
            elif quant == "fp16":
                proj = {name: _F16(w.half().contiguous()) for name, w in ws.items()}
            elif quant == "fp16_gemv":
                proj = {name: _F16GEMV(w.half().contiguous()) for name, w in ws.items()}
            else:
                raise ValueError("quant is 'int4', 'fp16' or 'fp16_gemv'")
            proj["qkv"].bias = qkv_b
            self.layers.append({"in_norm": layer.input_layernorm.weight.detach(),
                                "post_norm": layer.post_attention_layernorm.weight.detach(), **proj})
        n = len(self.layers)
        self.k_cache = torch.zeros(n, self.hkv, max_len, self.head_dim, dtype=torch.float16, device=dev)
        self.v_cache = torch.zeros_like(self.k_cache)

    def reset(self):
        self.k_cache.zero_()
        self.v_cache.zero_()

    def head_picks(self):
        """True when a one-row step's head can take the greedy pick along (lowbit_f16_gemv_pick)."""
        return self.hidden * 2 <= 65536

    def logits(self, xn, pick=None):
        """The tied fp16 head: the library's fp16 GEMV for up to 32 rows (hipBLASLt streams the head at ~3 TB/s at
        these shapes: 94 against 202 us at one row, 120 against 204 at 8, 135 against 204 at 16, 142 against 146 at
        32), hipBLASLt beyond (144 against 152 at 48). pick = (tokens, positions[, out_tokens, out_count, h_next]),
        one row (head_picks()): the GEMV also writes the greedy pick to tokens[0], advances positions[0] and, given
        the rest, appends the pick to out_tokens and writes its embedding row to h_next (the next step's input)."""
        if pick is not None:
            more = {}
            if len(pick) > 2:
                more = dict(out_tokens=pick[2], out_count=pick[3], embed=self.embed, h_out=pick[4])
            return ops.ext().f16_gemv_pick(xn, self.head, pick[0], pick[1], **more)
        m, k = xn.shape
        if (m <= 8 and m * k * 2 <= 65536) or (m <= 32 and k % 128 == 0):
            return ops.ext().f16_gemv(xn, self.head)
        return F.linear(xn, self.head)

    @torch.inference_mode()
    def forward(self, tokens, positions, last_only=False, pick=None, h=None):
        """tokens, positions: int64 [M] on the GPU -> logits fp16 [M, vocab] ([1, vocab] for the last position only
        when last_only, as a prefill needs). pick: see logits() (one-row steps). h: the tokens' embedding rows
        [M, hidden] when the caller already holds them (it becomes the residual stream, overwritten)."""
        ext = ops.ext()
        m = tokens.shape[0]
        h = F.embedding(tokens, self.embed) if h is None else h
        xn = torch.empty_like(h)
        q = torch.empty(m, self.hq, self.head_dim, dtype=torch.float16, device=h.device)
        attn = torch.empty(m, self.hq * self.head_dim, dtype=torch.float16, device=h.device)
        fuse = m == 1 and self.quant in ("int4", "fp16_gemv") and self.hidden <= 16384
        # more rows: the int4 GEMM that lay["qkv"] would pick (the MFMA GEMM up to 64 rows, the prefill GEMM where
        # prefill_path sends them) takes the RoPE epilogue too, its cos and sin from one table per step;
        # dequantize + BLAS keeps the separate rope_kv
        rope_rows = (not fuse and self.quant == "int4" and
                     (m <= 64 or ops.prefill_path(m, self.layers[0]["qkv"].wq)) if self.layers else False)
        table = ext.rope_table(positions, self.inv_freq) if rope_rows else None
        for i, lay in enumerate(self.layers):
            if fuse and self.quant == "fp16_gemv":
                ext.f16_qkv_rope(h, lay["qkv"].w, lay["qkv"].bias, positions, self.inv_freq, q, self.k_cache[i],
                                 self.v_cache[i], self.hq, self.hkv, norm=(lay["in_norm"], self.eps))
            elif fuse:                                        # RMSNorm in the prologue, RoPE + cache write in the store
                wq = lay["qkv"].wq
                ext.w4_qkv_rope(h, wq.packed_mma, wq.scales, wq.group, lay["qkv"].bias, positions, self.inv_freq, q,
                                self.k_cache[i], self.v_cache[i], self.hq, self.hkv, norm=(lay["in_norm"], self.eps))
            elif rope_rows:                                   # RoPE + cache write in the GEMM's store
                wq = lay["qkv"].wq
                if m <= FUSED_NORM_ROWS and self.hidden <= 8192:   # the MFMA GEMM normalizes its input itself
                    ext.w4_qkv_rope_rows(h, wq.packed_mma, wq.scales, wq.group, lay["qkv"].bias, positions, table, q,
                                         self.k_cache[i], self.v_cache[i], self.hq, self.hkv,
                                         norm=(lay["in_norm"], self.eps))
                else:
                    ext.rmsnorm(h, lay["in_norm"], self.eps, out=xn)
                    ext.w4_qkv_rope_rows(xn, wq.packed_mma, wq.scales, wq.group, lay["qkv"].bias, positions, table,
                                         q, self.k_cache[i], self.v_cache[i], self.hq, self.hkv)
            else:
                ext.rmsnorm(h, lay["in_norm"], self.eps, out=xn)
                qkv = lay["qkv"](xn, EPI_BIAS, lay["qkv"].bias)
                ext.rope_kv(qkv, positions, self.inv_freq, q, self.k_cache[i], self.v_cache[i], self.hq, self.hkv,
                            permuted=self.quant in ("int4", "fp16_gemv"))
            if fuse and self.hq <= 32:                        # the key partitions merged in the o projection
                o = lay["o"]
                if self.quant == "int4":
                    ext.w4_attention_linear(q, self.k_cache[i], self.v_cache[i], positions, self.hq, self.hkv,
                                            self.max_len, self.scale, o.wq.packed_mma, o.wq.scales, o.wq.group,
                                            EPI_RESIDUAL, h, out=h)
                else:
                    ext.f16_attention_linear(q, self.k_cache[i], self.v_cache[i], positions, self.hq, self.hkv,
                                             self.max_len, self.scale, o.w, EPI_RESIDUAL, h, out=h)
            else:
                ext.attention(q, self.k_cache[i], self.v_cache[i], positions, attn, self.hq, self.hkv, self.max_len,
                              self.scale)
                lay["o"](attn, EPI_RESIDUAL, h, out=h)
            if fuse or (self.quant == "int4" and m <= FUSED_NORM_ROWS and self.hidden <= 8192):   # normalized in the GEMM
                act = lay["gu"](h, EPI_SILU_MUL, norm=(lay["post_norm"], self.eps))
            else:
                ext.rmsnorm(h, lay["post_norm"], self.eps, out=xn)
                act = lay["gu"](xn, EPI_SILU_MUL)
            lay["down"](act, EPI_RESIDUAL, h, out=h)
        if last_only:
            h, xn = h[-1:], xn[-1:]
        ext.rmsnorm(h, self.final_norm, self.eps, out=xn)
        return self.logits(xn, pick if m == 1 else None)

    __call__ = forward


class FusedDecoder:
    """GraphDecoder's interface (prefill / capture / step / greedy) over a FusedQwen2."""

    def __init__(self, fused, chunk=1):
        self.f, self.chunk = fused, chunk
        dev = fused.embed.device
        self.tokens = torch.zeros(chunk, dtype=torch.long, device=dev)
        self.positions = torch.zeros(chunk, dtype=torch.long, device=dev)
        self.offsets = torch.arange(chunk, dtype=torch.long, device=dev)
        self.h = None                                       # the step's embedding rows when the head picks (capture)
        self.pos = 0
        self.graph = self.logits = self.next_token = None

    @torch.inference_mode()
    def prefill(self, ids):
        p = ids.shape[-1]
        if p > self.f.max_len:
            raise ValueError(f"a {p}-token prompt does not fit a {self.f.max_len}-token cache")
        self.f.reset()
        logits = self.f(ids.view(-1), torch.arange(p, device=ids.device), last_only=True)
        self.pos = p
        return logits[-1]

    @torch.inference_mode()
    def capture(self, warmup=2):
        if self.pos + self.chunk > self.f.max_len:
            raise ValueError("the cache has no room for a step after the prefill")
        self.positions.copy_(self.offsets + self.pos)
        # warm-up and capture on one stream, so the library's workspaces (keyed by stream) exist before capture
        # one token per step: the head GEMV picks the greedy token for the next replay itself (into tokens, one
        # position on, appended to out_tokens, its embedding row into h; lowbit_f16_gemv_pick), else argmax and the
        # feedback in torch. step() sets the buffers before each replay, so feeding given tokens is unaffected;
        # greedy() runs replays back to back
        pick, h = None, None
        if self.chunk == 1 and self.f.head_picks():
            dev = self.tokens.device
            self.h = F.embedding(self.tokens, self.f.embed)
            self.out_tokens = torch.zeros(self.f.max_len, dtype=torch.long, device=dev)
            self.out_count = torch.zeros(1, dtype=torch.int32, device=dev)
            pick, h = (self.tokens, self.positions, self.out_tokens, self.out_count, self.h), self.h
        s = _native.capture_stream(self.tokens.device)
        s.wait_stream(torch.cuda.current_stream())
        saved = (self.tokens.clone(), self.positions.clone(), None if h is None else h.clone())
        with torch.cuda.stream(s):
            for _ in range(warmup):
                self.f(self.tokens, self.positions, pick=pick, h=h)
                self.tokens.copy_(saved[0])
                self.positions.copy_(saved[1])
                if h is not None:
                    h.copy_(saved[2])
        torch.cuda.current_stream().wait_stream(s)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=s):
            self.logits = self.f(self.tokens, self.positions, pick=pick, h=h)
            if pick is not None:
                self.next_token = self.tokens
            else:
                self.next_token = self.logits[-1].argmax(-1)
                if self.chunk == 1:
                    self.tokens.copy_(self.next_token.view(1))
                    self.positions.add_(1)
        return self

    @torch.inference_mode()
    def eager_greedy(self, first, n):
        """n greedy tokens after a prefill, every step launched op by op from the host (no graph)."""
        if self.chunk != 1 or self.pos + n - 1 > self.f.max_len:
            raise ValueError("eager greedy decoding feeds one token per step within the cache")
        out = torch.empty(n, dtype=torch.long, device=self.tokens.device)
        out[0] = first
        for i in range(1, n):
            self.positions.fill_(self.pos)
            out[i] = self.f(out[i - 1].view(1), self.positions)[-1].argmax(-1)
            self.pos += 1
        return out

    @torch.inference_mode()
    def step(self, tokens):
        if self.pos + self.chunk > self.f.max_len:
            raise ValueError("the cache is full")
        self.tokens.copy_(tokens.view(self.chunk))
        self.positions.copy_(self.offsets + self.pos)
        if self.h is not None:
            torch.index_select(self.f.embed, 0, self.tokens, out=self.h)
        self.graph.replay()
        self.pos += self.chunk
        return self.logits

    @torch.inference_mode()
    def greedy(self, first, n):
        if self.chunk != 1:
            raise ValueError("greedy decoding feeds one token per step")
        if self.pos + n - 1 > self.f.max_len:
            raise ValueError("the cache is full")
        out = torch.empty(n, dtype=torch.long, device=self.tokens.device)
        out[0] = first
        self.tokens.copy_(out[:1])
        self.positions.fill_(self.pos)
        if self.h is not None:                              # the graph appends its picks and gathers their rows
            torch.index_select(self.f.embed, 0, self.tokens, out=self.h)
            self.out_count.zero_()
            for _ in range(1, n):
                self.graph.replay()
            self.pos += n - 1
            out[1:] = self.out_tokens[:n - 1]
            return out
        for i in range(1, n):                               # the graph feeds its argmax back (capture)
            self.graph.replay()
            self.pos += 1
            out[i] = self.next_token
        return out

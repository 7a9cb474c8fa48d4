"""Batch-1 decode of a Hugging Face causal LM with every step captured as one hipGraph over a static KV cache, and
the random-init Qwen2.5 architectures the benchmark runs it on.

The decode loop follows the reference's graph mode (bench/e2e.py:84-147): the prompt is prefilled eagerly into a
StaticCache (through ops.linear that is dequantize + hipBLASLt for every W4Linear), then a forward of `chunk` tokens
whose ids and cache positions live in fixed device tensors is captured once and replayed per step. The next token is
picked on the GPU inside the graph (argmax), so greedy decoding never synchronizes with the host.
"""
import torch

from . import _native

QWEN25 = {
    # hidden, intermediate, layers, query heads, kv heads (head_dim 128 throughout)
    "1.5b": (1536, 8960, 28, 12, 2),
    "3b": (2048, 11008, 36, 16, 2),
    "7b": (3584, 18944, 28, 28, 4),
    "tiny": (256, 512, 2, 2, 1),        # a two-layer model with real head geometry, for tests
}


def qwen25_config(name, vocab=None):
    """Qwen2Config of a Qwen2.5-`name`-shaped decoder: RMSNorm eps 1e-6, RoPE theta 1e6, SiLU MLP, q/k/v bias, tied
    fp16 embedding / head (untied for 7b), vocab 151936 unless `vocab` is given."""
    from transformers import Qwen2Config
    hidden, inter, layers, heads, kv = QWEN25[name]
    return Qwen2Config(hidden_size=hidden, intermediate_size=inter, num_hidden_layers=layers,
                       num_attention_heads=heads, num_key_value_heads=kv, head_dim=128,
                       vocab_size=vocab or (1024 if name == "tiny" else 151936), rms_norm_eps=1e-6,
                       rope_theta=1e6, max_position_embeddings=32768, hidden_act="silu",
                       tie_word_embeddings=name != "7b", initializer_range=0.02, use_cache=True)


@torch.no_grad()
def random_model(name, seed=0, device="cuda", vocab=None):
    """Qwen2ForCausalLM of that shape with its own initialisation (linear and embedding weights ~N(0, 0.02), zero
    biases, unit norms), built on `device` and cast to fp16, in eval mode. No checkpoint is read."""
    from transformers import Qwen2ForCausalLM
    torch.manual_seed(seed)
    with torch.device(device):
        m = Qwen2ForCausalLM(qwen25_config(name, vocab))
    gen = torch.Generator(device=device).manual_seed(seed + 1)
    for mod in m.modules():                     # draw every weight here, so the model depends only on `seed`
        if isinstance(mod, (torch.nn.Linear, torch.nn.Embedding)):
            mod.weight.normal_(0.0, 0.02, generator=gen)
            if getattr(mod, "bias", None) is not None:
                mod.bias.zero_()
    return m.half().eval()


def static_cache(model, max_len):
    from transformers import StaticCache
    return StaticCache(config=model.config, max_cache_len=max_len)


class GraphDecoder:
    """Feeds `chunk` tokens per step through `model` (batch 1) with the step captured as one hipGraph.

    prefill(ids) -> logits of the last prompt position (eager), step(tokens) -> logits [chunk, vocab] of the replayed
    graph (a view of a static tensor, overwritten by the next step), greedy(n) -> n greedy tokens after the prefill.
    """

    def __init__(self, model, max_len, chunk=1):
        self.m, self.chunk, self.max_len = model, chunk, max_len
        dev = next(model.parameters()).device
        self.cache = static_cache(model, max_len)
        self.tokens = torch.zeros(1, chunk, dtype=torch.long, device=dev)
        self.positions = torch.zeros(chunk, dtype=torch.long, device=dev)
        self.offsets = torch.arange(chunk, dtype=torch.long, device=dev)
        self.pos = 0
        self.graph = self.logits = self.next_token = None

    def _forward(self):
        out = self.m(input_ids=self.tokens, past_key_values=self.cache, cache_position=self.positions, use_cache=True)
        return out.logits[0]

    @torch.inference_mode()
    def prefill(self, ids):
        """Reset the cache and run the prompt ids [1, P] eagerly; returns the last position's logits."""
        p = ids.shape[1]
        if p > self.max_len:
            raise ValueError(f"a {p}-token prompt does not fit a {self.max_len}-token cache")
        self.cache.reset()
        out = self.m(input_ids=ids, past_key_values=self.cache,
                     cache_position=torch.arange(p, device=ids.device), use_cache=True)
        self.pos = p
        return out.logits[0, -1]

    def _sync_write_position(self):
        """Static cache layers (transformers >= 5) write new keys at a device-side counter of their own, advanced by
        every forward, not at cache_position; put it at the decoder's position (so warm-up forwards cannot run it past
        the end of the cache, and replays advance it in step with the decoder)."""
        for layer in getattr(self.cache, "layers", ()):
            n = getattr(layer, "cumulative_length", None)
            if torch.is_tensor(n):
                n.fill_(self.pos)

    @torch.inference_mode()
    def capture(self, warmup=3):
        """Warm up on the capture stream (first calls allocate the cache layers and the library's workspaces), then
        capture one step on the same stream. Must follow a prefill; the warm-up writes into cache rows past the prompt, which every
        real step overwrites before reading. Each replay then advances the cache's write position and the decoder's
        position together."""
        if self.pos + self.chunk > self.max_len:
            raise ValueError("the static cache has no room for a step after the prefill")
        self.positions.copy_(self.offsets + self.pos)
        # warm-up and capture on one stream, so the library's workspaces (keyed by stream) exist before capture
        s = _native.capture_stream(self.tokens.device)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(warmup):
                self._sync_write_position()          # every warm-up writes rows pos .. pos + chunk - 1 only
                self._forward()
            self._sync_write_position()
        torch.cuda.current_stream().wait_stream(s)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=s):
            self.logits = self._forward()
            self.next_token = self.logits[-1].argmax(-1)
        return self

    def step(self, tokens):
        """Feed `chunk` token ids (device tensor) at the current position; returns the step's logits."""
        if self.pos + self.chunk > self.max_len:
            raise ValueError("the static cache is full")
        self.tokens.copy_(tokens.view(1, self.chunk))
        self.positions.copy_(self.offsets + self.pos)
        self.graph.replay()
        self.pos += self.chunk
        return self.logits

    @torch.inference_mode()
    def greedy(self, first, n):
        """n tokens: `first` (the prefill's pick, a device scalar) then n - 1 greedy graph steps; stays on the GPU."""
        if self.chunk != 1:
            raise ValueError("greedy decoding feeds one token per step")
        out = torch.empty(n, dtype=torch.long, device=self.tokens.device)
        out[0] = first
        for i in range(1, n):
            self.step(out[i - 1])
            out[i] = self.next_token
        return out

    @torch.inference_mode()
    def eager_greedy(self, first, n):
        """greedy() without the graph: every step is the model's own forward, launched op by op from the host (the
        reference's eager decode, bench/e2e.py:54-69). Needs a prefill and a cache with room for n - 1 steps."""
        if self.chunk != 1 or self.pos + n - 1 > self.max_len:
            raise ValueError("eager greedy decoding feeds one token per step within the cache")
        out = torch.empty(n, dtype=torch.long, device=self.tokens.device)
        out[0] = first
        for i in range(1, n):
            self.tokens.copy_(out[i - 1].view(1, 1))
            self.positions.copy_(self.offsets + self.pos)
            self._sync_write_position()
            out[i] = self._forward()[-1].argmax(-1)
            self.pos += 1
        return out

"""lowbit_f16_gemv_pick on the GPU, through the C ABI: the logits are lowbit_f16_gemv's bit for bit, and the pick is
torch.argmax of those logits (random heads of the Qwen2.5 vocabulary size and ragged sizes; equal maxima, NaN rows,
signed zeros, all -inf), the feedback writes (token; position + 1, or none), and the pair captured in a graph and
replayed with new inputs between replays."""
import pytest
import torch

from lowbit import ops

pytestmark = pytest.mark.gpu


def run(x, w, positions=None):
    tokens = torch.full((1,), -7, dtype=torch.long, device=x.device)
    y = ops.ext().f16_gemv_pick(x, w, tokens, positions)
    return y, int(tokens.item())


@pytest.mark.parametrize("n,k", [(151936, 2048), (1, 8), (7, 64), (9, 136), (4099, 1536), (100, 3584)])
def test_pick_is_torch_argmax_of_the_logits(cuda, n, k):
    gen = torch.Generator().manual_seed(n + k)
    w = (torch.randn(n, k, generator=gen) * 0.05).half().cuda()
    for trial in range(3):
        x = torch.randn(1, k, generator=gen).half().cuda()
        y, tok = run(x, w)
        assert torch.equal(y, ops.ext().f16_gemv(x, w)), (n, k, trial)
        assert tok == int(torch.argmax(y[0]).item()), (n, k, trial)


def test_equal_maxima_take_the_first(cuda):
    gen = torch.Generator().manual_seed(2)
    n, k = 20000, 512
    w = (torch.randn(n, k, generator=gen) * 0.01).half()
    top = (torch.rand(k, generator=gen) + 1).half()
    x = torch.ones(1, k, dtype=torch.half).cuda()
    for idx in ([5, 9000, 19999], [19999, 19998], [0, 1], [12345, 8]):
        w2 = w.clone()
        w2[idx] = top                                       # the same row, so the same largest logit
        y, tok = run(x, w2.cuda())
        assert tok == min(idx) == int(torch.argmax(y[0]).item())


def test_special_values_follow_torch(cuda):
    k = 64
    x = torch.ones(1, k, dtype=torch.half).cuda()
    rows = {
        "all -inf": [torch.full((k,), float("-inf"))] * 9,
        "nan above numbers": [torch.full((k,), -1.0), torch.full((k,), float("nan")), torch.full((k,), 2.0),
                              torch.full((k,), float("nan"))],
        "-0 ties +0": [torch.full((k,), -1.0), torch.full((k,), -0.0), torch.zeros(k), torch.full((k,), -2.0)],
        "+0 then -0": [torch.full((k,), -1.0), torch.zeros(k), torch.full((k,), -0.0)],
    }
    for name, r in rows.items():
        w = torch.stack(r).half().cuda()
        y, tok = run(x, w)
        assert tok == int(torch.argmax(y[0]).item()), (name, y)


def test_feedback_and_graph_replays(cuda):
    gen = torch.Generator().manual_seed(4)
    n, k = 151936, 2048
    w = (torch.randn(n, k, generator=gen) * 0.05).half().cuda()
    x = torch.zeros(1, k, dtype=torch.half, device="cuda")
    tokens = torch.zeros(1, dtype=torch.long, device="cuda")
    positions = torch.tensor([40], dtype=torch.long, device="cuda")
    ops.ext().f16_gemv_pick(x, w, tokens, positions)                     # workspace exists before capture
    assert int(positions.item()) == 41
    ops.ext().f16_gemv_pick(x, w, tokens)                                # no positions: left as they are
    assert int(positions.item()) == 41
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.ext().f16_gemv_pick(x, w, tokens, positions)                 # this stream's workspace
    torch.cuda.current_stream().wait_stream(s)
    positions.fill_(0)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        y = ops.ext().f16_gemv_pick(x, w, tokens, positions)
    for i in range(4):
        x.copy_(torch.randn(1, k, generator=gen).half().cuda())
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = ops.ext().f16_gemv(x, w)
        assert torch.equal(y, want) and int(tokens.item()) == int(torch.argmax(want[0]).item())
        assert int(positions.item()) == i + 1


def test_append_and_next_embedding(cuda):
    """out_tokens / out_count: each call appends its pick while there is room and counts on past it; embed / h_out:
    h_out is the pick's row of embed, which may be a tensor other than the head (an untied embedding)."""
    gen = torch.Generator().manual_seed(6)
    n, k = 4099, 1536
    w = (torch.randn(n, k, generator=gen) * 0.05).half().cuda()
    embed = torch.randn(n, k, generator=gen).half().cuda()
    tokens = torch.zeros(1, dtype=torch.long, device="cuda")
    out_tokens = torch.full((3,), -1, dtype=torch.long, device="cuda")
    out_count = torch.zeros(1, dtype=torch.int32, device="cuda")
    h = torch.zeros(1, k, dtype=torch.half, device="cuda")
    picks = []
    for i in range(5):
        x = torch.randn(1, k, generator=gen).half().cuda()
        y = ops.ext().f16_gemv_pick(x, w, tokens, None, out_tokens=out_tokens, out_count=out_count, embed=embed, h_out=h)
        tok = int(torch.argmax(y[0]).item())
        picks.append(tok)
        assert int(tokens.item()) == tok and int(out_count.item()) == i + 1
        assert torch.equal(h[0], embed[tok]), i
    assert out_tokens.tolist() == picks[:3]
    with pytest.raises(RuntimeError, match="goes with"):
        ops.ext().f16_gemv_pick(x, w, tokens, out_tokens=out_tokens)
    with pytest.raises(RuntimeError, match="h_out"):
        ops.ext().f16_gemv_pick(x, w, tokens, embed=embed, h_out=h[:, :8])

"""Kernels and the model forward on side streams and in a captured graph.

Every launch of the library goes to the stream it is given (torch's current
stream in the Python layer), including the helper launches a call adds — the
weight prefetch ahead of a large persistent GEMM, the fill kernels of the
forward.  So a call on a side stream, and calls on two streams at once, give
results equal bit for bit to the same calls on the default stream, and no
work is left behind on the default stream.  The streams here are created at
the default priority.
"""

import pytest
import torch

from cutilegpt_amd import CutileGPT, GPTConfig
from cutilegpt_amd import kernels as K

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def bits(t):
    return t.view(torch.int32) if t.element_size() == 4 else t.view(torch.int16)


def randn(gpu, *shape, seed, scale=1.0, dtype=BF16):
    g = torch.Generator(device=gpu).manual_seed(seed)
    return (torch.randn(*shape, device=gpu, generator=g) * scale).to(dtype)


def on_stream(s, fn):
    """Run fn on stream s after the default stream's pending work; the
    default stream waits for s afterwards."""
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = fn()
    torch.cuda.current_stream().wait_stream(s)
    return out


def test_prefetched_gemm_on_side_stream(gpu):
    # A 77 MB weight and M >= 1024: the persistent GEMM is preceded by the
    # weight prefetch, which must run on the same stream.
    x = randn(gpu, 2048, 768, seed=1)
    w = randn(gpu, 50304, 768, seed=2, scale=0.02)
    ref = K.cutile_linear(x, w)
    torch.cuda.synchronize()
    s = torch.cuda.Stream(device=gpu)
    out = on_stream(s, lambda: K.cutile_linear(x, w))
    torch.cuda.synchronize()
    assert torch.equal(bits(out), bits(ref))


def test_two_streams_at_once(gpu):
    # Stream A: a GEMM chain (bias, then GELU epilogue); stream B: attention,
    # LayerNorm and GELU.  Each equals its serial run on the default stream.
    x = randn(gpu, 4096, 768, seed=3)
    w1 = randn(gpu, 2304, 768, seed=4, scale=0.05)
    b1 = randn(gpu, 2304, seed=5, scale=0.05)
    w2 = randn(gpu, 3072, 2304, seed=6, scale=0.02)
    b2 = randn(gpu, 3072, seed=7, scale=0.02)
    q, k, v = (randn(gpu, 4, 12, 512, 64, seed=8 + i) for i in range(3))
    y = randn(gpu, 8192, 768, seed=11)
    gam = randn(gpu, 768, seed=12, scale=0.1, dtype=torch.float32) + 1
    bet = randn(gpu, 768, seed=13, scale=0.1, dtype=torch.float32)

    def chain_a():
        return K.linear_bias_gelu(K.cutile_linear_bias(x, w1, b1), w2, b2)

    def chain_b():
        a = K.cutile_causal_attention(q, k, v, 12)
        return a, K.cutile_gelu(K.cutile_layer_norm(y, gam, bet))

    ref_a = chain_a()
    ref_att, ref_ln = chain_b()
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(device=gpu), torch.cuda.Stream(device=gpu)
    for _ in range(3):
        sa.wait_stream(torch.cuda.current_stream())
        sb.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(sa):
            out_a = chain_a()
        with torch.cuda.stream(sb):
            out_att, out_ln = chain_b()
        torch.cuda.current_stream().wait_stream(sa)
        torch.cuda.current_stream().wait_stream(sb)
        torch.cuda.synchronize()
        assert torch.equal(bits(out_a), bits(ref_a))
        assert torch.equal(bits(out_att), bits(ref_att))
        assert torch.equal(bits(out_ln), bits(ref_ln))


@pytest.mark.parametrize("dtype", [torch.float32, BF16])
def test_model_forward_on_side_stream(gpu, dtype):
    cfg = GPTConfig.gpt_mini()
    m = CutileGPT(cfg, dtype=dtype, seed=0)
    idx = torch.randint(0, cfg.vocab_size, (4, 100), generator=torch.Generator().manual_seed(0)).to(gpu)
    ref, _ = m(idx)
    torch.cuda.synchronize()
    s = torch.cuda.Stream(device=gpu)
    out, _ = on_stream(s, lambda: m(idx))
    torch.cuda.synchronize()
    assert torch.equal(bits(out), bits(ref))


@pytest.mark.parametrize("dtype", [torch.float32, BF16])
def test_model_forward_graph_replay(gpu, dtype):
    # The forward issues no host synchronisation and no memset, so it can be
    # captured; each replay (new token ids in the captured input buffer, eager
    # forwards in between) equals the eager forward bit for bit.
    cfg = GPTConfig.gpt_mini()
    m = CutileGPT(cfg, dtype=dtype, seed=0)
    gen = torch.Generator().manual_seed(1)
    idx = torch.randint(0, cfg.vocab_size, (4, 100), generator=gen).to(gpu)
    m(idx)  # allocations made once outside the capture (error flag)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream(device=gpu)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            static_out, _ = m(idx)
    torch.cuda.current_stream().wait_stream(s)
    for r in range(3):
        idx.copy_(torch.randint(0, cfg.vocab_size, (4, 100), generator=gen).to(gpu))
        graph.replay()
        replayed = static_out.clone()
        eager, _ = m(idx)
        torch.cuda.synchronize()
        assert torch.equal(bits(replayed), bits(eager)), f"replay {r}"

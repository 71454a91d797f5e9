"""The CPU oracle pinned against independent implementations and mathematics.

Every oracle function is checked against something that is not its own
formula: torch.nn.functional routines, brute-force loops, closed-form special
cases, the transformers GPT-2 implementation and the committed golden fixture.
"""

import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gpt_ref as R

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "nano_seed0.npz")


def test_gelu_matches_torch_tanh_gelu():
    x = torch.linspace(-8, 8, 4001, dtype=torch.float64)
    torch.testing.assert_close(R.gelu_tanh(x), F.gelu(x, approximate="tanh"), rtol=0, atol=1e-15)


def test_gelu_identities():
    x = torch.randn(1000, dtype=torch.float64, generator=torch.Generator().manual_seed(0)) * 4
    # 0.5 x (1 + tanh u) is odd-symmetric up to x: gelu(x) - gelu(-x) = x
    torch.testing.assert_close(R.gelu_tanh(x) - R.gelu_tanh(-x), x, rtol=0, atol=1e-12)
    assert R.gelu_tanh(torch.zeros(1, dtype=torch.float64)).item() == 0.0
    big = torch.tensor([30.0, -30.0], dtype=torch.float64)
    torch.testing.assert_close(R.gelu_tanh(big), torch.tensor([30.0, 0.0], dtype=torch.float64))
    # tanh(1) closed form at x where u = 1
    # u = sqrt(2/pi)(x + 0.044715 x^3) = 1 has a root near x = 1.1514...
    root = torch.tensor(1.0, dtype=torch.float64)
    for _ in range(60):
        u = math.sqrt(2 / math.pi) * (root + 0.044715 * root ** 3) - 1
        du = math.sqrt(2 / math.pi) * (1 + 3 * 0.044715 * root ** 2)
        root = root - u / du
    assert abs(R.gelu_tanh(root).item() - 0.5 * root.item() * (1 + math.tanh(1.0))) < 1e-14


def test_layer_norm_matches_torch():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(37, 768, dtype=torch.float64, generator=g) * 3 + 2
    w = 1 + 0.1 * torch.randn(768, dtype=torch.float64, generator=g)
    b = 0.1 * torch.randn(768, dtype=torch.float64, generator=g)
    torch.testing.assert_close(R.layer_norm(x, w, b), F.layer_norm(x, (768,), w, b, 1e-5),
                               rtol=1e-12, atol=1e-12)


def test_layer_norm_invariants():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(8, 48, dtype=torch.float64, generator=g)
    w, b = torch.ones(48, dtype=torch.float64), torch.zeros(48, dtype=torch.float64)
    y = R.layer_norm(x, w, b)
    torch.testing.assert_close(y.mean(-1), torch.zeros(8, dtype=torch.float64), atol=1e-12, rtol=0)
    # biased variance of the output is var/(var+eps)
    var = x.var(-1, unbiased=False)
    torch.testing.assert_close(y.var(-1, unbiased=False), var / (var + 1e-5), atol=1e-12, rtol=0)
    beta = torch.randn(48, dtype=torch.float64, generator=g)
    const = torch.full((3, 48), 7.25, dtype=torch.float64)
    torch.testing.assert_close(R.layer_norm(const, w, beta), beta.expand(3, 48))
    torch.testing.assert_close(R.layer_norm(x + 5.0, w, b), y, atol=1e-10, rtol=0)


def test_linear_brute_force():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 7, dtype=torch.float64, generator=g)
    w = torch.randn(3, 7, dtype=torch.float64, generator=g)
    b = torch.randn(3, dtype=torch.float64, generator=g)
    ref = torch.empty(5, 3, dtype=torch.float64)
    for i in range(5):
        for j in range(3):
            ref[i, j] = sum(x[i, k] * w[j, k] for k in range(7)) + b[j]
    torch.testing.assert_close(R.linear(x, w, b), ref)
    onehot = torch.zeros(3, 7, dtype=torch.float64)
    onehot[0, 4] = onehot[1, 0] = onehot[2, 6] = 1
    torch.testing.assert_close(R.linear(x, onehot), x[:, [4, 0, 6]])


def _attn_loop(q, k, v):
    B, H, T, d = q.shape
    out = torch.zeros_like(q)
    for b in range(B):
        for h in range(H):
            for i in range(T):
                s = torch.tensor([float(q[b, h, i] @ k[b, h, j]) / math.sqrt(d) for j in range(i + 1)],
                                 dtype=torch.float64)
                p = torch.exp(s - s.max())
                p = p / p.sum()
                out[b, h, i] = sum(p[j] * v[b, h, j] for j in range(i + 1))
    return out


def test_attention_brute_force_and_sdpa():
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(2, 2, 9, 16, dtype=torch.float64, generator=g) for _ in range(3))
    o = R.causal_attention(q, k, v)
    torch.testing.assert_close(o, _attn_loop(q, k, v), rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(o, F.scaled_dot_product_attention(q, k, v, is_causal=True),
                               rtol=1e-10, atol=1e-10)


def test_attention_special_cases():
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, 3, 17, 32, dtype=torch.float64, generator=g) for _ in range(3))
    o = R.causal_attention(q, k, v)
    torch.testing.assert_close(o[:, :, 0], v[:, :, 0])  # row 0 sees only key 0
    keq = k[:, :, :1].expand_as(k)  # equal keys -> prefix mean of V
    prefix_mean = v.cumsum(2) / torch.arange(1, 18, dtype=torch.float64).view(1, 1, 17, 1)
    torch.testing.assert_close(R.causal_attention(q, keq, v), prefix_mean)
    # a decode step (Tq = 1) equals the last row of the prefill
    torch.testing.assert_close(R.causal_attention(q[:, :, -1:], k, v), o[:, :, -1:])
    # Tq < Tk: the queries are the last Tq rows of the Tk-row prefill
    torch.testing.assert_close(R.causal_attention(q[:, :, -5:], k, v), o[:, :, -5:])


def test_attention_non_causal_matches_sdpa_and_closed_forms():
    g = torch.Generator().manual_seed(6)
    q, k, v = (torch.randn(2, 3, 11, 16, dtype=torch.float64, generator=g) for _ in range(3))
    o = R.causal_attention(q, k, v, causal=False)
    torch.testing.assert_close(o, F.scaled_dot_product_attention(q, k, v, is_causal=False),
                               rtol=1e-10, atol=1e-10)
    # every query sees every key: equal keys give the plain mean of V in every row
    keq = k[:, :, :1].expand_as(k)
    torch.testing.assert_close(R.causal_attention(q, keq, v, causal=False),
                               v.mean(2, keepdim=True).expand_as(v))
    # Tq < Tk without the mask: the rows are those of the full query set
    kk, vv = (torch.randn(2, 3, 19, 16, dtype=torch.float64, generator=g) for _ in range(2))
    torch.testing.assert_close(R.causal_attention(q[:, :, :4], kk, vv, causal=False),
                               F.scaled_dot_product_attention(q[:, :, :4], kk, vv),
                               rtol=1e-10, atol=1e-10)


def test_embedding_exact():
    w = torch.randn(11, 4, dtype=torch.float64)
    idx = torch.tensor([[3, 0, 10], [10, 10, 1]])
    assert torch.equal(R.embedding(idx, w), torch.stack([torch.stack([w[i] for i in r]) for r in idx]))


def test_init_recipe_matches_golden_recipe():
    from tests.golden.make_golden import nano_weights
    a = R.init_weights(3, 3, 48, seed=0)
    b = nano_weights(0)
    for key in b:
        assert torch.equal(a[key], b[key]), key
    assert a["lm_head.weight"] is a["wte"]


@pytest.fixture(scope="module")
def nano():
    from tests.golden.make_golden import hf_model
    w = R.init_weights(3, 3, 48, seed=0)
    return w, hf_model(w, 3, 3, 48)


def test_forward_matches_transformers_gpt2(nano):
    w, m = nano
    ids = torch.randint(0, 50257, (2, 40), generator=torch.Generator().manual_seed(7))
    with torch.no_grad():
        ref = m.double()(ids).logits
    out = R.gpt_forward(w, ids, 3, R.FLOWS["fp64"])
    assert (out - ref).abs().max().item() < 1e-10
    out32 = R.gpt_forward(w, ids, 3, R.FLOWS["fp32"])
    assert (out32.double() - ref).abs().max().item() < 1e-5


def test_forward_matches_transformers_with_checkpoint_like_params():
    """Every bias ~N(0, 0.1), LayerNorm gamma ~N(1, 0.1), beta ~N(0, 0.1), each
    drawn separately: the oracle's routing of each tensor
    (cutile_gpt/models/gpt.py:120-177) equals transformers' GPT-2 to fp64
    rounding, and exchanging any two of them (a planted slip) moves the
    transformers result far beyond the fp32 bar, so the comparison sees it."""
    from tests.golden.make_golden import hf_model
    L, H, D = 3, 3, 48
    w = R.randomize_affine(R.init_weights(L, H, D, seed=4), seed=40)
    for i in range(L):
        assert not torch.equal(w[f"h.{i}.attn.c_proj.bias"], w[f"h.{i}.mlp.c_proj.bias"])
        assert not torch.equal(w[f"h.{i}.ln_1.weight"], w[f"h.{i}.ln_2.weight"])
        assert (w[f"h.{i}.ln_2.weight"] - 1).abs().max() > 0.1
    assert not torch.equal(w["h.0.ln_1.bias"], w["h.1.ln_1.bias"])
    assert w["ln_f.bias"].abs().max() > 0.1 and w["lm_head.weight"] is w["wte"]
    ids = torch.randint(0, 50257, (2, 40), generator=torch.Generator().manual_seed(41))
    with torch.no_grad():
        ref = hf_model(w, L, H, D).double()(ids).logits
    out = R.gpt_forward(w, ids, H, R.FLOWS["fp64"])
    assert (out - ref).abs().max().item() < 1e-10
    for a, b in (("h.0.attn.c_proj.bias", "h.0.mlp.c_proj.bias"),
                 ("h.1.ln_1.weight", "h.1.ln_2.weight"), ("h.2.ln_1.bias", "h.2.ln_2.bias"),
                 ("h.0.attn.c_attn.bias", "h.1.attn.c_attn.bias"),
                 ("h.1.mlp.c_fc.bias", "h.2.mlp.c_fc.bias"), ("ln_f.bias", "h.2.ln_2.bias")):
        bad = dict(w)
        bad[a], bad[b] = w[b], w[a]
        d = (R.gpt_forward(bad, ids, H, R.FLOWS["fp64"]) - ref).abs().max().item()
        assert d > 1e-2, (a, b, d)


def test_forward_matches_golden_fixture():
    gold = np.load(GOLDEN)
    w = R.init_weights(3, 3, 48, seed=0)
    ids = torch.from_numpy(gold["ids"])
    out = R.gpt_forward(w, ids, 3, R.FLOWS["fp64"])[0]
    np.testing.assert_allclose(out[-1].numpy(), gold["last_logits"], rtol=0, atol=1e-10)
    np.testing.assert_array_equal(out.argmax(-1).numpy(), gold["argmax"])
    np.testing.assert_allclose(out.sum(-1).numpy(), gold["row_sum"], rtol=0, atol=1e-8)
    np.testing.assert_allclose(out.abs().amax(-1).numpy(), gold["row_absmax"], rtol=0, atol=1e-10)


def test_generate_matches_golden_greedy():
    gold = np.load(GOLDEN)
    w = R.init_weights(3, 3, 48, seed=0)
    out = R.generate(w, torch.from_numpy(gold["greedy_prompt"]), 3, 8, R.FLOWS["fp64"])
    np.testing.assert_array_equal(out.numpy(), gold["greedy_out"])


def test_bf16_flows_error_budget():
    """The bf16 flows stay within the bf16 tolerance of the exact result on a
    small model (a sanity bound on the flows themselves)."""
    w = R.init_weights(2, 4, 64, seed=3, dtype=torch.bfloat16, block_size=64)
    ids = torch.randint(0, 50257, (2, 64), generator=torch.Generator().manual_seed(9))
    exact = R.gpt_forward(w, ids, 4, R.FLOWS["fp64"])
    for name in ("bf16", "bf16_ref"):
        d = (R.gpt_forward(w, ids, 4, R.FLOWS[name]).double() - exact).abs().max().item()
        assert d < 3e-2, (name, d)


def test_forward_cached_in_parts_equals_one_pass():
    """Positions run in parts with the earlier keys/values kept give the logits
    of one pass over all positions (fp64: to rounding; bf16 flow: the same
    rounding points, so the same values up to fp32 summation order)."""
    w = R.init_weights(2, 4, 64, seed=12, dtype=torch.bfloat16, block_size=128)
    ids = torch.randint(0, 50257, (3, 37), generator=torch.Generator().manual_seed(13))
    for flow, tol in ((R.FLOWS["fp64"], 1e-10), (R.FLOWS["bf16"], 2e-2)):
        full = R.gpt_forward(w, ids, 4, flow)
        a, cache = R.forward_cached(w, ids[:, :20], 4, flow)
        b, cache = R.forward_cached(w, ids[:, 20:33], 4, flow, cache)
        c, cache = R.forward_cached(w, ids[:, 33:], 4, flow, cache)
        assert cache[0][0].shape == (3, 4, 37, 16)
        parts = torch.cat([a, b, c], dim=1)
        assert (parts.double() - full.double()).abs().max().item() <= tol, flow.name
        if flow.name == "fp64":
            assert torch.equal(parts.argmax(-1), full.argmax(-1))


@pytest.mark.parametrize("flow", ["fp64", "fp32", "bf16"])
def test_generate_cached_equals_full_recompute(flow):
    """The cached greedy loop (used to write the long-stream fixtures) gives the
    full-recompute generate's tokens, and its per-step logits are the last rows
    of a full forward over the produced sequence."""
    f = R.FLOWS[flow]
    w = R.init_weights(2, 2, 64, seed=14, dtype=torch.bfloat16 if flow == "bf16" else torch.float32)
    ids = torch.randint(0, 50257, (2, 9), generator=torch.Generator().manual_seed(15))
    ref = R.generate(w, ids, 2, 12, f)
    out, lg = R.generate_cached(w, ids, 2, 12, f, return_logits=True)
    assert torch.equal(out, ref)
    full = R.gpt_forward(w, out[:, :-1], 2, f)[:, 8:]
    tol = 1e-10 if flow == "fp64" else 2e-2
    assert (lg.double() - full.double()).abs().max().item() <= tol


def test_generate_cached_matches_golden_greedy():
    gold = np.load(GOLDEN)
    w = R.init_weights(3, 3, 48, seed=0)
    out = R.generate_cached(w, torch.from_numpy(gold["greedy_prompt"]), 3, 8, R.FLOWS["fp64"])
    np.testing.assert_array_equal(out.numpy(), gold["greedy_out"])


@pytest.mark.parametrize("lazy", [0.0, 8.0])
def test_online_attention_equals_two_pass(lazy):
    """The online form is exact algebra: in float64 it equals the two-pass
    softmax (causal, Tq < Tk, non-causal), lazy rescaling or not."""
    g = torch.Generator().manual_seed(16)
    q, k, v = (torch.randn(2, 3, 150, 16, dtype=torch.float64, generator=g) * 3 for _ in range(3))
    for args in ((q, k, v), (q[:, :, 100:], k, v)):
        torch.testing.assert_close(R.online_attention(*args, lazy_log2=lazy),
                                   R.causal_attention(*args), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(R.online_attention(q, k, v, causal=False, lazy_log2=lazy),
                               R.causal_attention(q, k, v, causal=False), rtol=1e-12, atol=1e-12)


def test_online_attention_rounding_point():
    """Where key 0 carries every row's largest score, the running maximum is the
    final one from the first block on, so P rounded to bf16 per block equals
    P rounded after a two-pass softmax; where a later block raises the maximum,
    the per-block rounding differs (it is relative to the running maximum)."""
    g = torch.Generator().manual_seed(17)
    q = torch.randn(1, 2, 200, 16, dtype=torch.float64, generator=g)
    q[..., 0] = 5.0  # every query points along axis 0 ...
    k = torch.randn(1, 2, 200, 16, dtype=torch.float64, generator=g) * 0.1
    k[:, :, 0, 0] = 4.0  # ... and key 0 does too: the largest score of every row
    v = torch.randn(1, 2, 200, 16, dtype=torch.float64, generator=g)
    s = q @ k.transpose(-1, -2)
    assert bool((s.argmax(-1) == 0).all())
    bf = torch.bfloat16
    torch.testing.assert_close(R.online_attention(q, k, v, bf), R.causal_attention(q, k, v, bf),
                               rtol=1e-12, atol=1e-12)
    k2 = torch.randn(1, 2, 200, 16, dtype=torch.float64, generator=g) * 2
    assert (R.online_attention(q, k2, v, bf) - R.causal_attention(q, k2, v, bf)).abs().max() > 1e-6

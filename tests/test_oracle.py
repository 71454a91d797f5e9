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

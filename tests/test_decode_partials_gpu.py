"""Decode-step kernels that hand a GEMM's split-K reduction to its consumer:
cgpt_gemm_partials, cgpt_add_layernorm_partials,
cgpt_attention_decode_partials and cgpt_partials_bias_act.

The partial products are pinned against fp64 products of the K chunks they
cover; the consumers are pinned against the direct-input kernels fed with the
same reduction done on the host in the same order (fp32 additions are exact
IEEE operations, so those inputs are bit-identical), and the attention's
multi-chunk path against the oracle's causal attention.
"""

import math

import pytest
import torch

from cutilegpt_amd import _lib
from cutilegpt_amd.decode import DecodeSession
from oracle import gpt_ref as R

pytestmark = pytest.mark.gpu
DT = {torch.float32: _lib.CGPT_F32, torch.bfloat16: _lib.CGPT_BF16}


def stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def kd(dtype):
    """k per double slab (the unit K chunks are counted in)."""
    return 64 if dtype == torch.bfloat16 else 32


def plan(lib, M, N, K, dtype):
    import ctypes
    ns = ctypes.c_int64()
    _lib.check(lib.cgpt_gemm_partials_plan(M, N, K, DT[dtype], ctypes.byref(ns)), "plan")
    return ns.value


def reduce_in_order(parts, bias=None):
    """P[0] + P[1] + ... (+ bias), fp32, left to right as the kernels add."""
    t = parts[0].clone()
    for s in range(1, parts.shape[0]):
        t = t + parts[s]
    if bias is not None:
        t = t + bias.float()
    return t


# --------------------------------------------------------------- GEMM partials

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K", [(1, 16, 64), (5, 50, 72), (17, 96, 256), (32, 1600, 1600),
                                   (32, 4800, 1600), (32, 1600, 6400), (33, 70, 520),
                                   (64, 200, 6400)])
def test_gemm_partials_chunks_vs_fp64(gpu, dtype, M, N, K):
    lib = _lib.load()
    g = torch.Generator().manual_seed(M * 31 + N + K)
    a = torch.randn(M, K, generator=g).to(dtype)
    w = (torch.randn(N, K, generator=g) * 0.05).to(dtype)
    ad, wd = a.to(gpu), w.to(gpu)
    dslabs = -(-K // kd(dtype))
    splits = sorted({1, plan(lib, M, N, K, dtype), min(dslabs, 16), dslabs})
    for S in splits:
        ldp = N + 3  # padded rows: the padding must stay untouched
        p = torch.full((S + 1, M, ldp), float("nan"), device=gpu)
        _lib.check(lib.cgpt_gemm_partials(ad.data_ptr(), wd.data_ptr(), p.data_ptr(), M, N, K, K, K,
                                          ldp, S, DT[dtype], stream(gpu)), "partials")
        torch.cuda.synchronize()
        pc = p.cpu().double()
        assert torch.isnan(pc[:S, :, N:]).all() and torch.isnan(pc[S]).all()
        # Chunk s covers double slabs [s * c, (s + 1) * c), c = ceil(dslabs / S).
        c = -(-dslabs // S)
        scale = (a.double().abs() @ w.double().abs().t()).max().item() + 1.0
        for s in range(S):
            k0, k1 = min(K, s * c * kd(dtype)), min(K, (s + 1) * c * kd(dtype))
            ref = a[:, k0:k1].double() @ w[:, k0:k1].double().t()
            e = (pc[s, :, :N] - ref).abs().max().item() if k1 > k0 else pc[s, :, :N].abs().max().item()
            assert e <= 2e-5 * scale, (S, s, e)
        tot = (a.double() @ w.double().t())
        assert (pc[:S, :, :N].sum(0) - tot).abs().max().item() <= 2e-5 * scale * S


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K", [(32, 1600, 6400), (32, 6400, 1600), (64, 1024, 4096),
                                   (8, 768, 3072), (32, 1280, 5120)])
def test_gemm_partials_plan_fits_the_consumers(gpu, dtype, M, N, K):
    """The planned split never exceeds the 16 partials the decode step's
    consumers add (fp32 at K = 6400 alone would take 20 chunks of 10)."""
    lib = _lib.load()
    dslabs = -(-K // kd(dtype))
    assert 1 <= plan(lib, M, N, K, dtype) <= min(16, dslabs)


def test_gemm_partials_unaligned_output_and_limits(gpu):
    lib = _lib.load()
    M, N, K = 7, 30, 128
    a = torch.randn(M, K, device=gpu).bfloat16()
    w = torch.randn(N, K, device=gpu).bfloat16()
    buf = torch.full((2 * M * N + 1,), float("nan"), device=gpu)
    # One float past a 16-byte boundary: scalar stores.
    _lib.check(lib.cgpt_gemm_partials(a.data_ptr(), w.data_ptr(), buf.data_ptr() + 4, M, N, K, K, K,
                                      N, 2, _lib.CGPT_BF16, stream(gpu)), "partials")
    torch.cuda.synchronize()
    p = buf[1:].view(2, M, N).double()
    ref = a.double() @ w.double().t()
    assert (p.sum(0) - ref).abs().max().item() <= 1e-3
    assert torch.isnan(buf[0])
    args = (a.data_ptr(), w.data_ptr(), buf.data_ptr())
    assert lib.cgpt_gemm_partials(*args, M, N, K, K, K, N, 0, _lib.CGPT_BF16, 0) == -1
    assert lib.cgpt_gemm_partials(*args, M, N, K, K, K, N, 3, _lib.CGPT_BF16, 0) == -1  # > 2 slabs
    assert lib.cgpt_gemm_partials(*args, M, N, K, K, K, N - 1, 1, _lib.CGPT_BF16, 0) == -1
    assert lib.cgpt_gemm_partials(*args, 65, N, K, K, K, N, 1, _lib.CGPT_BF16, 0) == -3


# ------------------------------------------------- residual + LayerNorm consumer

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,cols,S", [(32, 1600, 5), (3, 100, 1), (64, 768, 16), (5, 4096, 3)])
@pytest.mark.parametrize("with_bias", [True, False])
def test_add_layernorm_partials_matches_host_reduction(gpu, dtype, rows, cols, S, with_bias):
    lib = _lib.load()
    g = torch.Generator().manual_seed(rows + cols + S)
    ldp = cols + 4
    parts = torch.randn(S, rows, ldp, generator=g).to(gpu)
    x = torch.randn(rows, cols, generator=g).to(gpu)
    bias = (torch.randn(cols, generator=g) * 0.1).to(dtype).to(gpu) if with_bias else None
    gamma = (1 + 0.1 * torch.randn(cols, generator=g)).to(dtype).to(gpu)
    beta = (0.1 * torch.randn(cols, generator=g)).to(dtype).to(gpu)
    delta = reduce_in_order(parts[:, :, :cols], bias).to(dtype).contiguous()
    x_ref, y_ref = torch.empty_like(x), torch.empty(rows, cols, dtype=dtype, device=gpu)
    _lib.check(lib.cgpt_add_layernorm(x.data_ptr(), delta.data_ptr(), x_ref.data_ptr(),
                                      gamma.data_ptr(), beta.data_ptr(), y_ref.data_ptr(), rows,
                                      cols, 1e-5, _lib.CGPT_F32, DT[dtype], DT[dtype], DT[dtype],
                                      stream(gpu)), "ln")
    x_out, y = torch.full_like(x, float("nan")), torch.empty(rows, cols, dtype=dtype, device=gpu)
    _lib.check(lib.cgpt_add_layernorm_partials(
        x.data_ptr(), parts.data_ptr(), S, rows * ldp, ldp,
        bias.data_ptr() if with_bias else None, x_out.data_ptr(), gamma.data_ptr(),
        beta.data_ptr(), y.data_ptr(), rows, cols, 1e-5, _lib.CGPT_F32, DT[dtype], DT[dtype],
        DT[dtype], stream(gpu)), "ln partials")
    torch.cuda.synchronize()
    assert torch.equal(x_out, x_ref)
    # Only the statistics' summation order differs (4 waves vs 1 per row).
    tol = 1e-5 if dtype == torch.float32 else 2 ** -7
    e = ((y.float() - y_ref.float()).abs() / (y_ref.float().abs() + 1)).max().item()
    assert e <= tol, e
    # x_out NULL leaves x alone; y unchanged.
    y2 = torch.empty_like(y)
    _lib.check(lib.cgpt_add_layernorm_partials(
        x.data_ptr(), parts.data_ptr(), S, rows * ldp, ldp,
        bias.data_ptr() if with_bias else None, None, gamma.data_ptr(), beta.data_ptr(),
        y2.data_ptr(), rows, cols, 1e-5, _lib.CGPT_F32, DT[dtype], DT[dtype], DT[dtype],
        stream(gpu)), "ln partials")
    torch.cuda.synchronize()
    assert torch.equal(y2, y)


def test_add_layernorm_partials_rejects_bad_args(gpu):
    lib = _lib.load()
    t = torch.zeros(1 << 16, device=gpu)
    p = t.data_ptr()
    ok = dict(n=2, ps=4 * 64, ldp=64)

    def call(n=ok["n"], ps=ok["ps"], ldp=ok["ldp"], parts=p, x_dtype=_lib.CGPT_F32, cols=64):
        return lib.cgpt_add_layernorm_partials(p, parts, n, ps, ldp, None, None, p, p, p, 4, cols,
                                               1e-5, x_dtype, _lib.CGPT_F32, _lib.CGPT_F32,
                                               _lib.CGPT_F32, 0)
    assert call() == 0
    assert call(n=0) == -1 and call(n=17) == -1
    assert call(ldp=62) == -1 and call(ldp=66) == -1
    assert call(ps=100) == -1            # slices overlap the rows
    assert call(parts=p + 4) == -1       # partials not 16-byte aligned
    assert call(x_dtype=_lib.CGPT_BF16) == -2
    assert call(cols=66) == -3


# ------------------------------------------------------------ attention consumer

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("hd,pos,t_max", [(16, 0, 8), (64, 17, 40), (64, 255, 256),
                                          (128, 39, 40), (64, 520, 600)])
@pytest.mark.parametrize("S", [1, 5])
def test_attention_decode_partials_equals_direct(gpu, dtype, hd, pos, t_max, S):
    """Same outputs and cache bit for bit as cgpt_attention_decode fed with
    q / k / v reduced on the host in the same order."""
    lib = _lib.load()
    B, H = 3, 2
    D = H * hd
    g = torch.Generator().manual_seed(hd * 7 + pos + S)
    ldp = 3 * D + 8
    parts = torch.randn(S, B, ldp, generator=g).to(gpu)
    bias = (0.1 * torch.randn(3 * D, generator=g)).to(dtype).to(gpu)
    qkv = reduce_in_order(parts[:, :, :3 * D], bias).to(dtype).contiguous()
    cache_k = torch.randn(B, H, t_max, hd, generator=g).to(dtype)
    cache_v = torch.randn(B, H, t_max, hd, generator=g).to(dtype)
    kc1, vc1 = cache_k.to(gpu), cache_v.to(gpu)
    kc2, vc2 = kc1.clone(), vc1.clone()
    o1 = torch.empty(B, H, hd, dtype=dtype, device=gpu)
    o2 = torch.empty_like(o1)
    err = torch.zeros(2, dtype=torch.int32, device=gpu)
    pdev = torch.tensor([pos - 3], dtype=torch.int32, device=gpu)
    cs = kc1.stride()
    esz = qkv.element_size()
    scale = 1.0 / math.sqrt(hd)
    q0 = qkv.data_ptr()
    _lib.check(lib.cgpt_attention_decode(q0, q0 + D * esz, q0 + 2 * D * esz, kc1.data_ptr(),
                                         vc1.data_ptr(), o1.data_ptr(), B, H, hd, t_max, 3,
                                         pdev.data_ptr(), 3 * D, hd, 3 * D, hd, 3 * D, hd,
                                         cs[0], cs[1], cs[2], H * hd, hd, scale, DT[dtype],
                                         err.data_ptr(), stream(gpu)), "direct")
    _lib.check(lib.cgpt_attention_decode_partials(
        parts.data_ptr(), S, B * ldp, ldp, bias.data_ptr(), 0, D, 2 * D, kc2.data_ptr(),
        vc2.data_ptr(), o2.data_ptr(), B, H, hd, t_max, 3, pdev.data_ptr(), cs[0], cs[1], cs[2],
        H * hd, hd, scale, DT[dtype], err.data_ptr() + 4, stream(gpu)), "partials")
    torch.cuda.synchronize()
    assert err.tolist() == [0, 0]
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert torch.equal(o1, o2)
    # Against the oracle (covers the multi-chunk online softmax at pos >= 256).
    qh = qkv[:, :D].view(B, H, hd).cpu()
    exp_k, exp_v = cache_k.clone(), cache_v.clone()
    exp_k[:, :, pos] = qkv[:, D:2 * D].view(B, H, hd).cpu()
    exp_v[:, :, pos] = qkv[:, 2 * D:].view(B, H, hd).cpu()
    assert torch.equal(kc1.cpu(), exp_k) and torch.equal(vc1.cpu(), exp_v)
    ref = R.causal_attention(qh.double().unsqueeze(2), exp_k[:, :, :pos + 1].double(),
                             exp_v[:, :, :pos + 1].double(),
                             p_dtype=None if dtype == torch.float32 else torch.bfloat16)
    e = (o1.double().cpu() - ref.squeeze(2)).abs().max().item()
    assert e <= (2e-5 if dtype == torch.float32 else 2e-2), e


def test_attention_decode_partials_rejects_bad_args(gpu):
    lib = _lib.load()
    t = torch.zeros(1 << 16, device=gpu)
    p = t.data_ptr()
    B, H, hd, t_max = 2, 2, 64, 8
    D = H * hd

    def call(n=2, ps=2 * 3 * D, ldp=3 * D, v_off=2 * D, bias=p):
        return lib.cgpt_attention_decode_partials(p, n, ps, ldp, bias, 0, D, v_off, p, p, p, B, H,
                                                  hd, t_max, 0, None, H * t_max * hd, t_max * hd,
                                                  hd, D, hd, 0.125, _lib.CGPT_F32, None, 0)
    assert call() == 0
    assert call(n=0) == -1 and call(n=17) == -1
    assert call(ldp=3 * D - 1) == -1       # v block past the row
    assert call(ps=3 * D) == -1            # slices overlap
    assert call(v_off=3 * D) == -1
    assert call(bias=None) == -1


# --------------------------------------------------- bias + activation consumer

def _pba(lib, gpu, parts, S, rows, cols, ldp, bias, out, ldo, epi, out_dtype):
    return lib.cgpt_partials_bias_act(parts.data_ptr(), S, rows * ldp, ldp, bias.data_ptr(),
                                      DT[bias.dtype], out.data_ptr(), ldo, rows, cols, epi,
                                      DT[out_dtype], stream(gpu))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bias_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,cols,S", [(32, 6400, 5), (3, 100, 1), (64, 768, 16), (5, 4096, 9),
                                         (1, 4, 8)])
def test_partials_bias_act_matches_host_reduction(gpu, out_dtype, bias_dtype, rows, cols, S):
    """Bias only: bit-identical to the in-order host sum (fp32 additions are
    exact IEEE operations) rounded once.  GELU: within one rounding (plus the
    fp32 GELU's own error) of the fp64 GELU of that same fp32 sum.  Padding
    of the output rows untouched."""
    lib = _lib.load()
    g = torch.Generator().manual_seed(rows * 7 + cols + S)
    ldp, ldo = cols + 4, cols + 8
    parts = torch.randn(S, rows, ldp, generator=g).to(gpu)
    bias = torch.randn(cols, generator=g).to(bias_dtype).to(gpu)
    t = reduce_in_order(parts[:, :, :cols], bias)  # fp32, P[0] + ... + P[S-1] + bias
    for epi in (_lib.EPI_BIAS, _lib.EPI_BIAS_GELU):
        out = torch.full((rows, ldo), float("nan"), device=gpu).to(out_dtype)
        _lib.check(_pba(lib, gpu, parts, S, rows, cols, ldp, bias, out, ldo, epi, out_dtype), "pba")
        torch.cuda.synchronize()
        assert torch.isnan(out[:, cols:].float()).all()
        got = out[:, :cols]
        if epi == _lib.EPI_BIAS:
            assert torch.equal(got, t.to(out_dtype))
        else:
            ref = R.gelu_tanh(t.double())
            err = (got.double() - ref).abs() / (ref.abs() + 1e-3)
            # bf16: one rounding (half an ulp, 2^-8 relative) over the fp32
            # GELU's few-ulp error (x / (1 + exp2(.)) on the hardware exp2 and
            # reciprocal); fp32: that error alone.
            tol = 2 ** -8 + 4e-6 if out_dtype == torch.bfloat16 else 4e-6
            assert err.max().item() <= tol, err.max().item()


def test_partials_bias_act_agrees_with_gemm_epilogue(gpu):
    """cgpt_gemm_partials + cgpt_partials_bias_act against the skinny GEMM's own
    bias + GELU epilogue on the same operands (fp32 summation order only)."""
    lib = _lib.load()
    M, N, K = 32, 6400, 1600
    g = torch.Generator().manual_seed(5)
    a = torch.randn(M, K, generator=g).bfloat16().to(gpu)
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16().to(gpu)
    b = (torch.randn(N, generator=g) * 0.1).bfloat16().to(gpu)
    S = plan(lib, M, N, K, torch.bfloat16)
    p = torch.empty(S, M, N, device=gpu)
    _lib.check(lib.cgpt_gemm_partials(a.data_ptr(), w.data_ptr(), p.data_ptr(), M, N, K, K, K, N, S,
                                      _lib.CGPT_BF16, stream(gpu)), "partials")
    out = torch.empty(M, N, device=gpu)
    _lib.check(_pba(lib, gpu, p, S, M, N, N, b, out, N, _lib.EPI_BIAS_GELU, torch.float32), "pba")
    ref = torch.empty(M, N, device=gpu)
    _lib.check(lib.cgpt_gemm_skinny(a.data_ptr(), w.data_ptr(), b.data_ptr(), ref.data_ptr(), M, N,
                                    K, K, K, N, _lib.CGPT_BF16, _lib.CGPT_BF16, _lib.CGPT_F32,
                                    _lib.EPI_BIAS_GELU, None, 0, None, 0, stream(gpu)), "skinny")
    torch.cuda.synchronize()
    exact = R.gelu_tanh(a.double() @ w.double().t() + b.double())
    assert (out.double() - exact).abs().max().item() <= 1e-4
    assert (out - ref).abs().max().item() <= 1e-4


def test_partials_bias_act_rejects_bad_args(gpu):
    lib = _lib.load()
    rows, cols, S = 4, 64, 3
    parts = torch.zeros(S, rows, cols, device=gpu)
    bias = torch.zeros(cols, device=gpu)
    out = torch.empty(rows, cols, device=gpu)

    def call(S=S, ps=rows * cols, ldp=cols, b=bias, bdt=_lib.CGPT_F32, o=out.data_ptr(),
             ldo=cols, c=cols, epi=_lib.EPI_BIAS_GELU, odt=_lib.CGPT_F32, p=parts.data_ptr()):
        return lib.cgpt_partials_bias_act(p, S, ps, ldp, None if b is None else b.data_ptr(), bdt,
                                          o, ldo, rows, c, epi, odt, stream(gpu))

    assert call() == 0
    assert call(S=0) == -1 and call(S=17) == -1
    assert call(c=62, ldp=62, ldo=62) == -1       # cols % 4
    assert call(ldp=cols - 4) == -1
    assert call(ps=(rows - 1) * cols) == -1       # slices overlap
    assert call(ldo=cols - 4) == -1
    assert call(b=None) == -1
    assert call(epi=_lib.EPI_NONE) == -1
    assert call(odt=_lib.CGPT_F16) == -2
    assert call(p=parts.data_ptr() + 4) == -1     # partials 16-byte aligned
    assert call(o=out.data_ptr() + 4) == -1       # fp32 output 16-byte aligned
    torch.cuda.synchronize()


# ------------------------------------------------------------------ decode step

def test_decode_partials_matches_fixup_path(gpu):
    """The partial-product step and the in-kernel split-K step give the same
    greedy tokens (fp32) and logits within fp32 summation-order noise."""
    from test_decode_gpu import small_model
    m, _, cfg = small_model(torch.float32, n_layer=2, n_head=4, n_embd=256, seed=21)
    B, T0, n = 6, 11, 9
    idx = torch.randint(0, cfg.vocab_size, (B, T0), generator=torch.Generator().manual_seed(3)).to(gpu)
    runs = []
    for partials in (True, False):
        sess = DecodeSession(m, B, T0, n, partials=partials)
        sess.prefill(idx)
        sess.greedy_first()
        logits = []
        for _ in range(n - 1):
            sess.greedy_step()
            logits.append(sess.logits.clone())
        torch.cuda.synchronize()
        runs.append((sess.hist.clone(), torch.stack(logits)))
    assert torch.equal(runs[0][0], runs[1][0])
    assert (runs[0][1] - runs[1][1]).abs().max().item() <= 1e-4

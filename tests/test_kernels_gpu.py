"""Kernel parity on the GPU: every HIP kernel against the CPU oracle (fp64)
at small and ragged shapes, and at the standalone-kernel benchmark sizes.

Tolerances: fp32 outputs within a few fp32 ulps of the exact result scaled
by the problem (stated per test); bf16 outputs within one bf16 rounding
(relative 2^-8) plus the fp32 accumulation error.
"""

import math

import pytest
import torch

import cutilegpt_amd as cg
from cutilegpt_amd import _lib
from oracle import gpt_ref as R

pytestmark = pytest.mark.gpu

F32, BF16 = torch.float32, torch.bfloat16


def randn(*shape, seed=0, dtype=F32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def close(out, ref, atol, rtol, what=""):
    out = out.detach().cpu().double()
    ref = ref.detach().cpu().double()
    err = (out - ref).abs()
    bound = atol + rtol * ref.abs()
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.numel()} outside tolerance, "
                           f"max err {err.max().item():.3e}")


# --------------------------------------------------------------------- GELU

@pytest.mark.parametrize("dtype", [F32, BF16])
@pytest.mark.parametrize("n", [1, 7, 4099, 8200, (1 << 20) + 24, 32 * 512 * 768])
def test_gelu(gpu, dtype, n):
    x = randn(n, seed=n, dtype=dtype)
    y = cg.cutile_gelu(x.to(gpu))
    ref = R.gelu_tanh(x.double())
    if dtype == F32:
        close(y, ref, 2e-6, 2e-6, "gelu fp32")
    else:
        close(y, ref, 1e-6, 2 ** -8, "gelu bf16")


def test_gelu_3d_shape_and_special_values(gpu):
    x = torch.tensor([0.0, -0.0, 30.0, -30.0, 1e-8, -1e-8, 5.0, -5.0], dtype=F32)
    y = cg.cutile_gelu(x.view(2, 2, 2).to(gpu))
    assert y.shape == (2, 2, 2)
    close(y.view(-1), R.gelu_tanh(x.double()), 1e-7, 1e-6, "gelu special")


# ---------------------------------------------------------------- LayerNorm

@pytest.mark.parametrize("rows,cols", [(1, 4), (5, 48), (2, 512), (37, 768), (9, 1024),
                                       (3, 1600), (6, 1796), (4, 2048), (3, 2052), (7, 4096),
                                       (16384, 768)])
@pytest.mark.parametrize("xd,yd", [(F32, F32), (BF16, BF16), (F32, BF16)])
def test_layer_norm(gpu, rows, cols, xd, yd):
    x = randn(rows, cols, seed=rows + cols, dtype=xd, scale=2.0) + 0.5
    w = (1 + randn(cols, seed=1, scale=0.1)).to(xd)
    b = randn(cols, seed=2, scale=0.1).to(xd)
    y = cg.add_layer_norm(x.to(gpu), None, w.to(gpu), b.to(gpu), out_dtype=yd)
    ref = R.layer_norm(x.double(), w.double(), b.double())
    if yd == F32:
        close(y, ref, 1e-5, 1e-5, "ln fp32")
    else:
        close(y, ref, 1e-5, 2 ** -8 + 1e-5, "ln bf16")


@pytest.mark.parametrize("with_xo", [True, False])
@pytest.mark.parametrize("pd", [F32, BF16])
@pytest.mark.parametrize("offset", [0, 4])
@pytest.mark.parametrize("rows,cols", [(7, 200), (33, 1600), (1, 4096), (5, 768), (2, 8),
                                       (3, 264)])
def test_layer_norm_bf16_params_copy_and_alignment(gpu, pd, offset, rows, cols, with_xo):
    """bf16 rows without a delta, 16-byte aligned or offset by 4 elements (8 bytes,
    the smallest alignment the ABI accepts for bf16): gamma/beta in either type,
    x_out receives x unchanged.  Aligned, bf16 parameters and no x_out take the
    half-wave kernel with 16-byte accesses (odd row counts leave its last wave
    half empty; 200 and 264 columns end mid-chunk)."""
    x = (randn(rows, cols, seed=rows * cols, scale=2.0) + 0.5).to(BF16)
    w = (1 + randn(cols, seed=8, scale=0.1)).to(pd)
    b = randn(cols, seed=9, scale=0.1).to(pd)
    buf = torch.empty(rows * cols + offset, dtype=BF16, device=gpu)
    xg = buf[offset:].view(rows, cols)
    xg.copy_(x.to(gpu))
    xo = torch.empty_like(xg) if with_xo else None
    y = cg.add_layer_norm(xg, None, w.to(gpu), b.to(gpu), out_dtype=BF16, x_out=xo)
    close(y, R.layer_norm(x.double(), w.double(), b.double()), 1e-5, 2 ** -8 + 1e-5, "ln bf16")
    if with_xo:
        assert torch.equal(xo.cpu(), x)


@pytest.mark.parametrize("dd", [F32, BF16])
@pytest.mark.parametrize("rows,cols", [(300, 768), (301, 48), (33, 1600), (5, 4096)])
def test_add_layer_norm_writes_residual(gpu, dd, rows, cols):
    x = randn(rows, cols, seed=3)
    d = randn(rows, cols, seed=4, dtype=dd)
    w, b = randn(cols, seed=5) + 1, randn(cols, seed=6)
    xg = x.to(gpu)
    y = cg.add_layer_norm(xg, d.to(gpu), w.to(gpu), b.to(gpu), out_dtype=BF16, x_out=xg)
    s = x.double() + d.double()
    close(xg, s, 1e-6, 1e-6, "residual")  # x_out == x + delta (in place)
    close(y, R.layer_norm(s, w.double(), b.double()), 1e-5, 2 ** -8 + 1e-5, "add+ln")


def test_layer_norm_constant_rows(gpu):
    x = torch.full((4, 768), 3.5)
    beta = randn(768, seed=7)
    y = cg.cutile_layer_norm(x.to(gpu), torch.ones(768, device=gpu), beta.to(gpu))
    close(y, beta.expand(4, 768), 1e-6, 0, "constant row -> beta")


# --------------------------------------------------------------------- GEMM

GEMM_SHAPES = [(1, 1, 8), (17, 33, 40), (64, 64, 64), (130, 300, 768), (256, 512, 128),
               (77, 50257, 48), (300, 96, 3072)]


def gemm_ref(a, w, b, epi):
    y = a.double() @ w.double().t()
    if b is not None:
        y = y + b.double()
    if epi == _lib.EPI_BIAS_GELU:
        y = R.gelu_tanh(y)
    return y


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
@pytest.mark.parametrize("dtype", [BF16, F32])
@pytest.mark.parametrize("epi", [_lib.EPI_NONE, _lib.EPI_BIAS, _lib.EPI_BIAS_GELU])
def test_gemm_auto_tile(gpu, m, n, k, dtype, epi):
    a = randn(m, k, seed=m, dtype=dtype)
    w = randn(n, k, seed=n, dtype=dtype, scale=0.05)
    b = None if epi == _lib.EPI_NONE else randn(n, seed=k, dtype=dtype)
    out = cg.kernels._gemm(a.to(gpu), w.to(gpu), None if b is None else b.to(gpu), epi, F32, "t")
    ref = gemm_ref(a, w, b, epi)
    # fp32 accumulation of K products of |a w| ~ 0.05: error << 1e-4
    close(out, ref, 1e-4 * math.sqrt(k / 64), 1e-5, f"gemm {dtype} {m}x{n}x{k} epi{epi}")


@pytest.mark.parametrize("m,n,k,epi", [(4096, 1600, 1600, _lib.EPI_BIAS),    # XL prefill proj
                                        (4096, 1600, 6400, _lib.EPI_BIAS),    # XL MLP proj
                                        (4096, 6400, 1600, _lib.EPI_BIAS_GELU),
                                        (2048, 3072, 768, _lib.EPI_BIAS_GELU)])
def test_gemm_auto_tile_persistent_paths(gpu, m, n, k, epi):
    """TILE_AUTO on shapes that take the persistent tiles chosen by the number of
    idle CUs (fewer 256x192 tiles than CUs) or id 16 (GELU epilogue): equal, bit
    for bit, to tile 15 (every bf16 kernel adds the same k32 MFMA products in
    the same order), and close to the fp64 product."""
    a = randn(m, k, seed=m + 1, dtype=BF16)
    w = randn(n, k, seed=n + 1, dtype=BF16, scale=0.05)
    b = randn(n, seed=k + 1, dtype=BF16)
    ag, wg, bg = a.to(gpu), w.to(gpu), b.to(gpu)
    out = cg.kernels._gemm(ag, wg, bg, epi, BF16, "t", tile=_lib.TILE_AUTO)
    ref = gemm_ref(a, w, b, epi)
    close(out, ref, 1e-3 * math.sqrt(k / 64), 2 ** -8, f"auto {m}x{n}x{k}")
    alt = cg.kernels._gemm(ag, wg, bg, epi, BF16, "t", tile=15)
    assert torch.equal(out, alt)


@pytest.mark.parametrize("tile", range(5))
@pytest.mark.parametrize("m,n,k", [(300, 520, 136), (512, 256, 768), (1, 50257, 64)])
def test_gemm_every_bf16_tile(gpu, tile, m, n, k):
    a = randn(m, k, seed=1, dtype=BF16)
    w = randn(n, k, seed=2, dtype=BF16, scale=0.05)
    b = randn(n, seed=3, dtype=BF16)
    out = cg.kernels._gemm(a.to(gpu), w.to(gpu), b.to(gpu), _lib.EPI_BIAS, BF16, "t", tile=tile)
    close(out, gemm_ref(a, w, b, _lib.EPI_BIAS), 1e-3, 2 ** -8, f"tile {tile}")


DMA_TILES = [5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19]


@pytest.mark.parametrize("tile", DMA_TILES)
@pytest.mark.parametrize("m,n,k", [(300, 520, 192), (512, 256, 768), (1, 50257, 64),
                                   (257, 129, 128), (1000, 3072, 1600)])
@pytest.mark.parametrize("epi", [_lib.EPI_NONE, _lib.EPI_BIAS_GELU])
def test_gemm_dma_tiles(gpu, tile, m, n, k, epi):
    """Direct-to-LDS pipeline (K % 64 == 0): ragged M/N edges, 1..25 K steps."""
    a = randn(m, k, seed=11, dtype=BF16)
    w = randn(n, k, seed=12, dtype=BF16, scale=0.05)
    b = randn(n, seed=13, dtype=BF16)
    out = cg.kernels._gemm(a.to(gpu), w.to(gpu), b.to(gpu), epi, F32, "t", tile=tile)
    ref = gemm_ref(a, w, None if epi == _lib.EPI_NONE else b, epi)
    close(out, ref, 1e-4 * math.sqrt(k / 64), 1e-5, f"dma tile {tile} {m}x{n}x{k}")


PERSIST_TILES = [5, 7, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19]


@pytest.mark.parametrize("tile", PERSIST_TILES)
@pytest.mark.parametrize("m,n,k", [(300, 520, 128), (4096, 4096, 256), (257, 50257, 192),
                                   (16384, 768, 3072), (1, 3, 128), (1000, 1000, 64),
                                   (2000, 50304, 64)])
@pytest.mark.parametrize("epi", [_lib.EPI_BIAS, _lib.EPI_BIAS_GELU])
@pytest.mark.parametrize("dtype", [BF16, torch.float16])
def test_gemm_persistent_tiles(gpu, tile, m, n, k, epi, dtype):
    """Persistent kernel: several tiles per block (tile boundaries inside the
    flattened K stream), fewer tiles than CUs, ragged edges; bf16 and fp16
    inputs (the fp16 MFMA and fp16 bias / outputs)."""
    a = randn(m, k, seed=21, dtype=dtype)
    w = randn(n, k, seed=22, dtype=dtype, scale=0.05)
    b = randn(n, seed=23, dtype=dtype)
    out = cg.kernels._gemm(a.to(gpu), w.to(gpu), b.to(gpu), epi, dtype, "t", tile=tile)
    ref = gemm_ref(a, w, b, epi)
    close(out, ref, 2e-3, 2 ** -8 if dtype == BF16 else 2 ** -10,
          f"persistent tile {tile} {m}x{n}x{k} {dtype}")


@pytest.mark.parametrize("tile", [14, 15, 16])
@pytest.mark.parametrize("ldc_pad,c_off,out_dtype", [(0, 0, BF16), (8, 0, BF16), (4, 4, BF16),
                                                      (0, 0, F32), (4, 0, F32), (0, 2, F32)])
def test_gemm_staged_output_layouts(gpu, tile, ldc_pad, c_off, out_dtype):
    """Staged whole-line stores (tiles 14, 15) with padded output rows and a C pointer that
    is only 8/4-byte aligned: the aligned cases take the staged path, the others fall back
    to per-group buffer stores; every element outside the N columns keeps its old value."""
    m, n, k = 300, 520, 192
    a = randn(m, k, seed=31, dtype=BF16).to(gpu)
    w = randn(n, k, seed=32, dtype=BF16, scale=0.05).to(gpu)
    b = randn(n, seed=33, dtype=BF16).to(gpu)
    ldc = n + ldc_pad
    buf = torch.full((m * ldc + c_off + 8,), 7.0, device=gpu, dtype=out_dtype)
    c = buf[c_off:]
    lib = _lib.load()
    odt = _lib.CGPT_BF16 if out_dtype == BF16 else _lib.CGPT_F32
    _lib.check(lib.cgpt_gemm(a.data_ptr(), w.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, k, k,
                             ldc, _lib.CGPT_BF16, _lib.CGPT_BF16, odt, _lib.EPI_BIAS_GELU, tile,
                             torch.cuda.current_stream().cuda_stream), "staged")
    out = c[:m * ldc].view(m, ldc)
    ref = gemm_ref(a.cpu(), w.cpu(), b.cpu(), _lib.EPI_BIAS_GELU)
    tol = (2e-3, 2 ** -8) if out_dtype == BF16 else (1e-4, 1e-5)
    close(out[:, :n], ref, *tol, f"staged tile {tile} ldc {ldc} off {c_off}")
    assert torch.all(out[:, n:] == 7.0)
    assert torch.all(buf[:c_off] == 7.0) and torch.all(buf[c_off + m * ldc:] == 7.0)


def test_gemm_pipe_rejects_ragged_k(gpu):
    a = randn(64, 72, dtype=BF16).to(gpu)
    w = randn(64, 72, dtype=BF16).to(gpu)
    with pytest.raises(ValueError):
        cg.kernels._gemm(a, w, None, _lib.EPI_NONE, F32, "t", tile=5)
    a = randn(64, 96, dtype=BF16).to(gpu)  # K % 64 != 0 but K % 32 == 0: only SPS 1 tiles
    w = randn(64, 96, dtype=BF16).to(gpu)
    with pytest.raises(ValueError):
        cg.kernels._gemm(a, w, None, _lib.EPI_NONE, F32, "t", tile=5)
    out = cg.kernels._gemm(a, w, None, _lib.EPI_NONE, F32, "t", tile=6)
    close(out, gemm_ref(a.cpu(), w.cpu(), None, 0), 1e-3, 1e-4, "K=96 on a single-slab tile")


@pytest.mark.parametrize("tile", range(2))
def test_gemm_every_f32_tile(gpu, tile):
    a, w = randn(200, 100, seed=4), randn(333, 100, seed=5, scale=0.1)
    out = cg.kernels._gemm(a.to(gpu), w.to(gpu), None, _lib.EPI_NONE, F32, "t", tile=tile)
    close(out, gemm_ref(a, w, None, 0), 1e-5, 1e-5, f"f32 tile {tile}")


def test_gemm_strided_output_and_lda(gpu):
    """Row-padded A (lda > K) and C written into a wider buffer (ldc > N)."""
    lib = _lib.load()
    m, n, k = 70, 90, 64
    abig = randn(m, 80, seed=8, dtype=BF16).to(gpu)
    w = randn(n, k, seed=9, dtype=BF16, scale=0.1).to(gpu)
    c = torch.full((m, 100), 7.0, device=gpu)
    _lib.check(lib.cgpt_gemm(abig.data_ptr(), w.data_ptr(), None, c.data_ptr(), m, n, k, 80, k,
                             100, 1, 0, 0, 0, -1, torch.cuda.current_stream().cuda_stream), "g")
    close(c[:, :n], gemm_ref(abig[:, :k].cpu(), w.cpu(), None, 0), 1e-4, 1e-5, "strided")
    assert torch.all(c[:, n:] == 7.0)


@pytest.mark.parametrize("n,k", [(2304, 768), (768, 768), (3072, 768), (768, 3072), (50257, 768)])
def test_gemm_gpt2_shapes_vs_torch(gpu, n, k):
    """Full GPT-2 prefill shapes (M = 16384) against torch's fp32 matmul of the
    same bf16 operands."""
    m = 16384
    g = torch.Generator(device=gpu).manual_seed(n + k)
    a = torch.randn(m, k, device=gpu, generator=g).to(BF16)
    w = (torch.randn(n, k, device=gpu, generator=g) * 0.02).to(BF16)
    b = torch.randn(n, device=gpu, generator=g).to(BF16)
    out = cg.kernels._gemm(a, w, b, _lib.EPI_BIAS, F32, "t")
    ref = torch.addmm(b.float(), a.float(), w.float().t())
    err = (out - ref).abs().max().item()
    assert err < 2e-4 * math.sqrt(k / 64), err


@pytest.mark.parametrize("tile", [14, 16])
def test_gemm_weight_prefetch_strided_w(gpu, tile):
    """A persistent launch over a weight matrix past the prefetch threshold
    (>= 32 MiB, M >= 1024), with W rows padded (ldw > K): the read ahead of the
    GEMM covers exactly W's extent and the product is unchanged (against
    torch's fp32 matmul of the same bf16 operands)."""
    m, n, k, ldw = 1024, 21000, 768, 832
    g = torch.Generator(device=gpu).manual_seed(5)
    a = torch.randn(m, k, device=gpu, generator=g).to(BF16)
    wbig = (torch.randn(n, ldw, device=gpu, generator=g) * 0.02).to(BF16)
    w = wbig[:, :k]
    assert ((n - 1) * ldw + k) * 2 >= 32 << 20
    out = cg.kernels._gemm(a, w, None, _lib.EPI_NONE, F32, "t", tile=tile)
    ref = a.float() @ w.float().t()
    err = (out - ref).abs().max().item()
    assert err < 2e-4 * math.sqrt(k / 64), err


# ---------------------------------------------------------------- Attention

ATTN_SHAPES = [(1, 1, 1, 64), (1, 2, 5, 16), (2, 3, 17, 32), (1, 1, 130, 64), (2, 4, 64, 64),
               (1, 2, 300, 128), (1, 3, 64, 16)]


def attn_ref(q, k, v, dtype):
    return R.causal_attention(q.double(), k.double(), v.double(),
                              p_dtype=torch.bfloat16 if dtype == BF16 else None)


@pytest.mark.parametrize("shape", ATTN_SHAPES)
@pytest.mark.parametrize("dtype", [BF16, F32])
def test_attention(gpu, shape, dtype):
    q, k, v = (randn(*shape, seed=i, dtype=dtype) for i in range(3))
    o = cg.cutile_causal_attention(q.to(gpu), k.to(gpu), v.to(gpu), shape[1])
    ref = attn_ref(q, k, v, dtype)
    if dtype == F32:
        close(o, ref, 2e-5, 2e-5, f"attn fp32 {shape}")
    else:
        close(o, ref, 4e-3, 2 ** -8, f"attn bf16 {shape}")


@pytest.mark.parametrize("dtype", [BF16, F32])
def test_attention_standalone_config(gpu, dtype):
    """BASELINE standalone config: B=8, H=12, T=512, hd=64, causal."""
    shape = (8, 12, 512, 64)
    q, k, v = (randn(*shape, seed=10 + i, dtype=dtype) for i in range(3))
    o = cg.cutile_causal_attention(q.to(gpu), k.to(gpu), v.to(gpu), 12)
    ref = attn_ref(q, k, v, dtype)
    tol = (2e-5, 2e-5) if dtype == F32 else (4e-3, 2 ** -8)
    close(o, ref, *tol, f"attn standalone {dtype}")


def _attn_raw(q, k, v, causal, scale=None):
    """cgpt_attention_fwd on contiguous (B, H, T, hd) tensors, Tq = q rows, Tk = k rows."""
    B, H, Tq, hd = q.shape
    Tk = k.shape[2]
    o = torch.empty_like(q)
    lib = _lib.load()
    code = {F32: _lib.CGPT_F32, BF16: _lib.CGPT_BF16}[q.dtype]
    st = lambda t: t.stride()[:3]
    _lib.check(lib.cgpt_attention_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H,
                                      Tq, Tk, hd, *st(q), *st(k), *st(v), *st(o),
                                      1.0 / math.sqrt(hd) if scale is None else scale, int(causal),
                                      code, torch.cuda.current_stream().cuda_stream), "attention")
    return o


@pytest.mark.parametrize("dtype", [BF16, F32])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,H,Tq,Tk,hd", [(1, 2, 1, 77, 64), (2, 3, 40, 200, 64),
                                          (1, 2, 130, 130, 64), (2, 2, 65, 300, 128),
                                          (1, 3, 17, 50, 32), (2, 1, 9, 9, 16),
                                          (1, 2, 256, 512, 64)])
def test_attention_tq_tk_and_non_causal(gpu, dtype, causal, B, H, Tq, Tk, hd):
    """Query offset (Tk > Tq: query i at absolute position Tk - Tq + i) and the
    unmasked case, in both kernels (bf16 hd 64/128 take the DMA kernel)."""
    q = randn(B, H, Tq, hd, seed=31, dtype=dtype)
    k, v = (randn(B, H, Tk, hd, seed=32 + i, dtype=dtype) for i in range(2))
    o = _attn_raw(q.to(gpu), k.to(gpu), v.to(gpu), causal).cpu()
    ref = R.causal_attention(q.double(), k.double(), v.double(),
                             p_dtype=torch.bfloat16 if dtype == BF16 else None, causal=causal)
    tol = (2e-5, 2e-5) if dtype == F32 else (4e-3, 2 ** -8)
    close(o, ref, *tol, f"attn Tq={Tq} Tk={Tk} causal={causal}")


def test_attention_qkv_rejects_bad_arguments(gpu):
    x = torch.zeros(2, 8, 3 * 64, dtype=BF16, device=gpu)
    with pytest.raises(ValueError):
        cg.attention_qkv(x, 3)  # D = 64 not divisible by 3 heads
    with pytest.raises(ValueError):
        cg.attention_qkv(torch.zeros(2, 8, 100, dtype=BF16, device=gpu), 2)  # 3D not a multiple of 3
    with pytest.raises(ValueError):
        cg.attention_qkv(x, 2, out=torch.empty(2, 8, 32, dtype=BF16, device=gpu))  # wrong shape
    with pytest.raises(ValueError):
        cg.attention_qkv(x, 2, out=torch.empty(2, 8, 64, dtype=F32, device=gpu))  # wrong dtype
    with pytest.raises(ValueError):
        cg.attention_qkv(x, 2, out=torch.empty(2, 64, 8, dtype=BF16, device=gpu).transpose(1, 2))
    with pytest.raises(ValueError):
        cg.attention_qkv(x.cpu(), 2)
    with pytest.raises(ValueError):
        cg.attention_qkv(x.double(), 2)  # float64 is not a kernel dtype


def test_attention_qkv_strided_view(gpu):
    """A view of the first T2 positions of a longer buffer keeps its parent's
    batch stride: the kernel must read it through qkv.stride(), not T2 * 3D."""
    B, T, H, hd, T2 = 2, 96, 2, 64, 40
    D = H * hd
    full = randn(B, T, 3 * D, seed=41, dtype=BF16)
    view = full.to(gpu)[:, :T2]
    o = cg.attention_qkv(view, H).cpu()
    q, k, v = (t.reshape(B, T2, H, hd).transpose(1, 2) for t in full[:, :T2].split(D, dim=2))
    ref = attn_ref(q, k, v, BF16).transpose(1, 2).reshape(B, T2, D)
    close(o, ref, 4e-3, 2 ** -8, "qkv strided view")


def test_attention_row0_and_equal_keys(gpu):
    shape = (1, 2, 40, 64)
    q, k, v = (randn(*shape, seed=20 + i) for i in range(3))
    o = cg.cutile_causal_attention(q.to(gpu), k.to(gpu), v.to(gpu), 2).cpu()
    assert torch.equal(o[:, :, 0], v[:, :, 0])  # P = exp2(0) = 1 exactly
    keq = k[:, :, :1].expand(shape).contiguous()
    o2 = cg.cutile_causal_attention(q.to(gpu), keq.to(gpu), v.to(gpu), 2).cpu()
    prefix = v.double().cumsum(2) / torch.arange(1, 41, dtype=torch.float64).view(1, 1, 40, 1)
    close(o2, prefix, 1e-5, 1e-5, "equal keys -> prefix mean")


@pytest.mark.parametrize("dtype", [BF16, F32])
@pytest.mark.parametrize("B,T,H,hd", [(2, 100, 3, 16), (2, 256, 12, 64), (1, 1024, 25, 64)])
def test_attention_qkv_layout(gpu, dtype, B, T, H, hd):
    """Strided reads from the fused (B, T, 3D) projection, (B, T, D) output."""
    D = H * hd
    qkv = randn(B, T, 3 * D, seed=T, dtype=dtype)
    o = cg.attention_qkv(qkv.to(gpu), H).cpu()
    q, k, v = (t.reshape(B, T, H, hd).transpose(1, 2) for t in qkv.split(D, dim=2))
    ref = attn_ref(q, k, v, dtype).transpose(1, 2).reshape(B, T, D)
    tol = (2e-5, 2e-5) if dtype == F32 else (4e-3, 2 ** -8)
    close(o, ref, *tol, "qkv layout")


# ---------------------------------------------------------------- Embedding

@pytest.mark.parametrize("wd,od", [(F32, F32), (BF16, F32), (BF16, BF16)])
def test_token_pos_embedding_exact(gpu, wd, od):
    V, BS, D = 50257, 1024, 768
    wte, wpe = randn(V, D, seed=1, dtype=wd), randn(BS, D, seed=2, dtype=wd)
    idx = torch.randint(0, V, (3, 77), generator=torch.Generator().manual_seed(3))
    out = cg.token_pos_embedding(idx.to(gpu), wte.to(gpu), wpe.to(gpu), pos0=5, out_dtype=od).cpu()
    ref = (wte.float()[idx] + wpe.float()[5:82].unsqueeze(0)).to(od)
    assert torch.equal(out, ref)


def test_embedding_gather_and_range_check(gpu):
    w = randn(100, 48, seed=4)
    idx = torch.tensor([[0, 99, 5], [7, 7, 1]])
    out = cg.cutile_embedding(idx.to(gpu), w.to(gpu)).cpu()
    assert torch.equal(out, w[idx])
    with pytest.raises(IndexError):  # clamped in the kernel, reported on the host
        cg.cutile_embedding(torch.tensor([3, 100]).to(gpu), w.to(gpu))


@pytest.mark.parametrize("wd,yd", [(F32, F32), (BF16, BF16), (BF16, F32)])
@pytest.mark.parametrize("D", [48, 768, 1600, 2052])
def test_embedding_layernorm_equals_embedding_then_ln(gpu, wd, yd, D):
    """cgpt_embedding_layernorm == cgpt_embedding (fp32 out) then LayerNorm, bit for bit,
    and within LayerNorm tolerance of the fp64 oracle."""
    V, P, B, T = 1000, 64, 3, 21
    wte, wpe = randn(V, D, seed=11, dtype=wd), randn(P, D, seed=12, dtype=wd)
    g = (1 + randn(D, seed=13, scale=0.1)).to(wd)
    b = randn(D, seed=14, scale=0.1).to(wd)
    idx = torch.randint(0, V, (B, T), generator=torch.Generator().manual_seed(15))
    dg = [t.to(gpu) for t in (wte, wpe, g, b, idx)]
    x2 = cg.token_pos_embedding(dg[4], dg[0], dg[1], pos0=7, out_dtype=F32)
    y2 = cg.add_layer_norm(x2, None, dg[2], dg[3], out_dtype=yd)
    x1 = torch.empty(B * T, D, device=gpu)
    y1 = torch.empty(B * T, D, dtype=yd, device=gpu)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    lib = _lib.load()
    code = {F32: _lib.CGPT_F32, BF16: _lib.CGPT_BF16}
    _lib.check(lib.cgpt_embedding_layernorm(
        dg[4].data_ptr(), dg[0].data_ptr(), dg[1].data_ptr(), None, x1.data_ptr(), dg[2].data_ptr(),
        dg[3].data_ptr(), y1.data_ptr(), B * T, T, D, V, 7, P, 1e-5, code[wd], code[yd],
        err.data_ptr(), torch.cuda.current_stream().cuda_stream), "embedding_layernorm")
    torch.cuda.synchronize()
    assert err.item() == 0
    assert torch.equal(x1.view(B, T, D), x2.view(B, T, D))
    assert torch.equal(y1.view(B, T, D), y2.view(B, T, D))
    xr = wte.double()[idx] + wpe.double()[7:7 + T].unsqueeze(0)
    ref = R.layer_norm(xr, g.double(), b.double())
    close(y1.view(B, T, D), ref, 1e-5, 1e-5 if yd == F32 else 2 ** -8 + 1e-5, "emb+ln")


def test_embedding_layernorm_device_position_and_clamp(gpu):
    """Decode form: the position comes from device memory; out-of-range ids are
    clamped and flagged."""
    V, P, D = 97, 32, 64
    wte, wpe = randn(V, D, seed=21, dtype=BF16).to(gpu), randn(P, D, seed=22, dtype=BF16).to(gpu)
    g = torch.ones(D, dtype=BF16, device=gpu)
    b = torch.zeros(D, dtype=BF16, device=gpu)
    idx = torch.tensor([3, 96, 0, 500], dtype=torch.int64, device=gpu)
    pdev = torch.tensor([6], dtype=torch.int32, device=gpu)
    x = torch.empty(4, D, device=gpu)
    y = torch.empty(4, D, dtype=BF16, device=gpu)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    lib = _lib.load()
    _lib.check(lib.cgpt_embedding_layernorm(
        idx.data_ptr(), wte.data_ptr(), wpe.data_ptr(), pdev.data_ptr(), x.data_ptr(), g.data_ptr(),
        b.data_ptr(), y.data_ptr(), 4, 1, D, V, 10, P, 1e-5, _lib.CGPT_BF16, _lib.CGPT_BF16,
        err.data_ptr(), torch.cuda.current_stream().cuda_stream), "embedding_layernorm")
    torch.cuda.synchronize()
    ids = torch.tensor([3, 96, 0, V - 1], device=gpu)
    assert torch.equal(x, wte[ids].float() + wpe[16].float())
    assert err.item() == 1
    close(y, R.layer_norm(x.double().cpu(), g.double().cpu(), b.double().cpu()), 1e-5,
          2 ** -8 + 1e-5, "emb+ln decode")


# ------------------------------------------------------ residual epilogue

def _resid_gemm(a, w, b, c, tile=_lib.TILE_AUTO):
    """c += a @ w.T + b through cgpt_gemm's residual epilogue (in place)."""
    lib = _lib.load()
    code = {F32: _lib.CGPT_F32, BF16: _lib.CGPT_BF16}
    m, k = a.shape
    n = w.shape[0]
    _lib.check(lib.cgpt_gemm(a.data_ptr(), w.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k,
                             a.stride(0), w.stride(0), c.stride(0), code[a.dtype], code[b.dtype],
                             code[c.dtype], _lib.EPI_BIAS_RESID, tile,
                             torch.cuda.current_stream().cuda_stream), "resid")


@pytest.mark.parametrize("m,n,k", [(16384, 768, 768), (16384, 768, 3072), (4096, 512, 2048),
                                   (4096, 1600, 1600), (300, 520, 512), (257, 192, 1024), (256, 384, 1536), (600, 200, 768),
                                   (1000, 200, 640), (513, 768, 4096)])
def test_gemm_residual_epilogue_slab(gpu, m, n, k):
    """C += A W^T + bias in place (bf16 A, W; fp32 C), the slab kernel's residual
    ring (tile 14) where K gives it 8 k64 steps: against the fp64 sum; ragged M,
    N and several tiles per block included."""
    g = torch.Generator(device=gpu).manual_seed(m + n + k)
    a = torch.randn(m, k, device=gpu, generator=g).to(BF16)
    w = (torch.randn(n, k, device=gpu, generator=g) * 0.05).to(BF16)
    b = torch.randn(n, device=gpu, generator=g).to(BF16)
    x = torch.randn(m, n, device=gpu, generator=g) * 4
    ref = x.double() + a.double() @ w.double().t() + b.double()
    c = x.clone()
    _resid_gemm(a, w, b, c, tile=14)
    err = (c.double() - ref).abs().max().item()
    assert err <= 2e-4 * math.sqrt(k / 64), err


@pytest.mark.parametrize("tile", [14, _lib.TILE_AUTO])
@pytest.mark.parametrize("m,n,k", [(32768, 768, 768), (16384, 1536, 768), (8192, 2304, 512)])
def test_gemm_residual_epilogue_slab_multi_tile(gpu, tile, m, n, k):
    """The slab kernel's residual ring when a persistent block walks two tiles
    (512 / 512 / 384 tiles of 256x192 for 256 CUs): the first two C row blocks
    of a block's next tile are fetched into its LDS ring during the current
    tile's last two K steps, with the current tile's stores still in flight;
    K = 512 gives exactly 8 k64 steps, one per ring row.  TILE_AUTO takes the
    slab kernel here too (at least one tile per CU).  Against the fp64 sum."""
    g = torch.Generator(device=gpu).manual_seed(m + 5 * n + k + tile)
    a = torch.randn(m, k, device=gpu, generator=g).to(BF16)
    w = (torch.randn(n, k, device=gpu, generator=g) * 0.05).to(BF16)
    b = torch.randn(n, device=gpu, generator=g).to(BF16)
    x = torch.randn(m, n, device=gpu, generator=g) * 4
    ref = x.double() + a.double() @ w.double().t() + b.double()
    c = x.clone()
    _resid_gemm(a, w, b, c, tile=tile)
    err = (c.double() - ref).abs().max().item()
    assert err <= 2e-4 * math.sqrt(k / 64), err


@pytest.mark.parametrize("dt,tiles", [(F32, [14, 17, 19, 5, 2, -5, 99]),
                                      (BF16, [5, 16, -7, 99])])
def test_gemm_residual_unknown_tile_ids_mean_auto(gpu, dt, tiles):
    """With the residual epilogue a tile id the dtype does not take (fp32 with a
    bf16-only id, a persistent non-residual id, a negative id other than AUTO /
    SKINNY, an id past the tables) runs as TILE_AUTO: status OK and the
    TILE_AUTO result bit for bit."""
    m, n, k = 520, 264, 512
    a = randn(m, k, seed=61, dtype=dt).to(gpu)
    w = randn(n, k, seed=62, dtype=dt, scale=0.05).to(gpu)
    b = randn(n, seed=63, dtype=dt).to(gpu)
    x = randn(m, n, seed=64, scale=3.0).to(gpu)
    ref = x.clone()
    _resid_gemm(a, w, b, ref, tile=_lib.TILE_AUTO)
    for t in tiles:
        c = x.clone()
        _resid_gemm(a, w, b, c, tile=t)
        assert torch.equal(c, ref), t
    # Without the residual epilogue such ids are still rejected.
    lib = _lib.load()
    code = {F32: _lib.CGPT_F32, BF16: _lib.CGPT_BF16}[dt]
    out = torch.empty(m, n, device=gpu)
    assert lib.cgpt_gemm(a.data_ptr(), w.data_ptr(), b.data_ptr(), out.data_ptr(), m, n, k, k, k,
                         n, code, code, _lib.CGPT_F32, _lib.EPI_BIAS, 99, None) == -1


@pytest.mark.parametrize("tile", [_lib.TILE_AUTO, 0, 1, 2, 3, 4, 9])
@pytest.mark.parametrize("m,n,k", [(4096, 512, 2048), (300, 520, 512), (513, 200, 640)])
def test_gemm_residual_epilogue_tiles(gpu, tile, m, n, k):
    """The residual epilogue on every register-staged tile a planner may ask for
    (and TILE_AUTO, which takes the 128x64 pipeline tile when 256x192 slab
    tiles would leave most CUs idle; a persistent tile id other than 14 and
    17-19 means TILE_AUTO): C = C + A W^T + bias against the fp64 sum."""
    g = torch.Generator(device=gpu).manual_seed(m + 7 * n + k + tile)
    a = torch.randn(m, k, device=gpu, generator=g).to(BF16)
    w = (torch.randn(n, k, device=gpu, generator=g) * 0.05).to(BF16)
    b = torch.randn(n, device=gpu, generator=g).to(BF16)
    x = torch.randn(m, n, device=gpu, generator=g) * 4
    ref = x.double() + a.double() @ w.double().t() + b.double()
    c = x.clone()
    _resid_gemm(a, w, b, c, tile=tile)
    err = (c.double() - ref).abs().max().item()
    assert err <= 2e-4 * math.sqrt(k / 64), err


@pytest.mark.parametrize("tile", [17, 18, 19])
@pytest.mark.parametrize("m,n,k,ct", [(4096, 512, 2048, F32), (4096, 1600, 1600, F32),
                                      (8192, 1600, 768, F32),
                                      (300, 520, 512, F32), (513, 200, 640, F32),
                                      (1000, 96, 128, BF16), (130, 102, 64, F32)])
def test_gemm_residual_epilogue_small_pipeline_tiles(gpu, tile, m, n, k, ct):
    """The residual epilogue on the 4-wave persistent pipeline tiles (the old C
    values of a tile loaded before its stores; N % 4 != 0 takes per-element
    stores): against the fp64 sum.  These kernels launch two or three blocks a
    CU; 8192 x 1600 gives every tile size more tiles than such a grid, so
    blocks walk one or two (128x128) up to five (64x64) tiles."""
    g = torch.Generator(device=gpu).manual_seed(m + 3 * n + k + tile)
    a = torch.randn(m, k, device=gpu, generator=g).to(BF16)
    w = (torch.randn(n, k, device=gpu, generator=g) * 0.05).to(BF16)
    b = torch.randn(n, device=gpu, generator=g).to(BF16)
    x = (torch.randn(m, n, device=gpu, generator=g) * 4).to(ct)
    ref = x.double() + a.double() @ w.double().t() + b.double()
    c = x.clone()
    _resid_gemm(a, w, b, c, tile=tile)
    tol = (2e-4 * math.sqrt(k / 64), 1e-6) if ct == F32 else (4e-3, 2 ** -8)
    close(c, ref, *tol, f"resid tile {tile} {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k,dt,ct", [(77, 130, 96, BF16, F32), (300, 96, 200, BF16, BF16),
                                         (129, 64, 64, F32, F32), (64, 100, 1024, BF16, F32),
                                         (16, 768, 768, BF16, F32), (5, 20, 40, F32, BF16)])
def test_gemm_residual_epilogue_fallback(gpu, m, n, k, dt, ct):
    """Shapes and types outside the residual ring (K below 512 or not a
    multiple of 64, N not a multiple of 4, bf16 C, fp32 inputs, M <= 64) take
    the register-staged kernel: C = C + A W^T + bias all the same."""
    a = randn(m, k, seed=51, dtype=dt).to(gpu)
    w = randn(n, k, seed=52, dtype=dt, scale=0.05).to(gpu)
    b = randn(n, seed=53, dtype=dt).to(gpu)
    x = randn(m, n, seed=54, scale=3.0).to(ct).to(gpu)
    ref = x.double() + a.double() @ w.double().t() + b.double()
    c = x.clone()
    _resid_gemm(a, w, b, c)
    tol = (2e-4, 1e-6) if ct == F32 else (4e-3, 2 ** -8)
    close(c, ref, *tol, f"resid fallback {m}x{n}x{k}")


def test_gemm_residual_epilogue_rejects_skinny(gpu):
    lib = _lib.load()
    x = torch.zeros(64, 64, device=gpu)
    h = torch.zeros(64, 64, dtype=BF16, device=gpu)
    p = h.data_ptr()
    # explicit skinny tile / skinny entry points do not take the residual epilogue
    assert lib.cgpt_gemm(p, p, p, x.data_ptr(), 8, 64, 64, 64, 64, 64, 1, 1, 0, 3,
                         _lib.TILE_SKINNY, None) == -1
    assert lib.cgpt_gemm_skinny(p, p, p, x.data_ptr(), 8, 64, 64, 64, 64, 64, 1, 1, 0, 3, None, 0,
                                None, 0, None) == -1
    # the residual epilogue needs a bias
    assert lib.cgpt_gemm(p, p, None, x.data_ptr(), 8, 64, 64, 64, 64, 64, 1, 1, 0, 3, -1,
                         None) == -1

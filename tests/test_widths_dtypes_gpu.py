"""The drop-in wrappers at the shapes and dtypes the reference's wrappers take
beyond the GPT-2 family: float16 inputs (``cutile_gpt/kernels/linear.py:148-152,
208-212`` give fp16 its own tiles), LayerNorm rows of any width
(``kernels/layernorm.py:104-131`` pads to a power of two), embeddings of any
width (``kernels/embedding.py:73-80``), GEMMs with any K, and head_dim values
the attention kernels are not built for.  Each against the fp64 oracle on the
same (rounded) inputs.

Tolerances: fp32 outputs within a few fp32 ulps scaled by the problem; fp16
outputs within one fp16 rounding (relative 2^-11) plus the fp32 accumulation
error; bf16 outputs within one bf16 rounding (2^-8).
"""

import math

import pytest
import torch

import cutilegpt_amd as cg
from cutilegpt_amd import _lib
from oracle import gpt_ref as R

pytestmark = pytest.mark.gpu

F32, BF16, F16 = torch.float32, torch.bfloat16, torch.float16
REL = {F32: 1e-6, BF16: 2 ** -8, F16: 2 ** -11}


def randn(*shape, seed=0, dtype=F32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def close(out, ref, atol, rtol, what=""):
    out = out.detach().cpu().double()
    ref = ref.detach().cpu().double()
    err = (out - ref).abs()
    bad = err > atol + rtol * ref.abs()
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.numel()} outside tolerance, "
                           f"max err {err.max().item():.3e}")


def gemm_ref(a, w, b, epi, c0=None):
    y = a.double() @ w.double().T
    if epi != _lib.EPI_NONE:
        y = y + b.double()
    if epi == _lib.EPI_BIAS_GELU:
        y = R.gelu_tanh(y)
    if epi == _lib.EPI_BIAS_RESID:
        y = y + c0.double()
    return y


def unaligned(t, gpu):
    """A copy of t on the GPU whose data pointer is one element past a 16-byte
    boundary (a view into a larger buffer)."""
    buf = torch.empty(t.numel() + 16, dtype=t.dtype, device=gpu)
    off = 1 if buf.data_ptr() % 16 == 0 else 0
    v = buf[off:off + t.numel()].view(t.shape)
    v.copy_(t.to(gpu))
    assert v.data_ptr() % 16 != 0
    return v


def gemm_raw(a, w, b, c, epi, in_code, bias_code, out_code, tile=_lib.TILE_AUTO):
    """cgpt_gemm through the C ABI on (already placed) GPU tensors."""
    lib = _lib.load()
    m, k = a.shape
    n = w.shape[0]
    st = lib.cgpt_gemm(a.data_ptr(), w.data_ptr(), None if b is None else b.data_ptr(),
                       c.data_ptr(), m, n, k, a.stride(0), w.stride(0), c.stride(0), in_code,
                       bias_code, out_code, epi, tile, torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "gemm")


CODE = {F32: _lib.CGPT_F32, BF16: _lib.CGPT_BF16, F16: _lib.CGPT_F16}


# -------------------------------------------------------------------- fp16

@pytest.mark.parametrize("m,n,k", [(1, 3, 8), (33, 70, 136), (300, 520, 768), (2048, 768, 3072),
                                   (64, 50257, 64)])
@pytest.mark.parametrize("epi", [_lib.EPI_NONE, _lib.EPI_BIAS, _lib.EPI_BIAS_GELU])
@pytest.mark.parametrize("out_dtype", [F16, F32])
def test_gemm_fp16(gpu, m, n, k, epi, out_dtype):
    a = randn(m, k, seed=m, dtype=F16)
    w = randn(n, k, seed=n, dtype=F16, scale=0.05)
    b = None if epi == _lib.EPI_NONE else randn(n, seed=k, dtype=F16)
    out = cg.kernels._gemm(a.to(gpu), w.to(gpu), None if b is None else b.to(gpu), epi, out_dtype,
                           "t")
    assert out.dtype == out_dtype
    close(out, gemm_ref(a, w, b, epi), 1e-4 * math.sqrt(k / 64), REL[out_dtype],
          f"fp16 gemm {m}x{n}x{k} epi{epi}")


@pytest.mark.parametrize("tile", range(20))
def test_gemm_fp16_every_tile_and_fp32_bias(gpu, tile):
    """Every tile id on fp16 inputs: the register-staged tiles (0-4) and the
    persistent pipelines (5-19, K a multiple of 64), fp32 bias, fp16 out."""
    m, n, k = 300, 264, 520 if tile < 5 else 512
    a = randn(m, k, seed=1, dtype=F16)
    w = randn(n, k, seed=2, dtype=F16, scale=0.05)
    b = randn(n, seed=3, dtype=F32)
    c = torch.empty(m, n, dtype=F16, device=gpu)
    gemm_raw(a.to(gpu), w.to(gpu), b.to(gpu), c, _lib.EPI_BIAS, _lib.CGPT_F16, _lib.CGPT_F32,
             _lib.CGPT_F16, tile)
    close(c, gemm_ref(a, w, b, _lib.EPI_BIAS), 2e-3, 2 ** -11, f"fp16 tile {tile}")


@pytest.mark.parametrize("tile,m", [(_lib.TILE_AUTO, 1000), (14, 2048), (17, 1000), (4, 1000)])
def test_gemm_fp16_residual_epilogue(gpu, tile, m):
    """C += A W^T + bias into fp32 C from fp16 inputs: the slab kernel's residual
    ring (14), the 4-wave pipeline (TILE_AUTO at this size takes 18; 17) and a
    register-staged tile."""
    n, k = 768, 768
    a = randn(m, k, seed=4, dtype=F16)
    w = randn(n, k, seed=5, dtype=F16, scale=0.05)
    b = randn(n, seed=6, dtype=F16)
    c0 = randn(m, n, seed=7, dtype=F32)
    c = c0.to(gpu)
    gemm_raw(a.to(gpu), w.to(gpu), b.to(gpu), c, _lib.EPI_BIAS_RESID, _lib.CGPT_F16,
             _lib.CGPT_F16, _lib.CGPT_F32, tile)
    close(c, gemm_ref(a, w, b, _lib.EPI_BIAS_RESID, c0), 2e-4 * math.sqrt(k / 64), 1e-6,
          f"fp16 resid tile {tile}")


def test_gemm_fp16_dtype_rules(gpu):
    """fp16 inputs take fp16 / fp32 bias and outputs, not bf16; no skinny tile
    and no tile id past the table."""
    lib = _lib.load()
    a = torch.zeros(64, 64, dtype=F16, device=gpu)
    c = torch.zeros(64, 64, dtype=F16, device=gpu)
    s = torch.cuda.current_stream().cuda_stream
    args = lambda bias_code, out_code, tile: (a.data_ptr(), a.data_ptr(), a.data_ptr(), c.data_ptr(),
                                              64, 64, 64, 64, 64, 64, _lib.CGPT_F16, bias_code,
                                              out_code, _lib.EPI_BIAS, tile, s)
    assert lib.cgpt_gemm(*args(_lib.CGPT_BF16, _lib.CGPT_F16, -1)) == -2
    assert lib.cgpt_gemm(*args(_lib.CGPT_F16, _lib.CGPT_BF16, -1)) == -2
    assert lib.cgpt_gemm(*args(_lib.CGPT_F16, _lib.CGPT_F16, lib.cgpt_gemm_num_tiles())) == -1
    assert lib.cgpt_gemm(*args(_lib.CGPT_F16, _lib.CGPT_F16, _lib.TILE_SKINNY)) == -1
    torch.cuda.synchronize()


@pytest.mark.parametrize("n", [1, 7, 4099, 32 * 512 * 768])
def test_gelu_fp16(gpu, n):
    x = randn(n, seed=n, dtype=F16, scale=3.0)
    y = cg.cutile_gelu(x.to(gpu))
    assert y.dtype == F16
    close(y, R.gelu_tanh(x.double()), 1e-6, 2 ** -11, "gelu fp16")


@pytest.mark.parametrize("rows,cols", [(3, 48), (37, 768), (5, 1600), (2, 4100), (16384, 768)])
@pytest.mark.parametrize("with_delta", [False, True])
@pytest.mark.parametrize("pd", [F16, F32])
def test_layernorm_fp16(gpu, rows, cols, with_delta, pd):
    """fp16 rows: the register-resident kernel up to 4096 columns (fp16 or fp32
    gamma / beta), the block-per-row kernel beyond."""
    x = randn(rows, cols, seed=rows, dtype=F16)
    d = randn(rows, cols, seed=cols, dtype=F16) if with_delta else None
    g = (1 + 0.1 * randn(cols, seed=1)).to(pd)
    b = (0.1 * randn(cols, seed=2)).to(pd)
    xg = x.to(gpu)
    xo = torch.empty_like(xg) if with_delta else None
    y = cg.add_layer_norm(xg, None if d is None else d.to(gpu), g.to(gpu), b.to(gpu), 1e-5,
                          x_out=xo)
    s = x.double() if d is None else x.double() + d.double()
    close(y, R.layer_norm(s, g.double(), b.double()), 2e-3, 2 ** -11, f"ln fp16 {rows}x{cols}")
    if with_delta:
        close(xo, s, 1e-7, 2 ** -11, "ln fp16 x_out")


@pytest.mark.parametrize("B,H,hd,T", [(2, 3, 64, 200), (2, 3, 32, 64), (2, 3, 128, 300),
                                       (8, 16, 64, 1024)])
def test_attention_fp16(gpu, B, H, hd, T):
    """fp16 causal attention: the direct-to-LDS kernel (head_dim 64 / 128; 64-
    and, at 8x16x1024, 128-query blocks) and the register-staged one (32)."""
    q, k, v = (randn(B, H, T, hd, seed=i, dtype=F16) for i in range(3))
    o = cg.cutile_causal_attention(q.to(gpu), k.to(gpu), v.to(gpu), H)
    assert o.dtype == F16
    ref = R.causal_attention(q.double(), k.double(), v.double(), p_dtype=F16)
    close(o, ref, 1e-3, 2 ** -10, f"attention fp16 hd{hd}")


def test_embedding_fp16(gpu):
    wte = randn(100, 72, seed=1, dtype=F16)
    wpe = randn(32, 72, seed=2, dtype=F16)
    idx = torch.randint(0, 100, (3, 32), generator=torch.Generator().manual_seed(3))
    out = cg.kernels.token_pos_embedding(idx.to(gpu), wte.to(gpu), wpe.to(gpu), out_dtype=F32)
    ref = wte.double()[idx] + wpe.double()[torch.arange(32)]
    close(out, ref, 1e-6, 1e-6, "embedding fp16 -> fp32")
    out16 = cg.cutile_embedding(idx.to(gpu), wte.to(gpu))
    assert out16.dtype == F16 and torch.equal(out16.cpu(), wte[idx])


# ------------------------------------------------------------ GEMM, any K

@pytest.mark.parametrize("dtype", [F32, BF16, F16])
@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (5, 7, 3), (70, 130, 13), (300, 200, 771),
                                   (129, 65, 100)])
@pytest.mark.parametrize("epi", [_lib.EPI_NONE, _lib.EPI_BIAS, _lib.EPI_BIAS_GELU])
def test_gemm_any_k(gpu, dtype, m, n, k, epi):
    """K not a multiple of the 16-byte vector: the element-load kernel (rows of
    A and W start at any element)."""
    a = randn(m, k, seed=m + k, dtype=dtype)
    w = randn(n, k, seed=n + k, dtype=dtype, scale=0.05)
    b = None if epi == _lib.EPI_NONE else randn(n, seed=k, dtype=dtype)
    out_dtype = F32
    out = cg.kernels._gemm(a.to(gpu), w.to(gpu), None if b is None else b.to(gpu), epi, out_dtype,
                           "t")
    close(out, gemm_ref(a, w, b, epi), 1e-4 * math.sqrt(max(k, 64) / 64), 1e-5,
          f"any-K gemm {dtype} {m}x{n}x{k}")


@pytest.mark.parametrize("dtype", [F32, BF16, F16])
def test_gemm_unaligned_pointers_and_resid(gpu, dtype):
    """16-byte-aligned shapes through pointers one element off a 16-byte
    boundary (the element-load kernel), all four epilogues, the residual one
    into an fp32 C."""
    m, n, k = 77, 96, 64
    a = randn(m, k, seed=1, dtype=dtype)
    w = randn(n, k, seed=2, dtype=dtype, scale=0.05)
    b = randn(n, seed=3, dtype=F32)
    ag, wg, bg = unaligned(a, gpu), unaligned(w, gpu), unaligned(b, gpu)
    code = CODE[dtype]
    for epi in (_lib.EPI_NONE, _lib.EPI_BIAS, _lib.EPI_BIAS_GELU):
        c = torch.empty(m, n, dtype=F32, device=gpu)
        gemm_raw(ag, wg, bg, c, epi, code, _lib.CGPT_F32, _lib.CGPT_F32)
        close(c, gemm_ref(a, w, b, epi), 1e-4, 1e-5, f"unaligned {dtype} epi{epi}")
    c0 = randn(m, n, seed=4, dtype=F32)
    c = unaligned(c0, gpu)
    gemm_raw(ag, wg, bg, c, _lib.EPI_BIAS_RESID, code, _lib.CGPT_F32, _lib.CGPT_F32)
    close(c, gemm_ref(a, w, b, _lib.EPI_BIAS_RESID, c0), 1e-4, 1e-5, f"unaligned resid {dtype}")


def test_gemm_any_k_equals_padded_k(gpu):
    """The element-load kernel's K tail is zero-filled: a K = 100 product equals
    the vector kernel's on the same data zero-padded to K = 104, bit for bit
    (same tile and summation order: tile 4, k32 slabs)."""
    m, n, k = 256, 192, 100
    a = randn(m, k, seed=8, dtype=BF16)
    w = randn(n, k, seed=9, dtype=BF16, scale=0.05)
    ap = torch.nn.functional.pad(a, (0, 4))
    wp = torch.nn.functional.pad(w, (0, 4))
    out = cg.kernels._gemm(a.to(gpu), w.to(gpu), None, _lib.EPI_NONE, F32, "t")
    ref = cg.kernels._gemm(ap.to(gpu), wp.to(gpu), None, _lib.EPI_NONE, F32, "t", tile=4)
    assert torch.equal(out, ref)


# ------------------------------------------------------ LayerNorm, any width

@pytest.mark.parametrize("rows,cols", [(3, 1), (4, 6), (5, 50), (7, 1001), (3, 4099), (2, 8192),
                                       (2, 10000)])
@pytest.mark.parametrize("xd,yd", [(F32, F32), (BF16, BF16), (F32, BF16)])
def test_layernorm_any_width(gpu, rows, cols, xd, yd):
    x = randn(rows, cols, seed=cols, dtype=xd, scale=2.0) + 0.5
    d = randn(rows, cols, seed=cols + 1, dtype=xd)
    g = 1 + 0.1 * randn(cols, seed=3)
    b = 0.1 * randn(cols, seed=4)
    xg = x.to(gpu)
    y = cg.add_layer_norm(xg, d.to(gpu), g.to(gpu), b.to(gpu), 1e-5, out_dtype=yd, x_out=xg)
    s = x.double() + d.double()
    ref = R.layer_norm(s, g.double(), b.double())
    tol = 1e-4 if yd == F32 else 2 ** -8
    close(y, ref, 1e-4, tol, f"ln any width {rows}x{cols} {xd}->{yd}")
    # x_out aliased x: x now holds the residual sum (rounded to x's dtype).
    close(xg, s, 1e-6, REL[xd], "ln any width x_out")


def test_layernorm_unaligned_rows(gpu):
    """Rows of 4-multiple width through pointers off the 16-byte boundary take
    the block-per-row kernel, and agree with the vector kernel on aligned
    copies of the same data."""
    rows, cols = 9, 768
    x = randn(rows, cols, seed=5)
    g = 1 + 0.1 * randn(cols, seed=6)
    b = 0.1 * randn(cols, seed=7)
    y = cg.add_layer_norm(unaligned(x, gpu), None, g.to(gpu), b.to(gpu), 1e-5)
    y_vec = cg.add_layer_norm(x.to(gpu), None, g.to(gpu), b.to(gpu), 1e-5)
    ref = R.layer_norm(x.double(), g.double(), b.double())
    close(y, ref, 1e-5, 1e-5, "ln unaligned")
    close(y, y_vec, 1e-6, 1e-6, "ln unaligned vs vector")


# ------------------------------------------------------ embedding, any width

@pytest.mark.parametrize("D", [1, 6, 50, 1001])
@pytest.mark.parametrize("dtype", [F32, BF16])
def test_embedding_any_width(gpu, D, dtype):
    wte = randn(64, D, seed=D, dtype=dtype)
    wpe = randn(16, D, seed=D + 1, dtype=dtype)
    idx = torch.randint(0, 64, (2, 16), generator=torch.Generator().manual_seed(D))
    out = cg.kernels.token_pos_embedding(idx.to(gpu), wte.to(gpu), wpe.to(gpu), out_dtype=F32)
    close(out, wte.double()[idx] + wpe.double()[torch.arange(16)], 0, 1e-7,
          f"embedding D={D}")
    assert torch.equal(cg.cutile_embedding(idx.to(gpu), wte.to(gpu)).cpu(), wte[idx])


# ---------------------------------------------------- attention head_dim pad

@pytest.mark.parametrize("hd", [8, 24, 40, 96, 100])
@pytest.mark.parametrize("dtype", [F32, BF16])
def test_attention_padded_head_dim(gpu, hd, dtype):
    B, H, T = 2, 3, 130
    q, k, v = (randn(B, H, T, hd, seed=10 + i, dtype=dtype) for i in range(3))
    o = cg.cutile_causal_attention(q.to(gpu), k.to(gpu), v.to(gpu), H)
    assert o.shape == (B, H, T, hd) and o.is_contiguous()
    ref = R.causal_attention(q.double(), k.double(), v.double(),
                             p_dtype=None if dtype == F32 else dtype)
    if dtype == F32:
        close(o, ref, 2e-5, 2e-5, f"attention hd{hd} fp32")
    else:
        close(o, ref, 4e-3, 2 ** -8, f"attention hd{hd} bf16")


def test_attention_head_dim_limit(gpu):
    q = torch.zeros(1, 1, 4, 160, device=gpu)
    with pytest.raises(ValueError):
        cg.cutile_causal_attention(q, q, q, 1)

"""cgpt_gemm_skinny_noalloc (split-K skinny GEMM on the library's static
scratch array) against cgpt_gemm_skinny with a caller workspace: bit-identical
outputs on two calls in a row, the second with a smaller problem (the array
keeps the first call's contents), the largest split the planner makes for
M <= 64 (it fills the 8 MiB array but for 16 KiB), the call captured in a HIP
graph and replayed, no device memory taken by the calls, plus the argument
checks."""

import ctypes

import pytest
import torch

from cutilegpt_amd import _lib

pytestmark = pytest.mark.gpu


def _operands(gpu, M, N, K, dtype):
    g = torch.Generator(device=gpu).manual_seed(M * 131 + N + K)
    a = torch.randn(M, K, device=gpu, generator=g).to(dtype)
    w = (torch.randn(N, K, device=gpu, generator=g) * 0.05).to(dtype)
    b = torch.randn(N, device=gpu, generator=g).to(dtype)
    return a, w, b


def _run_pair(gpu, M, N, K, epi, dtype, out_dtype):
    lib = _lib.load()
    s = torch.cuda.current_stream(gpu).cuda_stream
    code = {torch.float32: _lib.CGPT_F32, torch.bfloat16: _lib.CGPT_BF16}
    a, w, b = _operands(gpu, M, N, K, dtype)
    wb, nc = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(lib.cgpt_gemm_skinny_workspace(M, N, K, code[dtype], ctypes.byref(wb),
                                              ctypes.byref(nc)), "workspace")
    ws = torch.empty(max(wb.value, 16) // 4 + 4, dtype=torch.float32, device=gpu)
    cnt = torch.zeros(max(nc.value, 1), dtype=torch.int32, device=gpu)
    ref = torch.full((M, N), float("nan"), dtype=out_dtype, device=gpu)
    out = torch.full((M, N), float("nan"), dtype=out_dtype, device=gpu)
    args = (a.data_ptr(), w.data_ptr(), b.data_ptr())
    tail = (M, N, K, K, K, N, code[dtype], code[dtype], code[out_dtype], epi)
    _lib.check(lib.cgpt_gemm_skinny(*args, ref.data_ptr(), *tail, ws.data_ptr(), wb.value,
                                    cnt.data_ptr(), nc.value, s), "skinny")
    _lib.check(lib.cgpt_gemm_skinny_noalloc(*args, out.data_ptr(), *tail, s), "skinny_noalloc")
    torch.cuda.synchronize()
    return out, ref, nc.value, wb.value


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_path_twice(gpu, dtype):
    """Two calls in a row, the second smaller: both bit-identical to the
    caller-workspace path (same kernels, same split, same summation order)."""
    for M, N, K, epi, od in ((32, 4800, 1600, _lib.EPI_BIAS, torch.float32),
                             (7, 1600, 1280, _lib.EPI_BIAS_GELU, dtype)):
        out, ref, n_counters, _ = _run_pair(gpu, M, N, K, epi, dtype, od)
        assert n_counters > 0  # the split-K path (workspace and counters) ran
        assert torch.isfinite(out).all()
        assert torch.equal(out, ref), (M, N, K)


def test_noalloc_argument_checks(gpu):
    lib = _lib.load()
    x = torch.zeros(128, 128, dtype=torch.bfloat16, device=gpu)
    p = x.data_ptr()
    # M > 64: the skinny kernels take at most 64 rows
    assert lib.cgpt_gemm_skinny_noalloc(p, p, None, p, 65, 64, 64, 64, 64, 64, 1, 1, 1, 0,
                                        None) == -3
    # K not a multiple of 8 for bf16; bias missing for a bias epilogue
    assert lib.cgpt_gemm_skinny_noalloc(p, p, None, p, 4, 64, 60, 64, 64, 64, 1, 1, 1, 0,
                                        None) == -3
    assert lib.cgpt_gemm_skinny_noalloc(p, p, None, p, 4, 64, 64, 64, 64, 64, 1, 1, 1, 1,
                                        None) == -1
    assert lib.cgpt_gemm_skinny_noalloc(None, None, None, None, 0, 64, 64, 64, 64, 64, 1, 1, 1,
                                        0, None) == 0
    assert b"static buffer" in lib.cgpt_status_string(-4)


def test_noalloc_largest_split_fits(gpu):
    """M = 64 (four m-tiles), N = 16352 (511 column slices, the most that still
    get split) and K = 1024 bf16 (enough double slabs for two chunks): the
    planner's largest workspace, 1022 slice-chunks x 4 m-tiles x 2 KiB =
    8 372 224 bytes, inside the 8 MiB array.  Returns OK and equals the
    caller-workspace path."""
    out, ref, n_counters, ws_bytes = _run_pair(gpu, 64, 16352, 1024, _lib.EPI_BIAS,
                                               torch.bfloat16, torch.float32)
    assert n_counters == 511 and ws_bytes == 1022 * 4 * 2048 <= 8 << 20
    assert torch.isfinite(out).all()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("N", [16352, 30000])
def test_noalloc_decode_form_within_capacity(gpu, N):
    """32 bf16 rows, K = 1024: the decode form's split (4 chunks, 8 n-tiles a
    block) needs exactly 8 MiB of chunk sums at N = 16352 and is taken; at
    N = 30000 it would need 15 MB, so both entry points take the other form
    instead — the workspace query stays within the static array and the two
    paths stay bit-identical."""
    out, ref, n_counters, ws_bytes = _run_pair(gpu, 32, N, 1024, _lib.EPI_BIAS,
                                               torch.bfloat16, torch.float32)
    assert ws_bytes <= 8 << 20 and n_counters <= 1024
    assert torch.isfinite(out).all()
    assert torch.equal(out, ref)
    a, w, b = _operands(gpu, 32, N, 1024, torch.bfloat16)
    exact = a.double() @ w.double().t() + b.double()
    assert (out.double() - exact).abs().max().item() <= 1e-4 * (exact.abs().max().item() + 1)


def test_noalloc_graph_capture_and_no_device_allocation(gpu):
    """The call captured in a HIP graph and replayed three times, with other
    work and synchronisations between the replays, gives the eager
    caller-workspace result bit for bit each time (the counters are cleared
    by a fill kernel, not a memset); eager calls leave the device's free
    memory and torch's allocation count unchanged."""
    lib = _lib.load()
    M, N, K = 32, 4800, 1600
    bf = torch.bfloat16
    a, w, b = _operands(gpu, M, N, K, bf)
    _, ref, n_counters, _ = _run_pair(gpu, M, N, K, _lib.EPI_BIAS, bf, torch.float32)
    assert n_counters > 0
    out = torch.full((M, N), float("nan"), device=gpu)
    tail = (M, N, K, K, K, N, _lib.CGPT_BF16, _lib.CGPT_BF16, _lib.CGPT_F32, _lib.EPI_BIAS)
    args = (a.data_ptr(), w.data_ptr(), b.data_ptr(), out.data_ptr())

    torch.cuda.synchronize()
    free0, alloc0 = torch.cuda.mem_get_info(gpu)[0], torch.cuda.memory_allocated(gpu)
    for _ in range(3):
        _lib.check(lib.cgpt_gemm_skinny_noalloc(*args, *tail,
                                                torch.cuda.current_stream(gpu).cuda_stream),
                   "noalloc")
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(gpu)[0] == free0
    assert torch.cuda.memory_allocated(gpu) == alloc0
    assert torch.equal(out, ref)

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            st = lib.cgpt_gemm_skinny_noalloc(*args, *tail, side.cuda_stream)
    assert st == 0
    torch.cuda.current_stream(gpu).wait_stream(side)
    other = torch.randn(2048, 2048, device=gpu)
    for r in range(3):
        out.fill_(float("nan"))
        _ = other @ other  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), r

"""bench.py's measurement arithmetic on the CPU: the algorithmic work units it
divides by match the figures the benchmark definition states (FLOP of a GPT-2
forward, bytes of the standalone GELU / LayerNorm, FLOP of the standalone
causal attention), and the multi-GPU guard refuses N > 1."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_gpt2_forward_flops():
    gemm, head, attn = bench.flops(12, 768, 16, 1024)
    assert gemm == 2_783_138_807_808
    assert head == 1_264_758_816_768
    assert attn == 309_539_635_200
    assert gemm + head + attn == 4_357_437_259_776


def test_medium_forward_flops():
    gemm, head, attn = bench.flops(8, 512, 16, 256)
    assert gemm + head + attn == 425_575_055_360


def test_standalone_work_units():
    n = 32 * 512 * 768
    assert 2 * n * 2 == 50_331_648 and 2 * n * 4 == 100_663_296          # GELU bf16 / fp32
    M, N = 16384, 768
    assert 2 * M * N * 2 + 2 * N * 2 == 50_334_720                        # LayerNorm bf16
    assert 2 * M * N * 4 + 2 * N * 4 == 100_669_440                       # LayerNorm fp32
    B, H, T, hd = 8, 12, 512, 64
    assert 4 * B * H * hd * T * (T + 1) // 2 == 3_227_516_928             # causal attention


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr

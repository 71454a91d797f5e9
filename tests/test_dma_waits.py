"""The DMA-staged skinny kernels' one scheduling assumption, checked in the
code the compiler emits for them (CPU only: hipcc cross-compiles).

gemm_decode_kernel and gemm_skinny_wide_kernel stage A in LDS with
direct-to-LDS buffer loads issued from inline assembly, then issue their
first round of W loads, then wait with ``s_waitcnt vmcnt(n)`` before the
barrier: n is the number of W loads of that round, so the wait completes
every DMA (vmcnt retires in order) without waiting for W.  That holds only
if exactly n vector-memory loads sit between the last DMA and the wait in
the emitted code.  The sources arrange it (W is not ``__restrict__``, so its
loads cannot move across the memory clobbers on either side); this test
reads the device assembly of every instance and checks it, and that M0,
which the helper writes from inline assembly, is used by nothing else.
"""

import os
import re
import shutil
import subprocess

import pytest

from cutilegpt_amd import build as B

KERNELS = re.compile(r"^(_ZN4cgpt(?:18gemm_decode_kernel|23gemm_skinny_wide_kernel)\S*):")


def _expected_loads(symbol):
    m = re.search(r"gemm_decode_kernelILi\d+ELi\d+ELi(\d+)E", symbol)
    if m:
        return 2 * int(m.group(1))  # KS double slabs x two 16-byte halves
    return 10                       # the wide kernel: kWideDpw (5) x 2


def _device_asm(tmp_path):
    out = tmp_path / "skinny.s"
    cmd = [B.hipcc(), *B.HIPCC_FLAGS, "-Wno-inline-asm", "--cuda-device-only", "-S",
           os.path.join(B.CSRC, "skinny.hip"), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text().splitlines()


def _check_m0(lines):
    """The DMA helper writes M0 from inline assembly (its LDS address); the
    compiler does not save M0 around it, so no compiler-emitted instruction
    may use M0: every line that names it must be one of the helper's moves,
    followed (after its wait state) by the DMA that reads it."""
    code = [l.strip() for l in lines if l.strip() and not l.strip().startswith(";")]
    moves = 0
    for i, line in enumerate(code):
        if re.search(r"\bm0\b", line):
            assert line.startswith("s_mov_b32 m0,"), line
            assert code[i + 1] == "s_nop 0" and code[i + 2].endswith("offen lds"), code[i:i + 3]
            moves += 1
    return moves


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="needs hipcc")
def test_dma_wait_counts_only_the_first_w_round(tmp_path):
    lines = _device_asm(tmp_path)
    assert _check_m0(lines) > 0
    found = {}
    cur = None
    for line in lines:
        m = KERNELS.match(line)
        if m:
            cur = m.group(1)
            found[cur] = {"last_dma": False, "after": 0, "wait": None, "barrier": False}
            continue
        if cur is None:
            continue
        st = found[cur]
        if st["barrier"]:
            continue
        if "offen lds" in line:
            st["last_dma"], st["after"], st["wait"] = True, 0, None
        elif "buffer_load" in line and st["last_dma"]:
            st["after"] += 1
        elif "s_waitcnt" in line and "vmcnt(" in line and st["last_dma"] and st["wait"] is None:
            st["wait"] = (st["after"], int(re.search(r"vmcnt\((\d+)\)", line).group(1)))
        elif "s_barrier" in line:
            st["barrier"] = True
    decode = [k for k in found if "gemm_decode_kernel" in k]
    wide = [k for k in found if "gemm_skinny_wide_kernel" in k]
    assert len(decode) >= 16 and len(wide) >= 6, (len(decode), len(wide))
    for sym, st in found.items():
        n = _expected_loads(sym)
        assert st["last_dma"] and st["barrier"], sym
        # The first vmcnt wait after the last DMA: n loads issued since, and it
        # leaves exactly those n outstanding.
        assert st["wait"] == (n, n), (sym, st["wait"], n)

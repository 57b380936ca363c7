"""Exhaustive host check of the quantiser's device arithmetic, compiled from
the library's own headers (tests/arith/quant_arith_check.cpp):

  * d = div127(amax), a product and an FMA correction, equals the IEEE
    division amax / 127.0f for every non-negative binary32 (the kernels use it
    instead of the division sequence);
  * the branch-free float_to_half_bits_rtz equals the oracle's truncating fp16
    encoder (restated from real_stock_dp4a_comparator.hip:43-62) for all 2^32
    binary32 patterns.

Runs on the host in a few seconds (OpenMP); the GPU tests then check the
same arithmetic bit-exactly inside the kernels.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _has_fma() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            return any(line.startswith("flags") and " fma " in line + " " for line in f)
    except OSError:
        return False


@pytest.mark.skipif(not os.path.exists(HIPCC) and shutil.which("hipcc") is None, reason="needs hipcc for the host build")
def test_div127_and_rtz_encoder_exhaustive(orc, tmp_path):
    from oracle.oracle import LIB_PATH

    exe = str(tmp_path / "quant_arith_check")
    cmd = [HIPCC if os.path.exists(HIPCC) else "hipcc", "-x", "hip", "--offload-host-only", "-O2", "-fopenmp",
           "-ffp-contract=off", "-I" + os.path.join(ROOT, "qwen_3.8_27b_optimizations_amd", "csrc"),
           os.path.join(ROOT, "tests", "arith", "quant_arith_check.cpp"), "-o", exe, "-ldl"]
    if _has_fma():
        cmd.insert(5, "-mfma")
    subprocess.run(cmd, check=True, capture_output=True)
    env = dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1)))
    r = subprocess.run([exe, LIB_PATH], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "div127 mismatches 0, rtz mismatches 0" in r.stdout

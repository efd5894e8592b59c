"""Host check of the multiply-high division (kernelproblems_amd/csrc/kp_div32.hpp)
that indexes rope_tile, rope_c64_tile and unshard_kernel: the same constexpr
make_div32 / div32 the kernels compile, built here with g++ (no HIP headers)
and run over ~2.6 million (n, d) pairs against the quotient n / d -- every
divisor up to 4096, 2^k and 2^k +- 1 / +- 2, the divisors just below 2^31,
numerators around multiples of d and around 2^31 - 1, and random pairs."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_div32_matches_quotient(tmp_path):
    exe = tmp_path / "div32_check"
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{ROOT / 'kernelproblems_amd' / 'csrc'}",
                    str(ROOT / "tests" / "native" / "div32_check.cpp"), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "0 mismatches" in res.stdout
    checked = int(res.stdout.split("checked ")[1].split()[0])
    assert checked > 2_000_000

"""The device kernels' integer requantization map (gemmkit_amd/csrc/requant.h)
equals the oracle's f64 formula bit for bit, over the reference's sweep
values, exact halves, near-ties where the f64 product rounds, special scales
and ~16M random cases (tests/requant_int_check.cpp)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_requant_bits_matches_oracle(tmp_path):
    lib_dir = os.path.join(ROOT, "oracle")
    if not os.path.exists(os.path.join(lib_dir, "liboracle.so")):
        subprocess.run(["make", "-C", lib_dir], check=True, capture_output=True)
    exe = str(tmp_path / "requant_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", os.path.join(ROOT, "gemmkit_amd", "csrc"),
                    os.path.join(HERE, "requant_int_check.cpp"), "-L", lib_dir, "-loracle",
                    f"-Wl,-rpath,{lib_dir}", "-o", exe], check=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout[-2000:]
    assert out.stdout.strip().splitlines()[-1].startswith("mismatches 0 ")

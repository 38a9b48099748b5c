"""hy_expf (the GPU's expf, hymt2_amd/csrc/hy_expf.h) equals the C library's expf, which the
reference calls in softmax and SiLU (src/model.c:787, :875), on every float in [-105, 90]
(the whole non-overflow/underflow range). Compiled for the host with g++ from the same header
the kernels include."""
import os
import subprocess

from conftest import ROOT


def test_expf_matches_libm_exhaustively(tmp_path):
    exe = tmp_path / "expf_check"
    src = os.path.join(ROOT, "tests", "helpers", "expf_check.cpp")
    inc = os.path.join(ROOT, "hymt2_amd", "csrc")
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-pthread", "-I", inc, src, "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe), "-105", "90", str(min(8, os.cpu_count() or 1))], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches=0" in r.stdout
    assert int(r.stdout.split("total=")[1]) > 2_000_000_000


def test_expf_special_values(tmp_path):
    src = tmp_path / "s.cpp"
    src.write_text('#include "hy_expf.h"\n#include <cmath>\n#include <cstdio>\n#include <cstring>\n'
                   'int main(){ float xs[] = {0.f, -0.f, INFINITY, -INFINITY, NAN, 88.72f, 88.8f, -103.9f, -104.f, '
                   '-200.f, 1e-30f, -1e-30f}; int bad = 0;\n'
                   ' for (float x : xs) { float a = hy_expf(x), r = expf(x); unsigned ba, br; memcpy(&ba,&a,4); '
                   'memcpy(&br,&r,4); if (ba != br && !(std::isnan(a) && std::isnan(r))) { printf("%a %a %a\\n", x, a, r); bad++; } }\n'
                   ' return bad; }\n')
    exe = tmp_path / "s"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-I", os.path.join(ROOT, "hymt2_amd", "csrc"),
                    str(src), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout

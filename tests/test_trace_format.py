"""CPU: the trace rows' number formatting (treesa_gpu_amd/host/tsa_fmt.h) writes what printf writes.

The binary's JSON trace is the reference's row format (csrc/treesa_gpu.cu:1830-1832: "%.4f", "%d", "%.6f",
"%.3f" fields).  tests/fmt_check.cpp compares fmt_fixed with snprintf("%.*f") at every precision 0..9 on about
600 000 doubles -- random bit patterns over all exponents, uniform values of the trace's ranges, exact ties
k / 2^j (round half to even) and their neighbours, values that round up across a power of ten, signed zeros,
subnormals and the snprintf fallbacks -- and fmt_int with "%lld"; every string must be identical.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_fixed_and_int_formatting_equal_printf(tmp_path):
    exe = str(tmp_path / "fmt_check")
    subprocess.run(["g++", "-O2", "-I", os.path.join(ROOT, "treesa_gpu_amd", "host"), os.path.join(HERE, "fmt_check.cpp"),
                    "-o", exe], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    bad, checked = map(int, r.stdout.split())
    assert bad == 0, r.stderr
    assert checked > 6_000_000

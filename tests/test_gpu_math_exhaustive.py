"""The float math the sweep kernels restate, as the gfx950 build evaluates it, against this host's libm on every
input (bin/tsa_mathcheck): expf and exp2f on all 2^32 floats, log2f on every float of [1, 2] through the
correction table, the reference's lse fold mx + log2f(1 + exp2f(mn - mx)) (csrc/common.h:119-125) for every
difference in [-24, 0] at six magnitudes, and the Metropolis threshold of every 24-bit uniform the kernels draw.
The host copies of the same functions are checked against libm by tests/test_math_exhaustive.py; this closes the
gap between the two builds (double fma, conversions, denormals on the device)."""
import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "treesa_gpu_amd", "bin", "tsa_mathcheck")


def test_device_math_equals_host_libm_exhaustively():
    assert os.path.exists(EXE), "bin/tsa_mathcheck is not built (make -C treesa_gpu_amd)"
    print("[gpu] tsa_mathcheck: expf/exp2f on 2^32 floats, log2f on [1,2], lse, thresholds", flush=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=110)
    assert r.returncode in (0, 1), r.stderr[-2000:]
    res = json.loads(r.stdout.strip().splitlines()[-1])
    print(res, flush=True)
    assert res["exp_inputs"] == 1 << 32 and res["log2f_inputs"] == (1 << 23) + 1
    assert res["threshold_inputs"] == 1 << 24 and res["lse_inputs"] == 6 * (0xC1C00000 - 0x80000000 + 1)
    bad = {k: v for k, v in res.items() if k.endswith("_mismatch") and v != 0}
    assert not bad, bad

"""The engine quantizer's division-free quotient (lt_numerics.h: lt_q8_quotient, used by
every device quantizer) equals IEEE division x / dq bit for bit, on the CPU over every
positive finite fp16 scale (tests/csrc/q8_quotient_check.c), and on the device together
with the hardware fp16 conversion of the scale (lt_selftest_numerics)."""
import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_quotient_matches_ieee_division_on_cpu(tmp_path):
    exe = tmp_path / "qchk"
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-o", str(exe),
                    str(ROOT / "tests" / "csrc" / "q8_quotient_check.c"), "-lm"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True)
    cases, bad_bits, bad_q = map(int, out.stdout.split())
    assert cases > 80_000_000
    assert (bad_bits, bad_q) == (0, 0), out.stderr


def _special_blocks():
    x = np.zeros(5 * 32, np.float32)
    x[0:32] = np.float32(1e-7) * np.linspace(-1, 1, 32, dtype=np.float32)    # amax/127 < 2^-25: d16 = 0
    x[32:64] = np.float32(1e10) * np.linspace(-1, 1, 32, dtype=np.float32)   # amax/127 > 65504: d16 = inf
    x[64:96] = np.float32(127 * 2.0 ** -24) * np.linspace(-1, 1, 32, dtype=np.float32)  # subnormal fp16 scale
    x[96:128] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5] + [126.5, -126.5, 0.49999997] + [0.0] * 21
    x[128:160] = np.float32(3.0) * np.linspace(-1, 1, 32, dtype=np.float32)
    return x


def test_quant_zero_and_infinite_scales(oracle):
    """x / 0 saturates to +-127 (0 for x = 0) and x / inf quantizes to 0, as the GPUs'
    saturating float->int conversion gives them."""
    x = _special_blocks()
    xq, xd = oracle.quant_q8(x)
    assert xd[0] == 0 and xd[1] == 0x7C00
    assert list(xq[0:32]) == [-127] * 16 + [127] * 16
    assert np.all(xq[32:64] == 0)
    assert list(xq[96:107]) == [127, 2, 4, -2, -4, 0, 2, 0, 126, -126, 0]


@pytest.mark.gpu
def test_device_quant_special_blocks(gpu, oracle):
    from llamatov_amd import engine as dr
    x = _special_blocks()
    xq, xd = oracle.quant_q8(x)
    dx = dr.DevTensor.from_host(x, gpu)
    dq = dr.DevTensor.empty((x.size,), np.int8, gpu)
    dd = dr.DevTensor.empty((x.size // 32,), np.uint16, gpu)
    dr.quant_q8_into(dx, dq, dd, x.size)
    assert np.array_equal(dq.to_host(), xq) and np.array_equal(dd.to_host(), xd)
    for t in (dx, dq, dd):
        t.free()


@pytest.mark.gpu
def test_device_fp16_conversion_and_quotient(gpu):
    from llamatov_amd import _lib
    out = (ctypes.c_ulonglong * 4)()
    _lib.call("lt_selftest_numerics", gpu.handle, out)
    f2h_bad, q_bits, q_bad, cases = list(out)
    assert cases > 8_000_000
    assert (f2h_bad, q_bits, q_bad) == (0, 0, 0)

"""Gate the gates: every comparator the parity tests use must fail on a known-bad artifact.

The reference's own probe (bpd/kernelgen/referee/fixtures/failed_test_injection.py:14-60) feeds
its comparison gate deliberate mismatches -- a flipped last bit, a flipped mantissa bit, a NaN,
a wrong shape -- and requires each to fail, since a gate that cannot fail protects nothing.
This does the same for the comparators written in this build's tests: the bit-exact helpers
(`bitexact`, `assert_bitexact`, `same_bits`) and the ULP distance (`ulp_diff`) behind the
oracle's float64 bounds.  Each probe also pins the semantics of the passing cases (identical
NaN bits compare equal bitwise; +0 and -0 differ bitwise but are 0 ULP apart)."""
import importlib.util
import sys
from pathlib import Path

import numpy as np
import pytest

HERE = Path(__file__).resolve().parent


def module(name):
    if str(HERE) not in sys.path:
        sys.path.insert(0, str(HERE))
    spec = importlib.util.spec_from_file_location(f"_gate_{name}", HERE / f"{name}.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def as_bool(fn):
    """A comparator as pass/fail, whether it returns a bool or asserts."""
    def check(a, b):
        try:
            r = fn(a, b) if fn.__code__.co_argcount == 2 else fn(a, b, "probe")
        except AssertionError:
            return False
        return True if r is None else bool(r)
    return check


BITEXACT = [("test_gpu_batch", "bitexact"), ("test_gpu_decode", "bitexact"), ("test_gpu_gguf", "bitexact"),
            ("test_gpu_fused", "assert_bitexact"), ("test_gpu_ggml", "assert_bitexact"),
            ("test_gpu_ops", "assert_bitexact"), ("test_golden", "same_bits")]


def base():
    return np.random.RandomState(1).randn(896).astype(np.float32)


def flip(a, i, bit):
    b = a.copy()
    b.view(np.uint32)[i] ^= np.uint32(1 << bit)
    return b


@pytest.mark.parametrize("mod,name", BITEXACT)
def test_bitexact_comparators_fail_on_bad_artifacts(mod, name):
    eq = as_bool(getattr(module(mod), name))
    a = base()
    assert eq(a, a.copy()), "control: identical arrays"
    assert not eq(a, flip(a, 895, 0)), "1 ULP on the last element"
    assert not eq(a, flip(a, 448, 22)), "the top mantissa bit of a middle element"
    nan = a.copy()
    nan[0] = np.nan
    assert not eq(a, nan), "one NaN"
    assert eq(nan, nan.copy()), "the same NaN bits in both arms compare equal (bitwise semantics)"
    other = nan.copy()
    other.view(np.uint32)[0] ^= np.uint32(1)   # another NaN payload
    assert np.isnan(other[0]) and not eq(nan, other), "NaNs with different bits"
    z = np.zeros(896, np.float32)
    assert eq(z, z.copy()), "all zeros against all zeros (degenerate but equal)"
    nz = z.copy()
    nz[5] = np.float32(-0.0)
    assert not eq(z, nz), "+0 against -0"
    assert not eq(a, a[:-1].copy()), "a truncated result"
    assert not eq(a.reshape(28, 32), a.reshape(32, 28).copy()), "a transposed shape"


@pytest.mark.parametrize("mod", ["test_gpu_fused", "test_gpu_ggml", "test_gpu_ops", "test_golden"])
def test_integer_comparators_fail_on_one_element(mod):
    """The helpers that also compare integer results (token ids, quants, scales)."""
    name = "same_bits" if mod == "test_golden" else "assert_bitexact"
    eq = as_bool(getattr(module(mod), name))
    q = np.random.RandomState(2).randint(-127, 128, 4864).astype(np.int8)
    assert eq(q, q.copy())
    r = q.copy()
    r[4863] = r[4863] + 1 if r[4863] < 127 else 126
    assert not eq(q, r)
    d = np.arange(152, dtype=np.uint16)
    e = d.copy()
    e[0] ^= 1
    assert not eq(d, e)


@pytest.mark.parametrize("mod", ["test_oracle_pins", "test_oracle_step_pins"])
def test_ulp_distance_is_exact(mod):
    ulp = module(mod).ulp_diff
    a = base()
    assert ulp(a, a).max() == 0
    assert ulp(a, flip(a, 3, 0))[3] == 1
    assert ulp(np.float32(1.0), np.nextafter(np.float32(1.0), np.float32(2.0))) == 1
    # across zero: every representable value between counts (the smallest subnormals, then 0)
    tiny = np.float32(1.4e-45)
    assert ulp(tiny, -tiny) == 2
    assert ulp(np.float32(0.0), np.float32(-0.0)) == 0, "+0 and -0 are 0 ULP apart"
    # a NaN is far beyond every bound the oracle tests allow (at most a few ULP)
    assert ulp(np.float32(1.0), np.float32(np.nan)) > 1 << 20
    assert ulp(np.float32(np.inf), np.float32(3.4e38)) >= 1

"""Pins of the oracle's ggml-compatible numerics (or_quant_q8_ggml, the vec_dot and llamafile
dot orders, the two qmatmul drivers).

Primary pin: the reference's own CPU substrate, bpd-substrate/bench/bpd_cpu.c and
bpd_gemm_q8_0_cpu.c, compiled from where they lie by `make -C oracle ref` into
oracle/_ref/libbpd_cpu.so (AVX1 + F16C, no FMA: the host the reference mirrors).  Those
tests skip where the reference tree is absent (the GPU box).  Secondary pins, which need
nothing but this file: closed forms of the quantizer (the single division id = 127/amax, ties
to even, the zero block) and of the dot (one non-zero lane is one exact product; the lane
and pairing layout shown by integer-valued probes; a float64 bound).

Known deviation, kept on purpose: for an odd block count the reference dispatcher's
single-token path (bpd_gemm_q8_0_cpu.c:54-76) has no tail loop and drops the last block;
ggml's vec_dot and the reference's bpd_qdot_q8_0_q8_0_cpu (bpd_cpu.c:4208-4221) add it.
The oracle follows the latter, so the dispatcher comparison runs at even block counts and
the odd-count tail is pinned against bpd_qdot_q8_0_q8_0_cpu.
"""
from __future__ import annotations

import ctypes
import subprocess
from ctypes import c_int, c_void_p, c_float
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

REF_SO = Path(__file__).resolve().parent.parent / "oracle" / "_ref" / "libbpd_cpu.so"
REF_SRC = Path("/root/reference/bpd-substrate/bench/bpd_cpu.c")


def _ref():
    if not REF_SO.exists() and REF_SRC.exists():
        subprocess.run(["make", "-s", "-C", str(REF_SO.parent.parent), "ref"], check=True,
                       stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    if not REF_SO.exists():
        pytest.skip("oracle/_ref/libbpd_cpu.so is not built (needs the reference tree)")
    L = ctypes.CDLL(str(REF_SO))
    L.bpd_quant_q8_0_cpu.argtypes = [c_void_p, c_void_p, c_int]
    L.bpd_quant_q8_0_cpu.restype = None
    L.bpd_qdot_q8_0_q8_0_cpu.argtypes = [c_void_p, c_void_p, c_int]
    L.bpd_qdot_q8_0_q8_0_cpu.restype = c_float
    L.bpd_qmatmul_q8_0_cpu.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int]
    L.bpd_qmatmul_q8_0_cpu.restype = None
    L.bpd_qmatmul_q8_0_llamafile_cpu.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int]
    L.bpd_qmatmul_q8_0_llamafile_cpu.restype = None
    return L


def _p(a):
    return c_void_p(a.ctypes.data)


def _activations(rng, n, K):
    """Rows with mixed magnitudes, exact zeros, a zero block and values on .5 ties."""
    X = (rng.standard_normal((n, K)) * np.exp(rng.uniform(-6, 6, (n, K // 32, 1))).repeat(32, 2).reshape(n, K))
    X = X.astype(np.float32)
    X[:, 5] = 0.0
    if K >= 64:
        X[0, 32:64] = 0.0                       # a zero block: d = 0, id = 0
    X[-1, :32] = np.arange(-16, 16) + 0.5       # amax 15.5: x * id lands near .5 boundaries
    X[-1, 0] = 127.0                            # amax 127 -> id = 1: exact ties 22.5 -> 22
    X[-1, 1:32] = np.float32(22.5) * np.sign(np.arange(1, 32) - 16)
    return X


def _weights(rng, N, K):
    return oracle.quantize_rows((rng.standard_normal((N, K)) * 0.05).astype(np.float32))


def _ref_blocks(L, x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(x.size // 32 * 34, np.uint8)
    L.bpd_quant_q8_0_cpu(_p(x), _p(y), x.size)
    return y


def _split(blocks):
    b = blocks.reshape(-1, 34)
    return b[:, 2:].copy().view(np.int8).reshape(-1), b[:, :2].copy().view(np.uint16).reshape(-1)


# ---- against the reference's compiled substrate --------------------------------------
def test_quant_matches_reference_substrate():
    L = _ref()
    rng = np.random.default_rng(1)
    X = _activations(rng, 6, 1024)
    for row in X:
        assert np.array_equal(oracle.quant_q8_0_ggml_blocks(row), _ref_blocks(L, row))
        xq, xd = oracle.quant_q8_ggml(row)
        q2, d2 = _split(_ref_blocks(L, row))
        assert np.array_equal(xq, q2) and np.array_equal(xd, d2)


@pytest.mark.parametrize("nb", [1, 2, 3, 28, 29, 152])
def test_vec_dot_matches_reference_substrate(nb):
    L = _ref()
    rng = np.random.default_rng(2 + nb)
    K = 32 * nb
    W = _weights(rng, 16, K)
    x = _activations(rng, 1, K)[0]
    ab = _ref_blocks(L, x)
    xq, xd = _split(ab)
    y = oracle.q8_gemv_ggml(W, xq, xd, K, oracle.GGML_VEC)
    Wr = W.reshape(16, nb * 34)
    for n in range(16):
        r = np.float32(L.bpd_qdot_q8_0_q8_0_cpu(_p(np.ascontiguousarray(Wr[n])), _p(ab), nb))
        assert y[n].view(np.uint32) == r.view(np.uint32), (nb, n)


@pytest.mark.parametrize("M", [1, 2, 5])
def test_qmatmul_matches_reference_substrate(M):
    L = _ref()
    rng = np.random.default_rng(10 + M)
    N, K = 40, 896
    W = _weights(rng, N, K)
    X = _activations(rng, M, K)
    ref = np.empty((M, N), np.float32)
    L.bpd_qmatmul_q8_0_cpu(_p(W), _p(X), _p(ref), M, N, K)
    assert np.array_equal(oracle.qmatmul_q8_0_ggml(W, X, N, K).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("m_tokens", [1, 2, 3, 4, 5, 6, 7, 9])
@pytest.mark.parametrize("K", [896, 32 * 29])
def test_llamafile_matches_reference_substrate(m_tokens, K):
    nb = K // 32
    if nb % 2 and m_tokens % 2:
        pytest.skip("odd block count on the single-token path: the reference dispatcher drops the "
                    "last block (module docstring); pinned by the vec_dot test instead")
    L = _ref()
    rng = np.random.default_rng(20 + m_tokens)
    mw = 24
    W = _weights(rng, mw, K)
    X = _activations(rng, m_tokens, K)
    ref = np.empty((m_tokens, mw), np.float32)
    L.bpd_qmatmul_q8_0_llamafile_cpu(_p(W), _p(X), _p(ref), mw, m_tokens, K)
    got = oracle.qmatmul_q8_0_llamafile(W, X, mw, K)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_llamafile_and_vec_orders_differ():
    """The two orders are distinct functions on ordinary data (so each comparison above
    pins its own order)."""
    rng = np.random.default_rng(30)
    K = 4864
    W = _weights(rng, 256, K)
    xq, xd = oracle.quant_q8_ggml(_activations(rng, 1, K)[0])
    a = oracle.q8_gemv_ggml(W, xq, xd, K, oracle.GGML_VEC)
    b = oracle.q8_gemv_ggml(W, xq, xd, K, oracle.GGML_LLAMAFILE)
    c = oracle.q8_gemv(W, xq, xd, K)
    assert np.any(a != b) and np.any(a != c)


# ---- closed forms (no reference needed) ------------------------------------------------
def test_quant_closed_forms():
    # amax = 127: id = 127/127 = 1 exactly, so q = rint(x): ties to even
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:8] = [22.5, 23.5, -0.5, 0.5, 1.5, -2.5, 126.5]
    xq, xd = oracle.quant_q8_ggml(x)
    assert list(xq[:8]) == [127, 22, 24, 0, 0, 2, -2, 126]
    assert xd[0] == oracle.float_to_half_bits(1.0)
    # the zero block stores d = 0 (the engine's quantizer stores 1)
    xq, xd = oracle.quant_q8_ggml(np.zeros(32, np.float32))
    assert xd[0] == 0 and not xq.any()
    assert oracle.quant_q8(np.zeros(32, np.float32))[1][0] == oracle.float_to_half_bits(1.0)
    # id = 127/amax in one division, not 1/(amax/127): find an amax where the two differ and
    # an x where that difference moves the code
    rng = np.random.default_rng(3)
    found = False
    for amax in rng.uniform(0.5, 2.0, 20000).astype(np.float32):
        id1 = np.float32(127.0) / amax
        id2 = np.float32(1.0) / (amax / np.float32(127.0))
        if id1 == id2:
            continue
        for k in range(1, 127):
            xv = np.float32((k + 0.5) / id1)
            if np.rint(xv * id1) != np.rint(xv * id2):
                blk = np.zeros(32, np.float32)
                blk[0], blk[1] = amax, xv
                assert oracle.quant_q8_ggml(blk)[0][1] == np.int8(np.rint(xv * id1))
                found = True
                break
        if found:
            break
    assert found


def test_dot_closed_forms():
    K = 128
    nb = K // 32
    # one non-zero quant pair: the row value is that block's delta * product, exactly
    W = np.zeros((1, nb, 34), np.uint8)
    W[0, :, :2] = np.array([oracle.float_to_half_bits(0.25)], np.uint16).view(np.uint8)
    W[0, 2, 2 + 7] = np.uint8(np.int8(-3).view(np.uint8))
    xq = np.zeros(K, np.int8)
    xq[2 * 32 + 7] = 5
    xd = np.full(nb, oracle.float_to_half_bits(0.5), np.uint16)
    for order in (oracle.GGML_VEC, oracle.GGML_LLAMAFILE):
        assert oracle.q8_gemv_ggml(W.reshape(-1), xq, xd, K, order)[0] == np.float32(-3 * 5 * 0.25 * 0.5)
    # lane layout and pairing: integer-valued lane sums, where every order is exact, give
    # the plain integer total for both orders (a dropped or doubled block would not)
    rng = np.random.default_rng(4)
    for nbb in (1, 2, 3, 5):
        Kb = 32 * nbb
        Wb = rng.integers(-127, 128, (3, nbb, 32)).astype(np.int8)
        blk = np.zeros((3, nbb, 34), np.uint8)
        blk[:, :, :2] = np.array([oracle.float_to_half_bits(1.0)], np.uint16).view(np.uint8)
        blk[:, :, 2:] = Wb.view(np.uint8)
        xqb = rng.integers(-127, 128, Kb).astype(np.int8)
        xdb = np.full(nbb, oracle.float_to_half_bits(1.0), np.uint16)
        exact = (Wb.reshape(3, Kb).astype(np.int64) * xqb.astype(np.int64)).sum(1)
        for order in (oracle.GGML_VEC, oracle.GGML_LLAMAFILE):
            got = oracle.q8_gemv_ggml(blk.reshape(-1), xqb, xdb, Kb, order)
            assert np.array_equal(got.astype(np.int64), exact), (nbb, order)
    # float64 bound against the dequantized dot
    K = 4864
    W = _weights(rng, 64, K)
    xq, xd = oracle.quant_q8_ggml(_activations(rng, 1, K)[0])
    Wd = oracle.dequant_rows(W, K).astype(np.float64)
    xdq = xq.astype(np.float64) * np.repeat(np.array([oracle.half_to_float(int(h)) for h in xd]), 32)
    exact = Wd @ xdq
    mag = np.abs(Wd) @ np.abs(xdq)
    for order in (oracle.GGML_VEC, oracle.GGML_LLAMAFILE):
        got = oracle.q8_gemv_ggml(W, xq, xd, K, order).astype(np.float64)
        assert np.all(np.abs(got - exact) <= (K / 32 + 8) * 2.0 ** -24 * mag * 2)

"""Pins of the CPU oracle (oracle/lt_oracle.c) by checks that do not restate it.

Each function of the oracle is checked against what the mathematics or an independent
tool fixes -- numpy's IEEE float16 conversion, float64 references with ULP bounds,
exact integer arithmetic, closed-form special cases, and constructed inputs whose
correct result under the reference's declared reduction order differs from the result
of any other plausible order (so a transposed tree, a dropped term or a missing fma
fails).  The reference holds no golden vectors for this path (its gates store seeds and
shapes, not outputs), so these checks are the oracle's anchor.
"""
import numpy as np
import pytest

from llamatov_amd import q8 as hq8


def ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, np.int64(-2**31) - a, a)
    b = np.where(b < 0, np.int64(-2**31) - b, b)
    return np.abs(a - b)


# ---- fp16 conversions ----------------------------------------------------------------
def test_half_to_float_all_patterns(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.half_to_float(int(x)) for x in h], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


def test_float_to_half_rne_matches_numpy(oracle):
    rng = np.random.default_rng(3)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000).astype(np.float32),
        # exact ties between representable halves, subnormal ties, overflow edge
        (np.arange(1, 2000, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -24),
        np.array([65504, 65519.99, 65520, 65536, 1e30, -1e30, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8,
                  0.0, -0.0, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11], np.float32),
    ]).astype(np.float32)
    ref = x.astype(np.float16).view(np.uint16)
    got = np.array([oracle.float_to_half_bits(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, ref)


# ---- transcendentals: float64 references --------------------------------------------
def test_expf_within_one_ulp_of_float64(oracle):
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.uniform(-103, 88, 40000), rng.uniform(-2, 2, 20000),
                        np.linspace(-87.3, 88.7, 5001)]).astype(np.float32)
    got = np.array([oracle.expf(float(v)) for v in x], np.float32)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    normal = ref > np.float32(1.2e-38)
    assert ulp_diff(got[normal], ref[normal]).max() <= 1
    # special cases the attention mask and L = 1 rely on
    assert oracle.expf(0.0) == 1.0
    assert oracle.expf(-1e30) == 0.0
    assert oracle.expf(-2e30) == 0.0
    assert oracle.expf(100.0) == float("inf")


def test_expf_branch_free_form_equals_expf(oracle):
    """The kernels' lt_expf_sel (selects instead of branches) equals lt_expf bit for bit on
    every one of the 2^32 binary32 inputs (nans, infinities, subnormals included)."""
    assert oracle.expf_sel_mismatches(0, 1, 1 << 32) == 0


def test_sincosf_within_one_ulp_of_float64(oracle):
    rng = np.random.default_rng(12)
    x = np.concatenate([rng.uniform(-2100, 2100, 20000), rng.uniform(-4, 4, 10000)]).astype(np.float32)
    s = np.empty_like(x)
    c = np.empty_like(x)
    for i, v in enumerate(x):
        s[i], c[i] = oracle.sincosf(float(v))
    xd = x.astype(np.float64)
    sr, cr = np.sin(xd), np.cos(xd)
    # relative to the larger of |value| and 2^-20 so zeros near multiples of pi are bounded
    for got, ref in ((s, sr), (c, cr)):
        err = np.abs(got.astype(np.float64) - ref)
        tol = np.maximum(np.abs(ref), 2.0 ** -20) * 2.0 ** -23
        assert np.all(err <= tol)
    assert oracle.sincosf(0.0) == (0.0, 1.0)


def test_rsqrtf_within_one_ulp(oracle):
    rng = np.random.default_rng(13)
    x = np.exp(rng.uniform(-40, 40, 20000)).astype(np.float32)
    got = np.array([oracle.rsqrtf(float(v)) for v in x], np.float32)
    ref = (1.0 / np.sqrt(x.astype(np.float64))).astype(np.float32)
    assert ulp_diff(got, ref).max() <= 1
    assert oracle.rsqrtf(0.25) == 2.0 and oracle.rsqrtf(65536.0) == 1.0 / 256


# ---- Q8_0 quantizer ------------------------------------------------------------------
def test_quant_closed_form_properties(oracle):
    rng = np.random.default_rng(7)
    x = (2.0 * rng.standard_normal(4864)).astype(np.float32)
    xq, xd = oracle.quant_q8(x)
    d = xd.view(np.float16).astype(np.float32)
    blk = x.reshape(-1, 32)
    amax = np.abs(blk).max(axis=1)
    # d16 is the fp16 rounding of amax/127 (IEEE float32 division)
    assert np.array_equal(xd, (amax / np.float32(127)).astype(np.float16).view(np.uint16))
    # every element reconstructs to within half a step (no clamping below 127.5 steps)
    err = np.abs(blk - xq.reshape(-1, 32).astype(np.float32) * d[:, None])
    assert np.all(err <= d[:, None] * 0.5000001)
    # the largest element of each block lands on +-127 or +-126 (scale rounding) and never beyond
    assert np.all(np.abs(xq) <= 127)
    top = np.abs(xq.reshape(-1, 32)).max(axis=1)
    assert np.all(top >= 126)


def test_quant_special_cases(oracle):
    x = np.zeros(96, np.float32)
    # block 1: scale exactly 1.0 (amax 127) with exact .5 ties -> round half to even
    x[32:64] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5] + [0.0] * 24
    # block 2: a value beyond 127.5 steps cannot occur (amax defines the scale), but the
    # smallest normal fp16 scale and subnormal scales must still encode exactly
    x[64:96] = np.float32(127 * 2.0 ** -20) * np.linspace(-1, 1, 32, dtype=np.float32)
    xq, xd = oracle.quant_q8(x)
    assert xd[0] == 0x3C00 and np.all(xq[:32] == 0)          # all-zero block: d = 1.0
    assert xd[1] == 0x3C00
    assert list(xq[32:40]) == [127, 2, 4, -2, -4, 0, 2, 0]
    assert xd[2] == np.float32(2.0 ** -20).astype(np.float16).view(np.uint16)


def test_weight_quantizer_host_matches_oracle(oracle):
    rng = np.random.default_rng(5)
    W = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    W[3, :32] = 0.0
    assert np.array_equal(hq8.quantize_rows(W), oracle.quantize_rows(W))
    # residency round trip: dequant -> requant reproduces the blocks (all-zero block aside)
    B = oracle.quantize_rows(W)
    R = oracle.quantize_rows(oracle.dequant_rows(B, 256))
    assert np.array_equal(B, R)


# ---- block dots and GEMV ------------------------------------------------------------
def _rand_blocks(rng, N, K, dstd=0.1):
    q = rng.integers(-127, 128, size=(N, K), dtype=np.int64).astype(np.int8)
    d = (rng.standard_normal((N, K // 32)) * dstd).astype(np.float16).view(np.uint16)
    return hq8.join_blocks(q, d), q, d


def test_block_dots_exact(oracle):
    rng = np.random.default_rng(8)
    K = 256
    W, q, _ = _rand_blocks(rng, 64, K)
    xq = rng.integers(-127, 128, size=K, dtype=np.int64).astype(np.int8)
    got = oracle.block_dots(W, xq, K)
    ref = (q.astype(np.int64).reshape(64, -1, 32) * xq.astype(np.int64).reshape(-1, 32)).sum(axis=2)
    assert np.array_equal(got, ref)
    # extremes: all -127 x -127 -> 32*16129
    Wx = hq8.join_blocks(np.full((1, 32), -127, np.int8), np.array([[0x3C00]], np.uint16))
    assert oracle.block_dots(Wx, np.full(32, -127, np.int8), 32)[0, 0] == 32 * 16129


def test_gemv_float64_bound(oracle):
    rng = np.random.default_rng(8)
    for (N, K) in ((896, 4864), (64, 256)):
        W, q, d = _rand_blocks(rng, N, K)
        xq = rng.integers(-127, 128, size=K, dtype=np.int64).astype(np.int8)
        xd = (rng.standard_normal(K // 32) * 0.1).astype(np.float16).view(np.uint16)
        y = oracle.q8_gemv(W, xq, xd, K)
        isum = (q.astype(np.int64).reshape(N, -1, 32) * xq.astype(np.int64).reshape(-1, 32)).sum(2)
        terms = d.view(np.float16).astype(np.float64) * xd.view(np.float16).astype(np.float64) * isum
        exact = terms.sum(axis=1)
        bound = np.abs(terms).sum(axis=1) * (K // 32 + 6) * 2.0 ** -24
        assert np.all(np.abs(y.astype(np.float64) - exact) <= bound)


def _one_block_row(val_isum, K, lanes_vals):
    """Row whose block b has wd = 1, xd = 1 and isum chosen by lanes_vals {b: isum}."""
    nb = K // 32
    q = np.zeros((1, K), np.int8)
    xq = np.zeros(K, np.int8)
    d = np.full((1, nb), 0x3C00, np.uint16)
    xd = np.full(nb, 0x3C00, np.uint16)
    for b, v in lanes_vals.items():
        # realize isum = v with w = v / 127^.. : use scale to carry magnitude
        q[0, b * 32] = 1
        xq[b * 32] = 1
        d[0, b] = np.float16(v).view(np.uint16)
    return hq8.join_blocks(q, d), xq, xd


def test_gemv_canonical_order_is_pinned(oracle):
    K = 64 * 32
    # lane 0 holds blocks 0 and 32; lane 16 holds block 16.  Canonical:
    # lane0 = fma(.., 16384, 0) then fma(.., -16384, 16384) = 0; lane16 = 2^-10; result 2^-10.
    # A block-sequential sum gives (16384 + 2^-10) - 16384 with the 2^-10 lost to the tie
    # (ulp(16384) = 2^-9, round half to even) -> 0.
    W, xq, xd = _one_block_row(None, K, {0: 16384.0, 32: -16384.0, 16: 2.0 ** -10})
    y = oracle.q8_gemv(W, xq, xd, K)
    assert y[0] == np.float32(2.0 ** -10)
    # tree pairing s = 16 then 8: lane0 = 2^13, lane16 = 2^-11*... choose values at the
    # float32 tie: 2^13 + 2^-11 is a tie (2^13 has ulp 2^-10); pairs (0,16) then (0,8) each
    # round to even -> 2^13; summing lanes 8 and 16 first would give 2^13 + 2^-10.
    W, xq, xd = _one_block_row(None, K, {0: 8192.0, 16: 2.0 ** -11, 8: 2.0 ** -11})
    y = oracle.q8_gemv(W, xq, xd, K)
    assert y[0] == np.float32(8192.0)
    # the residual epilogue is one fp32 add after the tree
    r = np.array([1.0], np.float32)
    assert oracle.q8_gemv(W, xq, xd, K, resid=r)[0] == np.float32(8192.0) + np.float32(1.0)


def test_gemv_fma_single_rounding(oracle):
    # nb = 1: y = fma(wd*xd, isum, 0) = round(wd*xd*isum) (exact product in float64)
    rng = np.random.default_rng(21)
    for _ in range(200):
        W, q, d = _rand_blocks(rng, 1, 32)
        xq = rng.integers(-127, 128, size=32, dtype=np.int64).astype(np.int8)
        xd = (rng.standard_normal(1) * 0.1).astype(np.float16).view(np.uint16)
        isum = int((q[0].astype(np.int64) * xq.astype(np.int64)).sum())
        exact = float(d.view(np.float16)[0, 0]) * float(xd.view(np.float16)[0]) * isum
        assert oracle.q8_gemv(W, xq, xd, 32)[0] == np.float32(exact)


# ---- RMSNorm -------------------------------------------------------------------------
def test_rmsnorm_closed_form_and_order(oracle):
    w = np.linspace(0.5, 1.5, 896).astype(np.float32)
    y = oracle.rmsnorm(np.full(896, 0.5, np.float32), w, 0.0)
    assert np.array_equal(y, w)  # ss = 224 exactly, inv = rsqrt(0.25) = 2
    # tree pairing: x[0]^2 = 2^24, x[128]^2 = x[64]^2 = 1.  Canonical: p0 += p128 (tie -> 2^24),
    # p0 += p64 (tie -> 2^24): mean 65536, inv exactly 1/256.  An order that adds the two
    # ones first gives 2^24 + 2 and a different inv.
    x = np.zeros(256, np.float32)
    x[0], x[128], x[64] = 4096.0, 1.0, 1.0
    y = oracle.rmsnorm(x, np.ones(256, np.float32), 0.0)
    assert y[0] == np.float32(16.0) and y[128] == np.float32(1.0 / 256)
    # and the converse: ones at 64 and 192 meet first in the tree (s = 128) -> 2^24 + 2, where a
    # sequential left fold would lose both to ties and give 2^24.
    x = np.zeros(256, np.float32)
    x[0], x[64], x[192] = 4096.0, 1.0, 1.0
    y = oracle.rmsnorm(x, np.ones(256, np.float32), 0.0)
    inv_tree = np.float32(1.0 / np.sqrt(np.float64(np.float32((2.0 ** 24 + 2) / 256))))
    inv_seq = np.float32(1.0 / 256)
    assert inv_tree != inv_seq
    assert y[0] == np.float32(4096.0) * inv_tree


def test_rmsnorm_float64_bound(oracle):
    rng = np.random.default_rng(7)
    x = (2.0 * rng.standard_normal(896)).astype(np.float32)
    w = (0.5 * rng.standard_normal(896) + 1.0).astype(np.float32)
    y = oracle.rmsnorm(x, w, 1e-6)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * w
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 4e-7 + 1e-30)


# ---- RoPE ----------------------------------------------------------------------------
def test_rope_special_cases_and_bound(oracle):
    rng = np.random.default_rng(4)
    hd, nheads = 64, 16
    x = rng.standard_normal(nheads * hd).astype(np.float32)
    assert np.array_equal(oracle.rope(x, 0, nheads, hd, 1e6), x)       # pos 0: identity
    f = oracle.rope_freqs(hd, 1e6)
    assert f[0] == 1.0
    ref_f = np.float64(1e6) ** (-(2.0 * np.arange(hd // 2, dtype=np.float32)) / np.float32(hd)).astype(np.float64)
    assert ulp_diff(f, ref_f.astype(np.float32)).max() == 0
    for pos in (1, 17, 1023):
        y = oracle.rope(x, pos, nheads, hd, 1e6)
        ang = (np.float32(pos) * f).astype(np.float64)
        c, s = np.cos(ang), np.sin(ang)
        xr = x.reshape(nheads, 2, hd // 2).astype(np.float64)
        ref = np.stack([xr[:, 0] * c - xr[:, 1] * s, xr[:, 0] * s + xr[:, 1] * c], axis=1).reshape(-1)
        assert np.all(np.abs(y - ref) <= 4e-7 * (np.abs(xr).max() + 1e-30))


# ---- attention -----------------------------------------------------------------------
def _kv(rng, L, nkv, hd, f16):
    k = rng.standard_normal((L, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((L, nkv * hd)).astype(np.float32)
    if f16:
        return k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
    return k, v


def test_attention_L1_is_V0(oracle):
    rng = np.random.default_rng(1)
    nh, nkv, hd = 14, 2, 64
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k, v = _kv(rng, 4, nkv, hd, False)
    out = oracle.attn_decode(q, k, v, 1, nh, nkv, hd, 0.125, False)
    exp = np.concatenate([v[0, (h // 7) * hd:(h // 7 + 1) * hd] for h in range(nh)])
    assert np.array_equal(out, exp)


@pytest.mark.parametrize("f16", [False, True])
def test_attention_float64_bound_and_split_identity(oracle, f16):
    rng = np.random.default_rng(2)
    nh, nkv, hd, L = 8, 2, 64, 300
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k, v = _kv(rng, L, nkv, hd, f16)
    kf = k.view(np.float16).astype(np.float64) if f16 else k.astype(np.float64)
    vf = v.view(np.float16).astype(np.float64) if f16 else v.astype(np.float64)
    scale = 0.125
    out1 = oracle.attn_decode(q, k, v, L, nh, nkv, hd, scale, f16, nsplit=1)
    for h in range(nh):
        g = h // (nh // nkv)
        s = kf[:, g * hd:(g + 1) * hd] @ q[h * hd:(h + 1) * hd].astype(np.float64) * scale
        p = np.exp(s - s.max())
        ref = (p @ vf[:, g * hd:(g + 1) * hd]) / p.sum()
        assert np.all(np.abs(out1[h * hd:(h + 1) * hd] - ref) <= 5e-6)
    # split-K with a single split is the single pass, bit for bit
    assert np.array_equal(oracle.attn_decode(q, k, v, L, nh, nkv, hd, scale, f16, nsplit=1), out1)
    for S in (2, 4, 7, 64):
        outS = oracle.attn_decode(q, k, v, L, nh, nkv, hd, scale, f16, nsplit=S)
        assert np.all(np.abs(outS - out1) <= 2e-6)


# ---- argmax --------------------------------------------------------------------------
def test_argmax_ties_lowest_index(oracle):
    rng = np.random.default_rng(9)
    x = rng.standard_normal(151936).astype(np.float32)
    assert oracle.argmax(x) == int(np.argmax(x))
    x[1000] = x[50000] = np.float32(100.0)
    assert oracle.argmax(x) == 1000


def test_attention_z_fold_order_is_pinned(oracle):
    """Z is a 64-lane strided fold plus a pairwise tree (bpd/lib/dev_residency.py:1968-2008),
    not a sequential sum.  Scores 0 at t = 0 and -17.5 elsewhere give e_0 = 1 and 63 values
    e ~ 2.5e-8, each below half an ulp of 1: a sequential sum drops every one of them (Z = 1),
    while the tree first adds them among themselves and its last levels add 4e..32e to lane
    0 (Z ~ 1 + 60e).  With V = 1 at t = 0 (dim 0) and 0 elsewhere, out = 1 / Z."""
    hd, L = 64, 64
    q = np.zeros(hd, np.float32)
    q[0] = 8.0
    k = np.zeros((L, hd), np.float32)
    k[1:, 0] = -17.5                  # s_t = 8 * k * 0.125 = k
    v = np.zeros((L, hd), np.float32)
    v[0, 0] = 1.0
    out = oracle.attn_decode(q, k, v, L, 1, 1, hd, 0.125, False)
    e = np.float32(oracle.expf(-17.5))
    assert np.float32(1.0) + e == np.float32(1.0)          # each alone is lost against 1
    # the declared tree, evaluated by hand: lane t (t < 64) holds e_t; s = 32, 16, ..., 1
    lanes = [np.float32(1.0)] + [e] * 63
    s = 32
    while s >= 1:
        for t in range(s):
            lanes[t] = np.float32(lanes[t] + lanes[t + s])
        s //= 2
    z_tree = lanes[0]
    assert z_tree > np.float32(1.0)
    assert out[0] == np.float32(np.float32(1.0) / z_tree)
    assert out[0] != np.float32(1.0)                        # the sequential-sum result
    assert np.all(out[1:] == 0.0)

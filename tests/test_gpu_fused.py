"""Parity of the fused decode-step launchers (lt_fused.hip) with the oracle's per-op chain,
through the C ABI.  Every fused launcher must reproduce the chain bit for bit."""
import ctypes

import numpy as np
import pytest

from llamatov_amd import _lib
from llamatov_amd import engine as dr
from llamatov_amd import model as M
from llamatov_amd import q8 as hq8
from llamatov_amd._lib import LT_KV_F16, LT_KV_F32, call

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[gpu-case] {msg}", flush=True)


def up(a):
    return dr.DevTensor.from_host(np.ascontiguousarray(a))


def empty(shape, dt):
    return dr.DevTensor.empty(shape, dt)


def assert_bitexact(got, exp, what):
    got, exp = np.asarray(got), np.asarray(exp)
    assert got.shape == exp.shape, (what, got.shape, exp.shape)
    g = got.view(np.uint32) if got.dtype == np.float32 else got
    e = exp.view(np.uint32) if exp.dtype == np.float32 else exp
    bad = np.flatnonzero(g.reshape(-1) != e.reshape(-1))
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]}: {got.reshape(-1)[bad[:5]]} vs {exp.reshape(-1)[bad[:5]]}"


def rand_weight(rng, N, K):
    return hq8.quantize_rows((rng.standard_normal((N, K)) * 0.02).astype(np.float32))


@pytest.mark.parametrize("N,K,bias", [(1152, 896, True), (896, 896, False), (6144, 4096, False),
                                      (40, 4864, True), (151936, 896, False), (24, 14336, True),
                                      (100003, 896, True), (50001, 640, False), (70001, 1024, True),
                                      (20003, 896, True), (30000, 512, False), (17000, 1024, False),
                                      (128256, 4096, False)])
def test_q8_gemv_rms(gpu, oracle, N, K, bias):
    case(f"gemv_rms N={N} K={K} bias={bias}")
    rng = np.random.default_rng(21)
    W = rand_weight(rng, N, K)
    x = (2.0 * rng.standard_normal(K)).astype(np.float32)
    nw = (0.5 * rng.standard_normal(K) + 1.0).astype(np.float32)
    b = (rng.standard_normal(N) * 0.02).astype(np.float32) if bias else None
    h = oracle.rmsnorm(x, nw, 1e-6)
    xq, xd = oracle.quant_q8(h)
    exp = oracle.q8_gemv(W, xq, xd, K, b)
    y = empty((N,), np.float32)
    call("lt_q8_gemv_rms", gpu.handle, up(x).vp, up(nw).vp, ctypes.c_float(1e-6), up(W).vp,
         up(b).vp if bias else None, y.vp, N, K)
    assert_bitexact(y.to_host(), exp, "gemv_rms")


def test_q8_gemv_embed_rms(gpu, oracle):
    case("gemv_embed_rms")
    rng = np.random.default_rng(22)
    V, E, N = 300, 896, 1152
    emb = rand_weight(rng, V, E)
    W = rand_weight(rng, N, E)
    nw = (0.5 * rng.standard_normal(E) + 1.0).astype(np.float32)
    b = (rng.standard_normal(N) * 0.02).astype(np.float32)
    demb, dW, dnw, db = up(emb), up(W), up(nw), up(b)
    xo, y, err = empty((E,), np.float32), empty((N,), np.float32), up(np.zeros(1, np.int32))
    for tok in (0, 157, V - 1):
        x = oracle.embed_row(emb, tok, E)
        xq, xd = oracle.quant_q8(oracle.rmsnorm(x, nw, 1e-6))
        call("lt_q8_gemv_embed_rms", gpu.handle, demb.vp, up(np.array([tok], np.int32)).vp, V, xo.vp, err.vp,
             dnw.vp, ctypes.c_float(1e-6), dW.vp, db.vp, y.vp, N, E)
        assert_bitexact(xo.to_host(), x, "embedding row")
        assert_bitexact(y.to_host(), oracle.q8_gemv(W, xq, xd, E, b), f"embed gemv tok={tok}")
    assert err.to_host()[0] == 0
    call("lt_q8_gemv_embed_rms", gpu.handle, demb.vp, up(np.array([V], np.int32)).vp, V, xo.vp, err.vp,
         dnw.vp, ctypes.c_float(1e-6), dW.vp, db.vp, y.vp, N, E)
    assert err.to_host()[0] == 1 and not np.any(xo.to_host())


@pytest.mark.parametrize("N,K", [(896, 4864), (4096, 14336), (64, 256), (896, 896)])
def test_q8_gemv_quant(gpu, oracle, N, K):
    case(f"gemv_quant N={N} K={K}")
    rng = np.random.default_rng(23)
    W = rand_weight(rng, N, K)
    x = rng.standard_normal(K).astype(np.float32)
    r = rng.standard_normal(N).astype(np.float32)
    xq, xd = oracle.quant_q8(x)
    y = empty((N,), np.float32)
    call("lt_q8_gemv_quant", gpu.handle, up(x).vp, up(W).vp, up(r).vp, y.vp, N, K)
    assert_bitexact(y.to_host(), oracle.q8_gemv(W, xq, xd, K, r), "gemv_quant")


@pytest.mark.parametrize("F,K", [(4864, 896), (14336, 4096), (64, 128)])
def test_q8_gemv_rms_silu(gpu, oracle, F, K):
    case(f"gemv_rms_silu F={F} K={K}")
    rng = np.random.default_rng(24)
    Wg, Wu = rand_weight(rng, F, K), rand_weight(rng, F, K)
    x = (2.0 * rng.standard_normal(K)).astype(np.float32)
    nw = (0.5 * rng.standard_normal(K) + 1.0).astype(np.float32)
    xq, xd = oracle.quant_q8(oracle.rmsnorm(x, nw, 1e-5))
    g = oracle.q8_gemv(Wg, xq, xd, K)
    u = oracle.q8_gemv(Wu, xq, xd, K)
    vq, vd = empty((F,), np.int8), empty((F // 32,), np.uint16)
    call("lt_q8_gemv_rms_silu", gpu.handle, up(x).vp, up(nw).vp, ctypes.c_float(1e-5),
         up(M.interleave_gateup(Wg, Wu)).vp, vq.vp, vd.vp, F, K)
    # the quantized SiLU*up vector is what the down GEMV consumes
    eq, ed = oracle.silu_mul_quant(g, u)
    assert_bitexact(vq.to_host(), eq, "silu*up quants")
    assert_bitexact(vd.to_host(), ed, "silu*up scales")


@pytest.mark.parametrize("F,K", [(4864, 896), (14336, 4096), (64, 128), (12, 96), (16384, 896), (20000, 512),
                                 (3000, 4864)])
def test_q8_gemv_rms_swiglu(gpu, oracle, F, K):
    """gate|up GEMV with the fp32 SiLU(g)*u epilogue (adjacent half-waves hold the gate and
    up rows of one output), then the down GEMV's quantizing prologue: the same quants as the
    quantizing epilogue, and the down GEMV's output equal to the oracle's."""
    case(f"gemv_rms_swiglu F={F} K={K}")
    rng = np.random.default_rng(25)
    Wg, Wu = rand_weight(rng, F, K), rand_weight(rng, F, K)
    x = (2.0 * rng.standard_normal(K)).astype(np.float32)
    nw = (0.5 * rng.standard_normal(K) + 1.0).astype(np.float32)
    xq, xd = oracle.quant_q8(oracle.rmsnorm(x, nw, 1e-6))
    g = oracle.q8_gemv(Wg, xq, xd, K)
    u = oracle.q8_gemv(Wu, xq, xd, K)
    v = empty((F,), np.float32)
    call("lt_q8_gemv_rms_swiglu", gpu.handle, up(x).vp, up(nw).vp, ctypes.c_float(1e-6),
         up(M.interleave_gateup(Wg, Wu)).vp, v.vp, F, K)
    assert_bitexact(v.to_host(), oracle.silu_mul(g, u), "silu*up")
    if F % 32 == 0 and F <= 16384:
        N = 256
        Wd = rand_weight(rng, N, F)
        r = rng.standard_normal(N).astype(np.float32)
        y = empty((N,), np.float32)
        call("lt_q8_gemv_quant", gpu.handle, v.vp, up(Wd).vp, up(r).vp, y.vp, N, F)
        sq, sd = oracle.silu_mul_quant(g, u)
        assert_bitexact(y.to_host(), oracle.q8_gemv(Wd, sq, sd, F, r), "down after swiglu")


def test_q8_gemv_attn_out(gpu, oracle):
    """Single-split O launcher on a quantized attention output (split partials come from
    lt_attn_step and are covered by test_attn_step_then_out)."""
    nsplit = 1
    case("gemv_attn_out nsplit=1")
    rng = np.random.default_rng(25)
    nh, nkv, hd, E, maxt, L = 14, 2, 64, 896, 64, 37
    W = rand_weight(rng, E, nh * hd)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    kc = rng.standard_normal((maxt, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((maxt, nkv * hd)).astype(np.float32)
    r = rng.standard_normal(E).astype(np.float32)
    att = oracle.attn_decode(q, kc, vc, L, nh, nkv, hd, 0.125, False, nsplit)
    xq, xd = oracle.quant_q8(att)
    exp = oracle.q8_gemv(W, xq, xd, nh * hd, r)
    dlen = up(np.array([L], np.int32))
    y = empty((E,), np.float32)
    call("lt_q8_gemv_attn_out", gpu.handle, up(xq).vp, up(xd).vp, None, 0, nsplit, nh, hd, up(W).vp, up(r).vp,
         y.vp, E, nh * hd, dlen.vp, maxt)
    assert_bitexact(y.to_host(), exp, "attn_out")
    assert int(dlen.to_host()[0]) == L + 1


@pytest.mark.parametrize("kv_dtype", [LT_KV_F32, LT_KV_F16])
@pytest.mark.parametrize("nsplit", [1, 3, 16])
@pytest.mark.parametrize("geom", [(14, 2, 64, 1e6), (32, 8, 128, 5e5)])
def test_attn_step_then_out(gpu, oracle, kv_dtype, nsplit, geom):
    """RoPE + append + attention (+ the split merge launch) against the oracle's
    rope -> append -> attention -> quant -> GEMV chain, over a length sweep; the new cache
    row and the length bump are checked too.  With nsplit > 1 the O launcher's own merge of
    the same partials gives the same O projection."""
    nh, nkv, hd, theta = geom
    f16 = kv_dtype == LT_KV_F16
    rng = np.random.default_rng(26)
    maxt, E = 96, 256
    width = nkv * hd
    W = rand_weight(rng, E, nh * hd)
    freqs = oracle.rope_freqs(hd, theta)
    dfreq = up(freqs)
    dW = up(W)
    dt = np.uint16 if f16 else np.float32
    kc_host = np.zeros((maxt, width), dt)
    vc_host = np.zeros((maxt, width), dt)
    base_k = rng.standard_normal((maxt, width)).astype(np.float32)
    base_v = rng.standard_normal((maxt, width)).astype(np.float32)
    ws_n = _lib.raw("lt_attn_workspace_size")(1, nh, hd, nsplit)
    ws = dr.DevTensor.zeros((max(ws_n, 16),), np.uint8, gpu)
    scale = float(hd ** -0.5)
    for L in (0, 1, 2, 40, maxt - 1):
        case(f"attn_step nh={nh} hd={hd} kv={kv_dtype} nsplit={nsplit} L={L}")
        # cache rows < L hold earlier tokens; rows >= L hold poison the kernel must not read
        kc_host[:] = (base_k.astype(np.float16).view(np.uint16) if f16 else base_k)
        vc_host[:] = (base_v.astype(np.float16).view(np.uint16) if f16 else base_v)
        if not f16:
            kc_host[L:] = np.nan
            vc_host[L:] = np.nan
        else:
            kc_host[L:] = 0x7E00
            vc_host[L:] = 0x7E00
        qkv = rng.standard_normal(nh * hd + 2 * width).astype(np.float32)
        # oracle chain
        roped = oracle.rope(qkv[: (nh + nkv) * hd], L, nh + nkv, hd, theta)
        knew = roped[nh * hd:]
        vnew = qkv[(nh + nkv) * hd:]
        ek, ev = kc_host.copy(), vc_host.copy()
        if f16:
            ek[L] = knew.astype(np.float16).view(np.uint16)
            ev[L] = vnew.astype(np.float16).view(np.uint16)
        else:
            ek[L] = knew
            ev[L] = vnew
        att = oracle.attn_decode(roped[: nh * hd], ek, ev, L + 1, nh, nkv, hd, scale, f16, nsplit)
        xq, xd = oracle.quant_q8(att)
        r = rng.standard_normal(E).astype(np.float32)
        exp = oracle.q8_gemv(W, xq, xd, nh * hd, r)
        # device
        dk, dv = up(kc_host), up(vc_host)
        dlen = up(np.array([L], np.int32))
        datt = empty((nh * hd,), np.float32)
        aq, ad = empty((nh * hd,), np.int8), empty((nh * hd // 32,), np.uint16)
        call("lt_attn_step", gpu.handle, up(qkv).vp, dfreq.vp, dk.vp, dv.vp, dlen.vp, datt.vp, aq.vp, ad.vp,
             nh, nkv, hd, ctypes.c_float(scale), maxt, nsplit, kv_dtype, ws.vp, ws.nbytes)
        assert_bitexact(datt.to_host(), att, "attention output")
        assert_bitexact(aq.to_host(), xq, "attention quants")
        assert_bitexact(ad.to_host(), xd, "attention scales")
        assert int(dlen.to_host()[0]) == L
        if nsplit > 1:
            y2 = empty((E,), np.float32)
            call("lt_q8_gemv_attn_out", gpu.handle, aq.vp, ad.vp, ws.vp, ws.nbytes, nsplit, nh, hd, dW.vp,
                 up(r).vp, y2.vp, E, nh * hd, None, maxt)
            assert_bitexact(y2.to_host(), exp, f"O after the launcher's own merge L={L}")
        y = empty((E,), np.float32)
        call("lt_q8_gemv_attn_out", gpu.handle, aq.vp, ad.vp, None, 0, 1, nh, hd, dW.vp, up(r).vp,
             y.vp, E, nh * hd, dlen.vp, maxt)
        assert_bitexact(y.to_host(), exp, f"O after attention L={L}")
        assert int(dlen.to_host()[0]) == L + 1
        gk, gv = dk.to_host(), dv.to_host()
        assert np.array_equal(gk[L].view(np.uint32 if not f16 else np.uint16), ek[L].view(np.uint32 if not f16 else np.uint16))
        assert np.array_equal(gv[L].view(np.uint32 if not f16 else np.uint16), ev[L].view(np.uint32 if not f16 else np.uint16))
        assert np.array_equal(gk[:L].view(np.uint8), kc_host[:L].view(np.uint8))


@pytest.mark.parametrize("nsplit", [1, 3, 16])
@pytest.mark.parametrize("nh,nkv,hd", [(14, 2, 64), (8, 1, 64), (32, 8, 128), (16, 2, 128)])
def test_attn_step_long_context(gpu, oracle, nsplit, nh, nkv, hd):
    """The fp16 step with 64 dims streams V in 8-row chunks (16 in flight) and requests its
    64-position K rounds two ahead; with 128 dims V runs through a ring of rows: lengths around
    one V ring (128 rows at 64 dims) and around one to four K rounds, ragged chunk tails,
    refills up to the cache's end, splits of a few rows, with poison past the new row."""
    theta, maxt = 1e6, 1024
    rng = np.random.default_rng(29)
    width = nkv * hd
    freqs = up(oracle.rope_freqs(hd, theta))
    base_k = rng.standard_normal((maxt, width)).astype(np.float16).view(np.uint16)
    base_v = rng.standard_normal((maxt, width)).astype(np.float16).view(np.uint16)
    ws_n = _lib.raw("lt_attn_workspace_size")(1, nh, hd, nsplit)
    ws = dr.DevTensor.zeros((max(ws_n, 16),), np.uint8, gpu)
    scale = float(hd ** -0.5)
    for L in (0, 5, 63, 64, 65, 95, 96, 97, 127, 128, 129, 190, 191, 192, 193, 200, 255, 256, 257, 383, 577,
              1023):
        case(f"attn_step long nh={nh} nkv={nkv} nsplit={nsplit} L={L}")
        kc, vc = base_k.copy(), base_v.copy()
        kc[L:] = 0x7E00
        vc[L:] = 0x7E00
        qkv = rng.standard_normal(nh * hd + 2 * width).astype(np.float32)
        roped = oracle.rope(qkv[: (nh + nkv) * hd], L, nh + nkv, hd, theta)
        ek, ev = kc.copy(), vc.copy()
        ek[L] = roped[nh * hd:].astype(np.float16).view(np.uint16)
        ev[L] = qkv[(nh + nkv) * hd:].astype(np.float16).view(np.uint16)
        att = oracle.attn_decode(roped[: nh * hd], ek, ev, L + 1, nh, nkv, hd, scale, True, nsplit)
        xq, xd = oracle.quant_q8(att)
        dk, dv = up(kc), up(vc)
        datt = empty((nh * hd,), np.float32)
        aq, ad = empty((nh * hd,), np.int8), empty((nh * hd // 32,), np.uint16)
        call("lt_attn_step", gpu.handle, up(qkv).vp, freqs.vp, dk.vp, dv.vp, up(np.array([L], np.int32)).vp,
             datt.vp, aq.vp, ad.vp, nh, nkv, hd, ctypes.c_float(scale), maxt, nsplit, LT_KV_F16, ws.vp, ws.nbytes)
        assert_bitexact(datt.to_host(), att, f"attention output L={L}")
        assert_bitexact(aq.to_host(), xq, f"attention quants L={L}")
        assert_bitexact(ad.to_host(), xd, f"attention scales L={L}")
        assert np.array_equal(dv.to_host()[L], ev[L]) and np.array_equal(dk.to_host()[L], ek[L])


def test_q8_gemv_rms_argmax(gpu, oracle):
    rng = np.random.default_rng(27)
    N, K = 151936, 896
    W = rand_weight(rng, N, K)
    x = (2.0 * rng.standard_normal(K)).astype(np.float32)
    nw = np.ones(K, np.float32)
    xq, xd = oracle.quant_q8(oracle.rmsnorm(x, nw, 1e-6))
    exp = oracle.q8_gemv(W, xq, xd, K)
    dW, dx, dnw = up(W), up(x), up(nw)
    logits = empty((N,), np.float32)
    out = empty((1,), np.int32)
    hist = up(np.full(8, -1, np.int32))
    cnt = up(np.zeros(1, np.int32))
    ws = empty((_lib.raw("lt_q8_gemv_argmax_workspace_size")(N),), np.uint8)
    case("gemv_rms_argmax vocab")
    call("lt_q8_gemv_rms_argmax", gpu.handle, dx.vp, dnw.vp, ctypes.c_float(1e-6), dW.vp, logits.vp, N, K,
         out.vp, hist.vp, cnt.vp, 8, ws.vp, ws.nbytes)
    assert_bitexact(logits.to_host(), exp, "logits")
    assert int(out.to_host()[0]) == oracle.argmax(exp)
    assert hist.to_host()[0] == oracle.argmax(exp) and cnt.to_host()[0] == 1
    # planted ties across workgroups: duplicate the winning row at a lower and a higher index
    best = oracle.argmax(exp)
    for lo, hi in ((5, best), (best, N - 1), (0, N - 1)):
        W2 = W.copy()
        W2[lo] = W[best]
        W2[hi] = W[best]
        e2 = oracle.q8_gemv(W2, xq, xd, K)
        call("lt_q8_gemv_rms_argmax", gpu.handle, dx.vp, dnw.vp, ctypes.c_float(1e-6), up(W2).vp, logits.vp, N, K,
             out.vp, None, None, 0, ws.vp, ws.nbytes)
        assert int(out.to_host()[0]) == oracle.argmax(e2) == min(lo, hi, oracle.argmax(e2))


# ---- the four-launch step's launchers ---------------------------------------------------
@pytest.mark.parametrize("nh,nkv,hd,E", [(14, 2, 64, 896), (32, 8, 128, 4096), (4, 2, 32, 128), (8, 1, 64, 512)])
@pytest.mark.parametrize("kv_dtype", [LT_KV_F16, LT_KV_F32])
@pytest.mark.parametrize("embed", [False, True])
def test_q8_gemv_rms_rope_kv(gpu, oracle, nh, nkv, hd, E, kv_dtype, embed):
    """QKV GEMV + bias, RoPE of q and k at position *len, k and v into the caches at row
    *len: the oracle's rms -> quant -> gemv(+bias) -> rope -> append, bit for bit."""
    case(f"rms_rope_kv nh={nh} nkv={nkv} hd={hd} E={E} kv={kv_dtype} embed={embed}")
    rng = np.random.default_rng(nh * hd + E)
    f16 = kv_dtype == LT_KV_F16
    N = (nh + 2 * nkv) * hd
    W = rand_weight(rng, N, E)
    bias = (rng.standard_normal(N) * 0.5).astype(np.float32) if nh != 8 else None
    nw = (0.5 * rng.standard_normal(E) + 1.0).astype(np.float32)
    theta, eps, maxt, pos = 1e6, 1e-6, 64, 37
    emb = rand_weight(rng, 50, E)
    tok = 13
    x = oracle.embed_row(emb, tok, E) if embed else (2.0 * rng.standard_normal(E)).astype(np.float32)
    xq, xd = oracle.quant_q8(oracle.rmsnorm(x, nw, eps))
    y = oracle.q8_gemv(W, xq, xd, E, bias)
    qk = oracle.rope(y[:(nh + nkv) * hd], pos, nh + nkv, hd, theta)
    exp = np.concatenate([qk, y[(nh + nkv) * hd:]])
    width = nkv * hd
    kc0 = rng.standard_normal((maxt, width), dtype=np.float32)
    vc0 = rng.standard_normal((maxt, width), dtype=np.float32)
    if f16:
        kc0, vc0 = kc0.astype(np.float16).view(np.uint16), vc0.astype(np.float16).view(np.uint16)
    dk, dv, dlen = up(kc0), up(vc0), up(np.array([pos], np.int32))
    out, xo, err = empty((N,), np.float32), empty((E,), np.float32), up(np.zeros(1, np.int32))
    freqs = up(dr.rope_freqs(hd, theta))
    call("lt_q8_gemv_rms_rope_kv", gpu.handle, None if embed else up(x).vp, up(emb).vp if embed else None,
         up(np.array([tok], np.int32)).vp if embed else None, 50, xo.vp if embed else None, err.vp, up(nw).vp,
         ctypes.c_float(eps), up(W).vp, up(bias).vp if bias is not None else None, out.vp, E, freqs.vp,
         dk.vp, dv.vp, dlen.vp, nh, nkv, hd, maxt, kv_dtype)
    assert_bitexact(out.to_host(), exp, "qkv")
    ek, ev = kc0.copy(), vc0.copy()
    krow, vrow = exp[nh * hd:(nh + nkv) * hd], exp[(nh + nkv) * hd:]
    ek[pos] = krow.astype(np.float16).view(np.uint16) if f16 else krow
    ev[pos] = vrow.astype(np.float16).view(np.uint16) if f16 else vrow
    assert np.array_equal(dk.to_host(), ek) and np.array_equal(dv.to_host(), ev)
    assert dlen.to_host()[0] == pos
    if embed:
        assert_bitexact(xo.to_host(), x, "embedding row")


@pytest.mark.parametrize("nh,nkv", [(14, 2), (8, 8), (10, 2), (4, 1), (12, 4)])
@pytest.mark.parametrize("kv_dtype", [LT_KV_F16, LT_KV_F32])
def test_q8_gemv_attn_o(gpu, oracle, nh, nkv, kv_dtype):
    """Attention over *len + 1 rows recomputed in the O GEMV's prologue: the oracle's masked
    attention -> quant -> O GEMV + residual, bit for bit, at lengths across the staging,
    lane-fold and 8-row boundaries up to the launch's limit, NaN past the length; past the
    limit the rows come back NaN."""
    hd, maxt, E = 64, 1024, 768
    f16 = kv_dtype == LT_KV_F16
    maxL = _lib.raw("lt_attn_o_max_len")(nh, nkv, hd, kv_dtype)
    assert maxL >= 32
    rng = np.random.default_rng(nh * 10 + nkv)
    K = nh * hd
    W = rand_weight(rng, E, K)
    dW = up(W)
    r = rng.standard_normal(E).astype(np.float32)
    dr_ = up(r)
    scale = float(hd ** -0.5)
    lens = sorted({L for L in (1, 2, 7, 8, 9, 63, 64, 65, 127, 128, 129, 200, maxL - 1, maxL) if 1 <= L <= maxL})
    for L in lens + [maxL + 1]:
        case(f"attn_o nh={nh} nkv={nkv} kv={kv_dtype} L={L} (max {maxL})")
        q = rng.standard_normal(K, dtype=np.float32)
        kc = rng.standard_normal((maxt, nkv * hd), dtype=np.float32)
        vc = rng.standard_normal((maxt, nkv * hd), dtype=np.float32)
        kc[L:] = np.nan
        vc[L:] = np.nan
        if f16:
            kc, vc = kc.astype(np.float16).view(np.uint16), vc.astype(np.float16).view(np.uint16)
        y = empty((E,), np.float32)
        dlen = up(np.array([L - 1], np.int32))
        call("lt_q8_gemv_attn_o", gpu.handle, up(q).vp, up(kc).vp, up(vc).vp, dlen.vp, nh, nkv, hd,
             ctypes.c_float(scale), maxt, kv_dtype, dW.vp, dr_.vp, y.vp, E)
        if L > maxL:
            assert np.all(np.isnan(y.to_host()))
            continue
        att = oracle.attn_decode(q, kc, vc, L, nh, nkv, hd, scale, f16)
        aq, ad = oracle.quant_q8(att)
        assert_bitexact(y.to_host(), oracle.q8_gemv(W, aq, ad, K, r), f"attn_o L={L}")
        assert dlen.to_host()[0] == L - 1
    assert _lib.raw("lt_attn_o_max_len")(14, 2, 128, LT_KV_F16) == 0
    assert _lib.raw("lt_attn_o_max_len")(32, 2, 64, LT_KV_F16) == 0


def test_q8_gemv_rms_silu_len(gpu, oracle):
    case("rms_silu_len")
    rng = np.random.default_rng(26)
    F, K = 4864, 896
    Wg, Wu = rand_weight(rng, F, K), rand_weight(rng, F, K)
    x = (2.0 * rng.standard_normal(K)).astype(np.float32)
    nw = (0.5 * rng.standard_normal(K) + 1.0).astype(np.float32)
    xq, xd = oracle.quant_q8(oracle.rmsnorm(x, nw, 1e-6))
    eq, ed = oracle.silu_mul_quant(oracle.q8_gemv(Wg, xq, xd, K), oracle.q8_gemv(Wu, xq, xd, K))
    Wil = up(M.interleave_gateup(Wg, Wu))
    for L0, maxt in ((5, 64), (63, 64), (64, 64)):
        vq, vd = empty((F,), np.int8), empty((F // 32,), np.uint16)
        dlen = up(np.array([L0], np.int32))
        call("lt_q8_gemv_rms_silu_len", gpu.handle, up(x).vp, up(nw).vp, ctypes.c_float(1e-6), Wil.vp, vq.vp,
             vd.vp, F, K, dlen.vp, maxt)
        assert_bitexact(vq.to_host(), eq, "silu*up quants")
        assert_bitexact(vd.to_host(), ed, "silu*up scales")
        assert dlen.to_host()[0] == (L0 + 1 if L0 < maxt else L0)

"""Per-op parity of the gfx950 kernels with the CPU oracle, through the C ABI.

Shapes, seeds and value distributions follow the reference's pair gates
(gate_quant_par.py:21-45, rms_canonical_pairgate.py:22-48, gemv_canonical_pairgate.py:36-42,
gate_addres.py:18-46, test_argmax2_bitexact.py:21-29, masked_attn_referee.py) plus the
BASELINE shapes.  The bar is bit-exact equality everywhere.
"""
import ctypes

import numpy as np
import pytest

from llamatov_amd import _lib
from llamatov_amd import engine as dr
from llamatov_amd import q8 as hq8
from llamatov_amd._lib import LT_KV_F16, LT_KV_F32, call

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[gpu-case] {msg}", flush=True)


def up(a):
    return dr.DevTensor.from_host(np.ascontiguousarray(a))


def empty(shape, dt):
    return dr.DevTensor.empty(shape, dt)


def bits(a):
    a = np.asarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def assert_bitexact(got, exp, what):
    got, exp = np.asarray(got), np.asarray(exp)
    assert got.shape == exp.shape, what
    bad = np.flatnonzero(bits(got).reshape(-1) != bits(exp).reshape(-1))
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]}: {got.reshape(-1)[bad[:5]]} vs {exp.reshape(-1)[bad[:5]]}"


@pytest.mark.parametrize("K", [32, 896, 4864, 14336])
def test_quant_q8(gpu, oracle, K):
    case(f"quant_q8 K={K}")
    rng = np.random.default_rng(7)
    x = (2.0 * rng.standard_normal(K)).astype(np.float32)
    x[:32] = 0.0                                  # all-zero block -> d = 1
    if K >= 64:
        x[32:64] = np.float32(1.0) * np.arange(-16, 16, dtype=np.float32) / np.float32(127 / 16.5)
    xq, xd = oracle.quant_q8(x)
    dx, dq, dd = up(x), empty((K,), np.int8), empty((K // 32,), np.uint16)
    dr.quant_q8_into(dx, dq, dd, K)
    assert_bitexact(dq.to_host(), xq, "xq")
    assert_bitexact(dd.to_host(), xd, "xd")


@pytest.mark.parametrize("K", [896, 4864, 14336])
def test_silu_mul_quant(gpu, oracle, K):
    case(f"silu_mul_quant K={K}")
    rng = np.random.default_rng(17)
    g = (3.0 * rng.standard_normal(K)).astype(np.float32)
    u = rng.standard_normal(K).astype(np.float32)
    g[:4] = [-100.0, 100.0, 0.0, -0.0]
    xq, xd = oracle.silu_mul_quant(g, u)
    dq, dd = empty((K,), np.int8), empty((K // 32,), np.uint16)
    call("lt_silu_mul_quant", gpu.handle, up(g).vp, up(u).vp, dq.vp, dd.vp, K)
    assert_bitexact(dq.to_host(), xq, "xq")
    assert_bitexact(dd.to_host(), xd, "xd")


@pytest.mark.parametrize("N,eps", [(896, 1e-6), (4096, 1e-5), (100, 1e-6), (14336, 1e-5)])
def test_rmsnorm_and_fused_quant(gpu, oracle, N, eps):
    case(f"rmsnorm N={N}")
    rng = np.random.default_rng(7)
    x = (2.0 * rng.standard_normal(N)).astype(np.float32)
    w = (0.5 * rng.standard_normal(N) + 1.0).astype(np.float32)
    exp = oracle.rmsnorm(x, w, eps)
    dx, dw, dy = up(x), up(w), empty((N,), np.float32)
    dr.rms_norm_into(dx, dw, eps, dy)
    assert_bitexact(dy.to_host(), exp, "rmsnorm")
    if N % 32 == 0:
        xq, xd = oracle.quant_q8(exp)
        dq, dd = empty((N,), np.int8), empty((N // 32,), np.uint16)
        call("lt_rmsnorm_quant", gpu.handle, dx.vp, dw.vp, dq.vp, dd.vp, N, ctypes.c_float(eps))
        assert_bitexact(dq.to_host(), xq, "rms_quant xq")
        assert_bitexact(dd.to_host(), xd, "rms_quant xd")


def test_rmsnorm_multirow(gpu, oracle):
    case("rmsnorm M=5 N=896")
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 896)).astype(np.float32)
    w = rng.standard_normal(896).astype(np.float32)
    dy = empty((5, 896), np.float32)
    dr.rms_norm_into(up(x), up(w), 1e-6, dy)
    exp = np.stack([oracle.rmsnorm(x[i], w, 1e-6) for i in range(5)])
    assert_bitexact(dy.to_host(), exp, "rmsnorm rows")


def _rand_gemv(rng, N, K):
    q = rng.integers(-127, 128, size=(N, K), dtype=np.int64).astype(np.int8)
    d = (rng.standard_normal((N, K // 32)) * 0.1).astype(np.float16).view(np.uint16)
    W = hq8.join_blocks(q, d)
    xq = rng.integers(-127, 128, size=K, dtype=np.int64).astype(np.int8)
    xd = (rng.standard_normal(K // 32) * 0.1).astype(np.float16).view(np.uint16)
    return W, xq, xd


GEMV_SHAPES = [(64, 256), (896, 4864), (896, 896), (1152, 896), (9728, 896), (151936, 896),
               (4864, 896), (4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096), (7, 96), (33, 32)]


@pytest.mark.parametrize("N,K", GEMV_SHAPES)
def test_q8_gemv_bitexact(gpu, oracle, N, K):
    case(f"q8_gemv N={N} K={K}")
    rng = np.random.default_rng(8)
    W, xq, xd = _rand_gemv(rng, N, K)
    exp = oracle.q8_gemv(W, xq, xd, K)
    dW = dr.Q8Weight(W, K)
    dq, dd, dy = up(xq), up(xd), empty((N,), np.float32)
    dr.q8_gemv_into(dW, dq, dd, dy)
    assert_bitexact(dy.to_host(), exp, f"gemv {N}x{K}")
    # addres / bias epilogue: one fp32 add at the store
    r = rng.standard_normal(N).astype(np.float32)
    dr.q8_gemv_into(dW, dq, dd, dy, up(r))
    assert_bitexact(dy.to_host(), oracle.q8_gemv(W, xq, xd, K, resid=r), "gemv+resid")
    dW.t.free()


@pytest.mark.parametrize("N,K", [(64, 256), (896, 4864), (33, 96)])
def test_q8_block_dots_exact(gpu, oracle, N, K):
    case(f"q8_gemv_isums N={N} K={K}")
    rng = np.random.default_rng(11)
    W, xq, _ = _rand_gemv(rng, N, K)
    W[:, 2:34] = 0x81  # a column of -127 quants
    xq[:32] = -127
    exp = oracle.block_dots(W, xq, K)
    dis = empty((N, K // 32), np.int32)
    call("lt_q8_gemv_isums", gpu.handle, up(W).vp, up(xq).vp, dis.vp, N, K)
    assert np.array_equal(dis.to_host(), exp)


@pytest.mark.parametrize("hd,nh,nkv,theta", [(64, 14, 2, 1e6), (128, 32, 8, 5e5)])
def test_rope_qk(gpu, oracle, hd, nh, nkv, theta):
    rng = np.random.default_rng(4)
    nheads = nh + nkv
    x = rng.standard_normal(nheads * hd).astype(np.float32)
    freqs = dr.rope_freqs(hd, theta)
    dfreq = up(freqs)
    for pos in (0, 1, 31, 255, 1023, 4095):
        case(f"rope hd={hd} pos={pos}")
        dx, dp = up(x), up(np.array([pos], np.int32))
        call("lt_rope_qk", gpu.handle, dx.vp, dp.vp, nheads, hd, dfreq.vp)
        assert_bitexact(dx.to_host(), oracle.rope(x, pos, nheads, hd, theta), f"rope pos={pos}")


@pytest.mark.parametrize("kv_dtype", [LT_KV_F32, LT_KV_F16])
def test_kv_append_incr(gpu, kv_dtype):
    case(f"kv_append kv_dtype={kv_dtype}")
    rng = np.random.default_rng(5)
    cache = dr.KVCache(8, 2, 64, kv_dtype)
    rows = []
    for t in range(9):  # the 9th append hits capacity and must change nothing
        k = rng.standard_normal(128).astype(np.float32)
        v = rng.standard_normal(128).astype(np.float32)
        rows.append((k, v))
        cache.append_at_len_incr(up(k), up(v))
    assert cache.device_length() == 8
    K = cache.rows_host("k", 8)
    V = cache.rows_host("v", 8)
    for t in range(8):
        k, v = rows[t]
        if kv_dtype == LT_KV_F16:
            k, v = k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
        assert np.array_equal(K[t], k) and np.array_equal(V[t], v)


def _attn_setup(rng, B, maxt, nkv, hd, kv_dtype, L_list, poison):
    k = rng.standard_normal((B, maxt, nkv * hd), dtype=np.float32)
    v = rng.standard_normal((B, maxt, nkv * hd), dtype=np.float32)
    for b, L in enumerate(L_list):
        k[b, L:] = poison
        v[b, L:] = poison
    if kv_dtype == LT_KV_F16:
        with np.errstate(over="ignore"):
            k = k.astype(np.float16).view(np.uint16)
            v = v.astype(np.float16).view(np.uint16)
    return k, v


@pytest.mark.parametrize("kv_dtype", [LT_KV_F32, LT_KV_F16])
@pytest.mark.parametrize("nsplit", [1, 4])
@pytest.mark.parametrize("poison", [np.nan, np.inf, 1e30])
def test_attention_masked_poison_and_length_sweep(gpu, oracle, kv_dtype, nsplit, poison):
    """masked_attn_referee.py:129-174 / test_masked_attn_poison.py:13-58: garbage beyond L
    must not change a bit; L in {1, 2, MAXT/2, MAXT-1, MAXT}."""
    rng = np.random.default_rng(6)
    nh, nkv, hd, maxt = 14, 2, 64, 256
    f16 = kv_dtype == LT_KV_F16
    ws_n = _lib.raw("lt_attn_workspace_size")(1, nh, hd, nsplit)
    ws = empty((max(ws_n, 1),), np.uint8)
    for L in (1, 2, maxt // 2, maxt - 1, maxt):
        case(f"attn L={L} nsplit={nsplit} f16={f16} poison={poison}")
        q = rng.standard_normal(nh * hd).astype(np.float32)
        k, v = _attn_setup(rng, 1, maxt, nkv, hd, kv_dtype, [L], poison)
        exp = oracle.attn_decode(q, k[0], v[0], L, nh, nkv, hd, 0.125, f16, nsplit)
        out = empty((nh * hd,), np.float32)
        call("lt_attn_decode", gpu.handle, up(q).vp, up(k).vp, up(v).vp, up(np.array([L], np.int32)).vp,
             out.vp, 1, nh, nkv, hd, ctypes.c_float(0.125), maxt, nsplit, kv_dtype, ws.vp, ws.nbytes)
        assert_bitexact(out.to_host(), exp, f"attn L={L}")


@pytest.mark.parametrize("kv_dtype,hd", [(LT_KV_F16, 128), (LT_KV_F16, 256), (LT_KV_F32, 64),
                                         (LT_KV_F32, 128)])
@pytest.mark.parametrize("nh,nkv", [(8, 8), (16, 8), (32, 8), (16, 2)])
def test_attention_decode_geometries(gpu, oracle, kv_dtype, hd, nh, nkv):
    """Batched decode across head sizes, GQA group sizes (1, 2, 4, 8 heads per KV head) and
    cache types, NaN past each sequence's length, split counts that leave ragged and empty
    splits (L = 3 with 4 splits), and the single-split path that divides in-kernel."""
    f16 = kv_dtype == LT_KV_F16
    rng = np.random.default_rng(hd + nh)
    B, maxt = 3, 300
    for nsplit, lens in ((1, [300, 129, 1]), (4, [3, 64, 65]), (7, [300, 200, 77])):
        case(f"attn decode hd={hd} nh={nh} nkv={nkv} f16={f16} nsplit={nsplit} lens={lens}")
        q = rng.standard_normal((B, nh * hd)).astype(np.float32)
        k, v = _attn_setup(rng, B, maxt, nkv, hd, kv_dtype, lens, np.nan)
        ws_n = _lib.raw("lt_attn_workspace_size")(B, nh, hd, nsplit)
        ws = empty((max(ws_n, 1),), np.uint8)
        out = empty((B, nh * hd), np.float32)
        scale = float(hd ** -0.5)
        call("lt_attn_decode", gpu.handle, up(q).vp, up(k).vp, up(v).vp, up(np.array(lens, np.int32)).vp,
             out.vp, B, nh, nkv, hd, ctypes.c_float(scale), maxt, nsplit, kv_dtype, ws.vp, ws.nbytes)
        got = out.to_host()
        for b in range(B):
            exp = oracle.attn_decode(q[b], k[b], v[b], lens[b], nh, nkv, hd, scale, f16, nsplit)
            assert_bitexact(got[b], exp, f"attn b={b} L={lens[b]}")


@pytest.mark.parametrize("kv_dtype,nh,nkv,hd", [(LT_KV_F16, 14, 2, 64), (LT_KV_F32, 14, 2, 64),
                                                 (LT_KV_F16, 32, 8, 128), (LT_KV_F32, 16, 2, 128),
                                                 (LT_KV_F16, 8, 8, 256)])
@pytest.mark.parametrize("len0,T,nsplit", [(0, 37, 1), (5, 40, 4), (0, 70, 16), (200, 33, 7), (250, 50, 5),
                                            (0, 300, 16), (3, 61, 64)])
def test_attention_prefill(gpu, oracle, kv_dtype, nh, nkv, hd, len0, T, nsplit):
    """Causal prefill attention: query t of T attends the first len0 + t + 1 rows of one
    cache, each exactly as a decode of that length (split layout per query, empty splits for
    short queries), NaN past len0 + T."""
    f16 = kv_dtype == LT_KV_F16
    case(f"attn prefill nh={nh} nkv={nkv} hd={hd} f16={f16} len0={len0} T={T} nsplit={nsplit}")
    rng = np.random.default_rng(nh * hd + T)
    maxt = 300
    q = rng.standard_normal((T, nh * hd)).astype(np.float32)
    k, v = _attn_setup(rng, 1, maxt, nkv, hd, kv_dtype, [len0 + T], np.nan)
    ws_n = _lib.raw("lt_attn_workspace_size")(T, nh, hd, nsplit)
    ws = empty((max(ws_n, 1),), np.uint8)
    out = empty((T, nh * hd), np.float32)
    scale = float(hd ** -0.5)
    call("lt_attn_prefill", gpu.handle, up(q).vp, nh * hd, up(k).vp, up(v).vp, up(np.array([len0], np.int32)).vp,
         out.vp, T, nh, nkv, hd, ctypes.c_float(scale), maxt, nsplit, kv_dtype, ws.vp, ws.nbytes)
    got = out.to_host()
    for t in range(T):
        exp = oracle.attn_decode(q[t], k[0], v[0], len0 + t + 1, nh, nkv, hd, scale, f16, nsplit)
        assert_bitexact(got[t], exp, f"query {t} L={len0 + t + 1}")


@pytest.mark.parametrize("B,L,nsplit", [(1, 4096, 32), (8, 4096, 32), (1, 16384, 64), (2, 32768, 128),
                                         (8, 16384, 64), (8, 32768, 128),
                                         # the split counts engine.attn_nsplit_for picks at C4
                                         (1, 4096, 64), (1, 16384, 128), (1, 32768, 128), (1, 32768, 64),
                                         (8, 16384, 32),
                                         (8, 32768, 64)])
def test_attention_long_context_batched(gpu, oracle, B, L, nsplit):
    """BASELINE config 4 geometry: 32 Q heads, 8 KV heads, hd 128, fp16 KV."""
    case(f"attn C4 B={B} L={L} nsplit={nsplit}")
    rng = np.random.default_rng(10)
    nh, nkv, hd = 32, 8, 128
    lens = [L - 37 * b for b in range(B)]
    q = rng.standard_normal((B, nh * hd)).astype(np.float32)
    k, v = _attn_setup(rng, B, L, nkv, hd, LT_KV_F16, lens, 0.0)
    scale = float(hd ** -0.5)
    ws_n = _lib.raw("lt_attn_workspace_size")(B, nh, hd, nsplit)
    ws = empty((ws_n,), np.uint8)
    out = empty((B, nh * hd), np.float32)
    call("lt_attn_decode", gpu.handle, up(q).vp, up(k).vp, up(v).vp, up(np.array(lens, np.int32)).vp,
         out.vp, B, nh, nkv, hd, ctypes.c_float(scale), L, nsplit, LT_KV_F16, ws.vp, ws.nbytes)
    got = out.to_host()
    for b in range(B):
        exp = oracle.attn_decode(q[b], k[b], v[b], lens[b], nh, nkv, hd, scale, True, nsplit)
        assert_bitexact(got[b], exp, f"attn b={b}")



@pytest.mark.parametrize("kv_dtype,hd", [(LT_KV_F16, 128), (LT_KV_F16, 64), (LT_KV_F32, 128), (LT_KV_F32, 64)])
@pytest.mark.parametrize("nh,nkv", [(32, 8), (16, 8), (16, 2)])
def test_attention_decode_one_round_splits(gpu, oracle, kv_dtype, hd, nh, nkv):
    """Small-grid batched decode whose splits hold at most one 64-row K round (maxt / nsplit
    <= 64), where V is requested together with K: NaN past each length, lengths that end
    inside, at and one past a round, ragged and empty splits."""
    f16 = kv_dtype == LT_KV_F16
    rng = np.random.default_rng(7 * hd + nh)
    maxt, B = 256, 3
    for nsplit, lens in ((4, [256, 255, 1]), (4, [64, 65, 63]), (8, [200, 3, 129]), (16, [17, 256, 100])):
        case(f"attn one-round hd={hd} nh={nh} nkv={nkv} f16={f16} nsplit={nsplit} lens={lens}")
        q = rng.standard_normal((B, nh * hd)).astype(np.float32)
        k, v = _attn_setup(rng, B, maxt, nkv, hd, kv_dtype, lens, np.nan)
        ws_n = _lib.raw("lt_attn_workspace_size")(B, nh, hd, nsplit)
        ws = empty((max(ws_n, 1),), np.uint8)
        out = empty((B, nh * hd), np.float32)
        scale = float(hd ** -0.5)
        call("lt_attn_decode", gpu.handle, up(q).vp, up(k).vp, up(v).vp, up(np.array(lens, np.int32)).vp,
             out.vp, B, nh, nkv, hd, ctypes.c_float(scale), maxt, nsplit, kv_dtype, ws.vp, ws.nbytes)
        got = out.to_host()
        for b in range(B):
            exp = oracle.attn_decode(q[b], k[b], v[b], lens[b], nh, nkv, hd, scale, f16, nsplit)
            assert_bitexact(got[b], exp, f"attn b={b} L={lens[b]}")

def test_argmax_ties(gpu, oracle):
    case("argmax V=151936")
    rng = np.random.default_rng(9)
    x = rng.standard_normal(151936).astype(np.float32)
    ws = empty((_lib.raw("lt_argmax_workspace_size")(),), np.uint8)
    out = empty((1,), np.int32)
    for planted in (None, (1000, 50000), (151935, 151934), (0, 151935)):
        xx = x.copy()
        if planted:
            xx[list(planted)] = np.float32(50.0)
        dr.argmax_into(up(xx), xx.size, out.ptr, ws)
        assert int(out.to_host()[0]) == oracle.argmax(xx)
    for n in (1, 255, 256, 257, 70000):
        xx = x[:n].copy()
        dr.argmax_into(up(xx), n, out.ptr, ws)
        assert int(out.to_host()[0]) == oracle.argmax(xx)


def test_embed_q8(gpu, oracle):
    case("embed_q8")
    rng = np.random.default_rng(12)
    V, E = 300, 896
    emb = hq8.quantize_rows((rng.standard_normal((V, E)) * 0.02).astype(np.float32))
    demb, x, err = up(emb), empty((E,), np.float32), up(np.zeros(1, np.int32))
    for tok in (0, 1, 157, V - 1):
        call("lt_embed_q8", gpu.handle, demb.vp, up(np.array([tok], np.int32)).vp, x.vp, E, V, err.vp)
        assert_bitexact(x.to_host(), oracle.embed_row(emb, tok, E), f"embed {tok}")
    assert err.to_host()[0] == 0
    call("lt_embed_q8", gpu.handle, demb.vp, up(np.array([V], np.int32)).vp, x.vp, E, V, err.vp)
    assert err.to_host()[0] == 1 and not np.any(x.to_host())

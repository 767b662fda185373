"""The batched prefill path: the int8-MFMA Q8_0 GEMM against the oracle's GEMV per token,
and a batched prefill against the token-by-token prefill (the reference's device-uniform
requirement, bpd/lib/dev_residency.py:1338-1356): KV cache, logits and the continued greedy
stream bit-identical."""
import numpy as np
import pytest

from llamatov_amd import engine as dr
from llamatov_amd import model as M
from llamatov_amd import q8 as hq8
from llamatov_amd._lib import LT_KV_F16, LT_KV_F32, call

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[gpu-case] {msg}", flush=True)


def up(a):
    return dr.DevTensor.from_host(np.ascontiguousarray(a))


def bits(a):
    a = np.asarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


@pytest.mark.parametrize("T,K", [(37, 896), (1, 4096), (130, 4096), (9, 14336)])
def test_rmsnorm_quant_block_major(gpu, T, K):
    """One launch of RMSNorm + block-major quant equals lt_rmsnorm followed by lt_quant_q8_bm."""
    case(f"rmsnorm_quant_bm T={T} K={K}")
    rng = np.random.default_rng(T + K)
    X = (2.0 * rng.standard_normal((T, K))).astype(np.float32)
    X[0, :64] = 0.0
    w = (0.5 * rng.standard_normal(K) + 1.0).astype(np.float32)
    dx, dw = up(X), up(w)
    h = dr.DevTensor.empty((T, K), np.float32)
    q1, d1 = dr.DevTensor.empty((K // 32, T, 32), np.int8), dr.DevTensor.empty((K // 32, T), np.uint16)
    q2, d2 = dr.DevTensor.empty((K // 32, T, 32), np.int8), dr.DevTensor.empty((K // 32, T), np.uint16)
    call("lt_rmsnorm", gpu.handle, dx.vp, dw.vp, h.vp, T, K, 1e-5)
    call("lt_quant_q8_bm", gpu.handle, h.vp, q1.vp, d1.vp, T, K)
    call("lt_rmsnorm_quant_bm", gpu.handle, dx.vp, dw.vp, q2.vp, d2.vp, T, K, 1e-5)
    assert np.array_equal(q1.to_host(), q2.to_host())
    assert np.array_equal(d1.to_host(), d2.to_host())


@pytest.mark.parametrize("kv_dtype,nh,nkv,hd,T,len0,maxt", [(LT_KV_F16, 32, 8, 128, 77, 5, 100),
                                                             (LT_KV_F32, 14, 2, 64, 40, 0, 64),
                                                             (LT_KV_F16, 8, 8, 256, 9, 3, 10),
                                                             (LT_KV_F32, 4, 1, 128, 6, -2, 8)])
def test_rope_append_batch(gpu, kv_dtype, nh, nkv, hd, T, len0, maxt):
    """One launch of RoPE + KV append equals lt_rope_batch followed by lt_kv_append_batch: the
    same q rows and cache rows, rows at positions outside [0, maxt) roped but not stored."""
    case(f"rope_append_batch kv={kv_dtype} nh={nh} nkv={nkv} hd={hd} T={T} len0={len0} maxt={maxt}")
    rng = np.random.default_rng(nh * T + hd)
    NQ = (nh + 2 * nkv) * hd
    X = (3.0 * rng.standard_normal((T, NQ))).astype(np.float32)
    freqs = (1e4 ** (-np.arange(hd // 2) * 2.0 / hd)).astype(np.float32)
    et = np.float16 if kv_dtype == LT_KV_F16 else np.float32
    fill = np.full((maxt, nkv * hd), 7, et)
    x1, x2, fr, ln = up(X), up(X), up(freqs), up(np.array([len0], np.int32))
    k1, v1, k2, v2 = up(fill), up(fill), up(fill), up(fill)
    call("lt_rope_batch", gpu.handle, x1.vp, T, NQ, ln.vp, nh + nkv, hd, fr.vp)
    call("lt_kv_append_batch", gpu.handle, k1.vp, v1.vp, x1.vp, NQ, nh * hd, (nh + nkv) * hd, T, ln.vp, nkv * hd,
         maxt, kv_dtype)
    call("lt_rope_append_batch", gpu.handle, x2.vp, T, NQ, ln.vp, nh, nkv, hd, fr.vp, k2.vp, v2.vp, maxt, kv_dtype)
    a, b = x1.to_host(), x2.to_host()
    assert bits(a[:, :nh * hd]).tobytes() == bits(b[:, :nh * hd]).tobytes(), "q rows"
    assert np.array_equal(a[:, (nh + nkv) * hd:], b[:, (nh + nkv) * hd:]), "v rows untouched"
    for c1, c2, what in ((k1, k2, "K"), (v1, v2, "V")):
        assert c1.to_host().tobytes() == c2.to_host().tobytes(), f"{what} cache"
    lens = up(np.array([0, 5, maxt - 1, maxt], np.int32))
    call("lt_len_add_n", gpu.handle, lens.vp, 3, T, maxt)
    assert lens.to_host().tolist() == [min(T, maxt), min(5 + T, maxt), maxt, maxt]


@pytest.mark.parametrize("N,K,T,epi", [(1152, 896, 37, "bias"), (896, 4864, 130, "resid"), (100, 96, 5, "store"),
                                       (64, 1024, 129, "store"), (4096, 4096, 33, "store"), (40, 14336, 3, "resid")])
def test_q8_gemm_matches_gemv_per_token(gpu, oracle, N, K, T, epi):
    case(f"q8_gemm N={N} K={K} T={T} {epi}")
    rng = np.random.default_rng(31)
    W = hq8.quantize_rows((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    X = (rng.standard_normal((T, K))).astype(np.float32)
    X[0, :64] = 0.0
    xq = np.empty((T, K), np.int8)
    xd = np.empty((T, K // 32), np.uint16)
    for t in range(T):
        xq[t], xd[t] = oracle.quant_q8(X[t])
    bias = (rng.standard_normal(N) * 0.02).astype(np.float32) if epi == "bias" else None
    resid = rng.standard_normal((T, N)).astype(np.float32) if epi == "resid" else None
    Y = dr.DevTensor.empty((T, N), np.float32)
    call("lt_q8_gemm", gpu.handle, up(W).vp, up(xq).vp, up(xd).vp, up(bias).vp if bias is not None else None,
         up(resid).vp if resid is not None else None, Y.vp, T, N, K)
    got = Y.to_host()
    for t in range(T):
        r = bias if bias is not None else (resid[t] if resid is not None else None)
        exp = oracle.q8_gemv(W, xq[t], xd[t], K, r)
        assert np.array_equal(bits(got[t]), bits(exp)), f"token {t}: {np.flatnonzero(bits(got[t]) != bits(exp))[:5]}"


@pytest.mark.parametrize("F,K,T", [(4864, 896, 40), (64, 128, 7)])
def test_q8_gemm_silu(gpu, oracle, F, K, T):
    case(f"q8_gemm_silu F={F} K={K} T={T}")
    rng = np.random.default_rng(32)
    Wg = hq8.quantize_rows((rng.standard_normal((F, K)) * 0.02).astype(np.float32))
    Wu = hq8.quantize_rows((rng.standard_normal((F, K)) * 0.02).astype(np.float32))
    X = rng.standard_normal((T, K)).astype(np.float32)
    xq = np.empty((T, K), np.int8)
    xd = np.empty((T, K // 32), np.uint16)
    for t in range(T):
        xq[t], xd[t] = oracle.quant_q8(X[t])
    V = dr.DevTensor.empty((T, F), np.float32)
    call("lt_q8_gemm_silu", gpu.handle, up(M.interleave_gateup(Wg, Wu)).vp, up(xq).vp, up(xd).vp, V.vp, T, F, K)
    got = V.to_host()
    for t in range(T):
        g = oracle.q8_gemv(Wg, xq[t], xd[t], K)
        u = oracle.q8_gemv(Wu, xq[t], xd[t], K)
        assert np.array_equal(bits(got[t]), bits(oracle.silu_mul(g, u))), f"token {t}"


def tiles_host(W, N, K):
    """The tile-major layout restated on the host: tile block (rt, b) = the 32 quant bytes of
    rows 32*rt .. 32*rt+31 of block b, then their 32 fp16 scales (1088 bytes)."""
    nb = K // 32
    nt = (N + 31) // 32
    pad = np.zeros((nt * 32, nb * 34), np.uint8)
    pad[:N] = W
    blk = pad.reshape(nt, 32, nb, 34).transpose(0, 2, 1, 3)          # [rt][b][r][34]
    return np.concatenate([blk[..., 2:].reshape(nt, nb, 1024), blk[..., :2].reshape(nt, nb, 64)], axis=2)


@pytest.mark.parametrize("N,K", [(1152, 896), (100, 96), (33, 4864), (32, 32)])
def test_q8_tiles_layout(gpu, N, K):
    case(f"q8_tiles N={N} K={K}")
    from llamatov_amd._lib import raw
    rng = np.random.default_rng(N + K)
    W = rng.integers(0, 256, (N, K // 32 * 34), dtype=np.uint8)
    n = int(raw("lt_q8_tiles_bytes")(N, K))
    assert n == (N + 31) // 32 * 32 * (K // 32) * 34
    Wt = dr.DevTensor.empty((n,), np.uint8)
    Wt.dev.fill(Wt.ptr, 0xA5, Wt.nbytes)
    call("lt_q8_tiles", gpu.handle, up(W).vp, Wt.vp, N, K)
    assert np.array_equal(Wt.to_host(), tiles_host(W, N, K).reshape(-1))


def rope_pair_rows(nh, nkv, hd):
    """The rope-pair row order restated: within each q and k head, row 2j + e of the copy is
    row j + e*hd/2 of the head; v rows keep their places."""
    head = np.arange(hd)
    per = (head >> 1) + (head & 1) * (hd // 2)
    qk = (np.arange(nh + nkv)[:, None] * hd + per[None, :]).reshape(-1)
    return np.concatenate([qk, np.arange((nh + nkv) * hd, (nh + 2 * nkv) * hd)])


@pytest.mark.parametrize("nh,nkv,hd,K", [(14, 2, 64, 896), (4, 4, 64, 96), (2, 1, 6, 64)])
def test_q8_tiles_rope_layout(gpu, nh, nkv, hd, K):
    """lt_q8_tiles_rope = the tile-major copy of the rows in the rope-pair order."""
    case(f"q8_tiles_rope nh={nh} nkv={nkv} hd={hd} K={K}")
    N = (nh + 2 * nkv) * hd
    rng = np.random.default_rng(N + K)
    W = rng.integers(0, 256, (N, K // 32 * 34), dtype=np.uint8)
    perm = rope_pair_rows(nh, nkv, hd)
    assert sorted(perm.tolist()) == list(range(N))
    n = int(dr._lib.raw("lt_q8_tiles_bytes")(N, K))
    Wt = dr.DevTensor.empty((n,), np.uint8)
    Wt.dev.fill(Wt.ptr, 0xA5, Wt.nbytes)
    call("lt_q8_tiles_rope", gpu.handle, up(W).vp, Wt.vp, N, K, nh, nkv, hd)
    assert np.array_equal(Wt.to_host(), tiles_host(W[perm], N, K).reshape(-1))
    with pytest.raises(RuntimeError, match="N = \\(nh \\+ 2 nkv\\) hd"):
        call("lt_q8_tiles_rope", gpu.handle, up(W).vp, Wt.vp, N - hd, K, nh, nkv, hd)


@pytest.mark.parametrize("T,K", [(37, 896), (1, 32), (130, 4864), (67, 14336)])
def test_quant_q8_block_major(gpu, oracle, T, K):
    case(f"quant_q8_bm T={T} K={K}")
    rng = np.random.default_rng(T * K)
    X = rng.standard_normal((T, K)).astype(np.float32)
    X[0, :32] = 0.0
    X[-1, 32 * (K // 64):32 * (K // 64) + 32] *= 1e-30
    xq = dr.DevTensor.empty((K // 32, T, 32), np.int8)
    xd = dr.DevTensor.empty((K // 32, T), np.uint16)
    call("lt_quant_q8_bm", gpu.handle, up(X).vp, xq.vp, xd.vp, T, K)
    gq, gd = xq.to_host(), xd.to_host()
    for t in range(T):
        q, d = oracle.quant_q8(X[t])
        assert np.array_equal(gq[:, t, :].reshape(-1), q), f"token {t} quants"
        assert np.array_equal(gd[:, t], d), f"token {t} scales"


def subnormal_scales(rng, W, xd, frac=0.25):
    """Replaces a fraction of the weight and activation scales by fp16 subnormals (bits
    0x0001 .. 0x03FF, either sign): the scale products must stay exact."""
    nb = xd.shape[1]
    sc = W.reshape(W.shape[0], nb, 34)[..., :2].copy().view(np.uint16)[..., 0]
    m = rng.random(sc.shape) < frac
    sc[m] = rng.integers(1, 0x400, m.sum()).astype(np.uint16) | (rng.integers(0, 2, m.sum()) << 15).astype(np.uint16)
    W.reshape(W.shape[0], nb, 34)[..., :2] = sc[..., None].view(np.uint8).reshape(W.shape[0], nb, 2)
    m = rng.random(xd.shape) < frac
    xd[m] = rng.integers(1, 0x400, m.sum()).astype(np.uint16)


def force_walk(monkeypatch, walk: str) -> None:
    """Pin the tiled GEMM's kernel: "ls" / "ls8" the leaf-split kernel with 4 / 8 waves per
    tile (its compile-time schedule where K <= 5120), "lsd" / "lsd8" the same with the
    run-time walk at every K, else k_q8_gemm with the leaf walk LT_GEMM_GROUPED = walk (all
    read at every launch)."""
    if walk.startswith("ls"):
        dyn = walk.startswith("lsd")
        monkeypatch.setenv("LT_GEMM_LS", "1")
        monkeypatch.setenv("LT_GEMM_LS_W", walk[3 if dyn else 2:] or "4")
        monkeypatch.setenv("LT_GEMM_LS_STATIC", "0" if dyn else "1")
    else:
        monkeypatch.setenv("LT_GEMM_LS", "0")
        monkeypatch.setenv("LT_GEMM_GROUPED", walk)


@pytest.mark.parametrize("N,K,T,epi", [(1152, 896, 37, "bias"), (896, 4864, 130, "resid"), (100, 96, 5, "store"),
                                       (64, 1024, 129, "store"), (4096, 4096, 33, "store"), (40, 14336, 3, "resid"),
                                       (96, 256, 70, "subnormal"), (64, 2048, 45, "bias"), (72, 6144, 130, "resid"),
                                       (33, 4096, 7, "subnormal"), (96, 8192, 77, "subnormal"),
                                       (130, 14336, 67, "bias")])
@pytest.mark.parametrize("grouped", ["2", "1", "0", "ls", "ls8", "ls16", "lsd", "lsd8", "lsd16"])
def test_q8_gemm_tiled_matches_gemv_per_token(gpu, oracle, N, K, T, epi, grouped, monkeypatch):
    """Every leaf walk of the tiled kernel (grouped leaves with a 4- or 2-slot ring where K
    allows them, the dynamic walk; forced with LT_GEMM_GROUPED) and the leaf-split kernel
    (forced with LT_GEMM_LS) against the oracle's GEMV per token."""
    force_walk(monkeypatch, grouped)
    case(f"q8_gemm_t N={N} K={K} T={T} {epi} grouped={grouped}")
    rng = np.random.default_rng(33)
    W = hq8.quantize_rows((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    X = (rng.standard_normal((T, K))).astype(np.float32)
    X[0, :64] = 0.0
    xq = np.empty((T, K), np.int8)
    xd = np.empty((T, K // 32), np.uint16)
    for t in range(T):
        xq[t], xd[t] = oracle.quant_q8(X[t])
    if epi == "subnormal":
        subnormal_scales(rng, W, xd)
        epi = "store"
    xq_bm = np.ascontiguousarray(xq.reshape(T, K // 32, 32).transpose(1, 0, 2))
    xd_bm = np.ascontiguousarray(xd.T)
    bias = (rng.standard_normal(N) * 0.02).astype(np.float32) if epi == "bias" else None
    resid = rng.standard_normal((T, N)).astype(np.float32) if epi == "resid" else None
    Y = dr.DevTensor.empty((T, N), np.float32)
    call("lt_q8_gemm_t", gpu.handle, up(tiles_host(W, N, K)).vp, up(xq_bm).vp, up(xd_bm).vp,
         up(bias).vp if bias is not None else None, up(resid).vp if resid is not None else None, Y.vp, T, N, K)
    got = Y.to_host()
    for t in range(T):
        r = bias if bias is not None else (resid[t] if resid is not None else None)
        exp = oracle.q8_gemv(W, xq[t], xd[t], K, r)
        assert np.array_equal(bits(got[t]), bits(exp)), f"token {t}: {np.flatnonzero(bits(got[t]) != bits(exp))[:5]}"


@pytest.mark.parametrize("F,K,T", [(4864, 896, 40), (64, 128, 7), (48, 96, 70), (128, 6144, 33), (96, 4096, 140)])
@pytest.mark.parametrize("grouped", ["2", "1", "0", "ls", "ls8", "ls16", "lsd", "lsd8", "lsd16"])
def test_q8_gemm_silu_tiled(gpu, oracle, F, K, T, grouped, monkeypatch):
    force_walk(monkeypatch, grouped)
    case(f"q8_gemm_silu_t F={F} K={K} T={T} grouped={grouped}")
    rng = np.random.default_rng(34)
    Wg = hq8.quantize_rows((rng.standard_normal((F, K)) * 0.02).astype(np.float32))
    Wu = hq8.quantize_rows((rng.standard_normal((F, K)) * 0.02).astype(np.float32))
    X = rng.standard_normal((T, K)).astype(np.float32)
    xq = np.empty((T, K), np.int8)
    xd = np.empty((T, K // 32), np.uint16)
    for t in range(T):
        xq[t], xd[t] = oracle.quant_q8(X[t])
    xq_bm = np.ascontiguousarray(xq.reshape(T, K // 32, 32).transpose(1, 0, 2))
    xd_bm = np.ascontiguousarray(xd.T)
    V = dr.DevTensor.empty((T, F), np.float32)
    Wgu = M.interleave_gateup(Wg, Wu)
    call("lt_q8_gemm_silu_t", gpu.handle, up(tiles_host(Wgu, 2 * F, K)).vp, up(xq_bm).vp, up(xd_bm).vp, V.vp,
         T, F, K)
    got = V.to_host()
    for t in range(T):
        g = oracle.q8_gemv(Wg, xq[t], xd[t], K)
        u = oracle.q8_gemv(Wu, xq[t], xd[t], K)
        assert np.array_equal(bits(got[t]), bits(oracle.silu_mul(g, u))), f"token {t}"


@pytest.mark.parametrize("F,K,T", [(4864, 896, 64), (4864, 896, 37), (64, 128, 7), (96, 4096, 70), (128, 6144, 33),
                                   (4864, 896, 128)])
@pytest.mark.parametrize("static", ["1", "0"])
def test_q8_gemm_silu_quant_equals_gemm_then_quant(gpu, F, K, T, static, monkeypatch):
    """lt_q8_gemm_silu_quant_t equals lt_q8_gemm_silu_t followed by lt_quant_q8_bm of its
    output: the block-major quants and scales byte for byte (both leaf-split schedules,
    LT_GEMM_LS_STATIC)."""
    monkeypatch.setenv("LT_GEMM_LS_STATIC", static)
    case(f"q8_gemm_silu_quant_t F={F} K={K} T={T} static={static}")
    rng = np.random.default_rng(F + T)
    Wgu = hq8.quantize_rows((rng.standard_normal((2 * F, K)) * 0.02).astype(np.float32))
    X = rng.standard_normal((T, K)).astype(np.float32)
    xq = dr.DevTensor.empty((T * K,), np.int8)
    xd = dr.DevTensor.empty((T * K // 32,), np.uint16)
    call("lt_quant_q8_bm", gpu.handle, up(X).vp, xq.vp, xd.vp, T, K)
    Wt = up(tiles_host(Wgu, 2 * F, K))
    V = dr.DevTensor.empty((T, F), np.float32)
    vq_a, vd_a = dr.DevTensor.empty((T * F,), np.int8), dr.DevTensor.empty((T * F // 32,), np.uint16)
    vq_b, vd_b = dr.DevTensor.empty((T * F,), np.int8), dr.DevTensor.empty((T * F // 32,), np.uint16)
    call("lt_q8_gemm_silu_t", gpu.handle, Wt.vp, xq.vp, xd.vp, V.vp, T, F, K)
    call("lt_quant_q8_bm", gpu.handle, V.vp, vq_a.vp, vd_a.vp, T, F)
    call("lt_q8_gemm_silu_quant_t", gpu.handle, Wt.vp, xq.vp, xd.vp, vq_b.vp, vd_b.vp, T, F, K)
    assert np.array_equal(vq_a.to_host(), vq_b.to_host()), "quants"
    assert np.array_equal(vd_a.to_host(), vd_b.to_host()), "scales"
    from llamatov_amd._lib import raw
    rc = raw("lt_q8_gemm_silu_quant_t")(gpu.handle, Wt.vp, xq.vp, xd.vp, xq.vp, vd_b.vp, T, F, K)
    assert rc != 0, "in-place output refused"
    for t in (xq, xd, Wt, V, vq_a, vd_a, vq_b, vd_b):
        t.free()


_W = {}


def weights(cfg):
    if cfg.name not in _W:
        _W[cfg.name] = M.synth_weights(cfg, seed=1234)
    return _W[cfg.name]


@pytest.mark.parametrize("cfg_name,n_prompt,kv_dtype,nsplit", [
    ("tiny", 9, LT_KV_F32, 1), ("tiny", 40, LT_KV_F16, 2), ("small-qwen-arch", 32, LT_KV_F16, 1),
    ("small-qwen-arch", 33, LT_KV_F32, 4), ("small-qwen-arch", 70, LT_KV_F16, 16),
    ("tiny", 40, LT_KV_F32, 32)])
def test_prefill_equals_stepwise(gpu, oracle, cfg_name, n_prompt, kv_dtype, nsplit):
    cfg = M.CONFIGS[cfg_name]
    case(f"prefill vs stepwise {cfg_name} T={n_prompt} kv={kv_dtype} nsplit={nsplit}")
    model = dr.ResidentModel(cfg, weights(cfg), gpu, layouts="fused")
    prof = dr.Profile(kv_dtype=kv_dtype, attn_nsplit=nsplit)
    prompt = M.random_prompt(cfg, n_prompt, seed=11)
    a = dr.DecodePlan(model, prof)
    b = dr.DecodePlan(model, prof)
    la = dr.forward_tokens(a, prompt)
    dr.forward_prefill(b, prompt)
    lb = b.read_logits()
    assert np.array_equal(bits(la), bits(lb))
    assert a.read_token() == b.read_token()
    assert list(a.lengths()) == list(b.lengths()) == [n_prompt] * cfg.n_layers
    for il in range(cfg.n_layers):
        for w in "kv":
            assert np.array_equal(a.caches[il].rows_host(w, n_prompt).view(np.uint8),
                                  b.caches[il].rows_host(w, n_prompt).view(np.uint8)), (il, w)
    # decoding continues identically (graph replay after the batched prefill)
    gb = dr.StepGraph(b)
    gb.capture()
    seq_b = gb.replay_tokens(6)
    seq_a = []
    for _ in range(6):
        a.step()
        seq_a.append(a.read_token())
    assert seq_a == seq_b
    # and against the oracle
    orc = oracle.OracleModel(cfg, weights(cfg), kv_f16=kv_dtype == LT_KV_F16, attn_nsplit=nsplit)
    exp, _ = orc.generate(prompt, 7)
    first = int(oracle.argmax(lb))
    assert [first] + seq_b == exp
    gb.free()
    a.free()
    b.free()
    model.free()


@pytest.mark.parametrize("cfg_name,kv_dtype,nsplit", [("tiny", LT_KV_F32, 1), ("small-qwen-arch", LT_KV_F16, 4),
                                                      ("tiny", LT_KV_F16, 16)])
def test_prefill_into_non_empty_cache(gpu, oracle, cfg_name, kv_dtype, nsplit):
    """A batched prefill that starts from a non-empty cache: chunk A, then chunk B, then three
    decode steps, then chunk C.  RoPE positions, the causal attention over the rows already
    cached and the shared length update all start at the current length; the result equals
    the single-token path over the same tokens (KV rows, lengths, logits, greedy token) and
    the oracle's logits."""
    cfg = M.CONFIGS[cfg_name]
    case(f"prefill non-empty {cfg_name} kv={kv_dtype} nsplit={nsplit}")
    model = dr.ResidentModel(cfg, weights(cfg), gpu, layouts="fused")
    prof = dr.Profile(kv_dtype=kv_dtype, attn_nsplit=nsplit)
    toks = M.random_prompt(cfg, 40, seed=21)
    A, B, C = toks[:11], toks[11:24], toks[24:37]
    a = dr.DecodePlan(model, prof)
    b = dr.DecodePlan(model, prof)
    orc = oracle.OracleModel(cfg, weights(cfg), kv_f16=kv_dtype == LT_KV_F16, attn_nsplit=nsplit)
    dr.forward_prefill(b, A)
    dr.forward_prefill(b, B)
    seq = list(A) + list(B)
    for _ in range(3):
        t = b.read_token()
        seq.append(t)
        b.step()
    dr.forward_prefill(b, C)
    seq += list(C)
    la = dr.forward_tokens(a, seq)
    lb = b.read_logits()
    exp = None
    for t in seq:
        exp = orc.step(t)
    assert np.array_equal(bits(la), bits(lb))
    assert np.array_equal(bits(lb), bits(exp))
    assert a.read_token() == b.read_token()
    n = len(seq)
    assert list(a.lengths()) == list(b.lengths()) == [n] * cfg.n_layers
    assert all(c.length == n for c in b.caches)
    for il in range(cfg.n_layers):
        for w in "kv":
            assert np.array_equal(a.caches[il].rows_host(w, n).view(np.uint8),
                                  b.caches[il].rows_host(w, n).view(np.uint8)), (il, w)
    a.free()
    b.free()
    model.free()


def test_capacity_is_refused_on_the_host(gpu):
    """Steps, replays and prefills that would pass max_ctx raise before launching anything."""
    cfg = M.TINY
    case("capacity refusal")
    model = dr.ResidentModel(cfg, weights(cfg), gpu, layouts="fused")
    plan = dr.DecodePlan(model, dr.Profile(), max_ctx=8, hist_cap=16)
    dr.forward_prefill(plan, M.random_prompt(cfg, 6, seed=2))
    with pytest.raises(ValueError):
        dr.forward_prefill(plan, [1, 2, 3])
    gr = dr.StepGraph(plan)
    gr.capture()
    with pytest.raises(ValueError):
        gr.replay_tokens(3)
    gr.replay_tokens(2)
    assert list(plan.lengths()) == [8] * cfg.n_layers
    with pytest.raises(ValueError):
        gr.replay_token()
    with pytest.raises(ValueError):
        plan.step(1)
    assert list(plan.lengths()) == [8] * cfg.n_layers
    gr.free()
    plan.free()
    model.free()

"""Batched decode (bs > 1, BatchDecodePlan): every sequence of the batch against that
sequence decoded alone -- the oracle's step logits and KV rows bit for bit over ragged prompt
lengths, fp32 and fp16 caches and split-K attention, eager and graph-replayed -- and
batch_generate against generate at the C2 geometry; plus the row argmax's tie rule."""
import numpy as np
import pytest

from llamatov_amd import engine as dr
from llamatov_amd import model as M
from llamatov_amd._lib import LT_KV_F16, LT_KV_F32, call

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[gpu-case] {msg}", flush=True)


def bitexact(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


_W = {}


def weights(cfg):
    if cfg.name not in _W:
        _W[cfg.name] = M.synth_weights(cfg, 1234)
    return _W[cfg.name]


@pytest.mark.parametrize("linear", ["gemv", "gemm", "mixed", "gemm+rope", "mixed+rope"])
@pytest.mark.parametrize("kv_dtype,nsplit", [(LT_KV_F32, 1), (LT_KV_F16, 1), (LT_KV_F16, 4)])
def test_batch_rows_equal_lone_sequences(gpu, oracle, kv_dtype, nsplit, linear, monkeypatch):
    """+rope: q|k|v on the GEMM with the RoPE + KV-append epilogue and, in the mixed form with
    one split, O on the GEMM fed by the attention's block-major quants (QKV_GEMM_MIN_BATCH and
    O_GEMM_MIN_BATCH lowered to this batch)."""
    cfg = M.SMALL_QWEN
    case(f"batch vs lone sequences kv={kv_dtype} nsplit={nsplit} linear={linear}")
    linear, rope = linear.split("+")[0], linear.endswith("+rope")
    monkeypatch.setattr(dr, "QKV_GEMM_MIN_BATCH", 1 if rope else 10 ** 6)
    monkeypatch.setattr(dr, "O_GEMM_MIN_BATCH", 1 if rope else 10 ** 6)
    w = weights(cfg)
    model = dr.ResidentModel(cfg, w, gpu)
    lens = [3, 9, 1, 14]
    prompts = [M.random_prompt(cfg, n, seed=40 + i) for i, n in enumerate(lens)]
    plan = dr.BatchDecodePlan(model, len(prompts), dr.Profile(kv_dtype=kv_dtype, attn_nsplit=nsplit), max_ctx=64,
                              linear=linear)
    assert plan.linear == linear and plan.qkv_gemm == rope
    assert plan.o_gemm == (nsplit == 1 and (linear == "gemm" or (rope and linear == "mixed")))
    orcs = [oracle.OracleModel(cfg, w, kv_f16=kv_dtype == LT_KV_F16, attn_nsplit=nsplit) for _ in prompts]
    exp = []
    for b, pr in enumerate(prompts):
        plan.prefill(b, pr)
        for t in pr:
            lg = orcs[b].step(t)
        exp.append(lg)
    got = plan.read_logits()
    for b in range(len(prompts)):
        assert bitexact(got[b], exp[b]), f"prefill logits of sequence {b}"
    assert plan.read_tokens() == [int(np.argmax(e)) for e in exp]
    # eager steps, then graph replays
    gr = dr.BatchStepGraph(plan)
    for i in range(14):
        toks = plan.read_tokens()
        if i < 8:
            plan.step()
        else:
            if i == 8:
                gr.capture()
            gr.replay()
        got = plan.read_logits()
        for b in range(len(prompts)):
            e = orcs[b].step(toks[b])
            assert bitexact(got[b], e), f"step {i} sequence {b}"
    assert plan.length == [n + 14 for n in lens]
    width = cfg.kv_dim
    esz = 2 if kv_dtype == LT_KV_F16 else 4
    dt = np.uint16 if kv_dtype == LT_KV_F16 else np.float32
    for il in (0, cfg.n_layers - 1):
        for which, arr in (("k", plan.k[il]), ("v", plan.v[il])):
            host = arr.to_host().view(dt).reshape(len(prompts), plan.max_ctx, width)
            for b in range(len(prompts)):
                n = plan.length[b]
                assert np.array_equal(host[b, :n], orcs[b].kv_rows(il, which, n)), (il, which, b)
    assert plan.slot_bytes == plan.max_ctx * width * esz
    gr.free()
    plan.free()
    model.free()


@pytest.mark.parametrize("B,linear", [(8, "auto"), (20, "auto"), (20, "gemm"), (40, "auto"), (64, "auto")])
def test_batch_generate_c2_geometry(gpu, B, linear):
    """batch_generate at the C2 model (Qwen2.5-0.5B geometry, B sequences of ragged prompts,
    multi-token GEMV or GEMM linear layers) equals generate per sequence."""
    cfg = M.QWEN25_05B
    case(f"batch_generate C2 x{B} {linear}")
    w = weights(cfg)
    model = dr.ResidentModel(cfg, w, gpu)
    prompts = [M.random_prompt(cfg, 32 - (3 * b) % 29, seed=70 + b) for b in range(B)]
    prof = dr.Profile(kv_dtype=LT_KV_F16)
    got = dr.batch_generate(model, prompts, 24, prof, linear=linear)
    for b, pr in enumerate(prompts):
        assert got[b] == dr.generate(model, pr, 24, prof), f"sequence {b}"
    model.free()


@pytest.mark.parametrize("N,K", [(1152, 896), (896, 4864), (9728, 896), (4096, 14336), (37, 96)])
@pytest.mark.parametrize("T", [1, 3, 8, 11])
def test_gemv_multi_equals_gemv(gpu, oracle, N, K, T):
    """lt_q8_gemv_multi: every token's row values equal the oracle GEMV of that token, for
    every epilogue; lt_rmsnorm_quant_rows equals the per-row oracle norm + quant."""
    from llamatov_amd import _lib
    from llamatov_amd import q8 as hq8
    case(f"gemv_multi N={N} K={K} T={T}")
    rng = np.random.default_rng(N + K + T)
    W = hq8.quantize_rows((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
    X = (rng.standard_normal((T, K)) * 2).astype(np.float32)
    nw = (rng.standard_normal(K) * 0.3 + 1).astype(np.float32)
    xq = dr.DevTensor.empty((T * K,), np.int8, gpu)
    xd = dr.DevTensor.empty((T * K // 32,), np.uint16, gpu)
    call("lt_rmsnorm_quant_rows", gpu.handle, dr.DevTensor.from_host(X, gpu).vp, dr.DevTensor.from_host(nw, gpu).vp,
         xq.vp, xd.vp, T, K, __import__("ctypes").c_float(1e-6))
    eq, ed = zip(*[oracle.quant_q8(oracle.rmsnorm(X[t], nw, 1e-6)) for t in range(T)])
    assert np.array_equal(xq.to_host().reshape(T, K), np.stack(eq))
    assert np.array_equal(xd.to_host().reshape(T, K // 32), np.stack(ed))
    dW = dr.DevTensor.from_host(W, gpu)
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    resid = rng.standard_normal((T, N)).astype(np.float32)
    exp = np.stack([oracle.q8_gemv(W, eq[t], ed[t], K) for t in range(T)])
    for epi, add, want in ((0, None, exp), (0, bias, np.stack([oracle.q8_gemv(W, eq[t], ed[t], K, bias) for t in range(T)])),
                           (1, resid, np.stack([oracle.q8_gemv(W, eq[t], ed[t], K, resid[t]) for t in range(T)]))):
        y = dr.DevTensor.empty((T, N), np.float32, gpu)
        da = dr.DevTensor.from_host(add, gpu) if add is not None else None
        call("lt_q8_gemv_multi", gpu.handle, dW.vp, xq.vp, xd.vp, T, da.vp if da is not None else None, y.vp, N, K, epi)
        assert bitexact(y.to_host(), want), f"epi {epi}"
    if N % 2 == 0:
        y = dr.DevTensor.empty((T, N // 2), np.float32, gpu)
        call("lt_q8_gemv_multi", gpu.handle, dW.vp, xq.vp, xd.vp, T, None, y.vp, N, K, 2)
        want = np.stack([oracle.silu_mul(exp[t][0::2], exp[t][1::2]) for t in range(T)])
        assert bitexact(y.to_host(), want), "silu"


@pytest.mark.parametrize("nh,nkv,hd,K", [(14, 2, 64, 896), (8, 2, 128, 1024), (4, 4, 64, 96)])
@pytest.mark.parametrize("T", [1, 3, 8, 13])
@pytest.mark.parametrize("kv_dtype", [LT_KV_F16, LT_KV_F32])
def test_gemv_multi_rope_equals_gemv_then_rope(gpu, nh, nkv, hd, K, T, kv_dtype):
    """lt_q8_gemv_multi_rope equals lt_q8_gemv_multi (bias) followed by lt_rope_append_seqs:
    the q|k|v buffer and both caches byte for byte, with positions spread over the cache and
    one past its end (no append)."""
    from llamatov_amd import q8 as hq8
    case(f"gemv_multi_rope nh={nh} nkv={nkv} hd={hd} K={K} T={T} kv={kv_dtype}")
    rng = np.random.default_rng(T * 7 + nh + kv_dtype)
    N, maxt = (nh + 2 * nkv) * hd, 40
    W = dr.DevTensor.from_host(hq8.quantize_rows((rng.standard_normal((N, K)) * 0.05).astype(np.float32)), gpu)
    xq = dr.DevTensor.from_host(rng.integers(-127, 128, (T, K), dtype=np.int64).astype(np.int8), gpu)
    xd = dr.DevTensor.from_host((rng.random((T, K // 32)) * 0.05 + 0.01).astype(np.float16).view(np.uint16), gpu)
    bias = dr.DevTensor.from_host((rng.standard_normal(N) * 0.1).astype(np.float32), gpu)
    pos = rng.integers(0, maxt, T).astype(np.int32)
    if T > 2:
        pos[1] = maxt          # past the cache: rotated q, no append
    lens = dr.DevTensor.from_host(pos, gpu)
    freqs = dr.DevTensor.from_host((10000.0 ** (-np.arange(hd // 2) * 2.0 / hd)).astype(np.float32), gpu)
    eb = 2 if kv_dtype == LT_KV_F16 else 4
    init = rng.integers(0, 255, T * maxt * nkv * hd * eb, dtype=np.int64).astype(np.uint8)
    outs = []
    for fused in (False, True):
        qkv = dr.DevTensor.empty((T, N), np.float32, gpu)
        kc, vc = dr.DevTensor.from_host(init, gpu), dr.DevTensor.from_host(init[::-1].copy(), gpu)
        if fused:
            call("lt_q8_gemv_multi_rope", gpu.handle, W.vp, xq.vp, xd.vp, T, bias.vp, qkv.vp, N, K, lens.vp, nh, nkv,
                 hd, freqs.vp, kc.vp, vc.vp, maxt, kv_dtype)
        else:
            call("lt_q8_gemv_multi", gpu.handle, W.vp, xq.vp, xd.vp, T, bias.vp, qkv.vp, N, K, 0)
            call("lt_rope_append_seqs", gpu.handle, qkv.vp, T, N, lens.vp, nh, nkv, hd, freqs.vp, kc.vp, vc.vp, maxt,
                 kv_dtype)
        outs.append((qkv.to_host(), kc.to_host(), vc.to_host()))
        for t in (qkv, kc, vc):
            t.free()
    assert bitexact(outs[0][0], outs[1][0]), "q|k|v rows"
    assert np.array_equal(outs[0][1], outs[1][1]) and np.array_equal(outs[0][2], outs[1][2]), "caches"
    for t in (W, xq, xd, bias, lens, freqs):
        t.free()


@pytest.mark.parametrize("nh,nkv,hd,K,T", [(14, 2, 64, 896, 1), (14, 2, 64, 896, 13), (14, 2, 64, 896, 64),
                                          (14, 2, 64, 896, 70), (8, 2, 128, 1024, 8), (4, 4, 64, 96, 33),
                                          (32, 8, 128, 4096, 5)])
@pytest.mark.parametrize("kv_dtype", [LT_KV_F16, LT_KV_F32])
@pytest.mark.parametrize("static", ["1", "0"])
def test_gemm_rope_equals_gemm_then_rope(gpu, nh, nkv, hd, K, T, kv_dtype, static, monkeypatch):
    """lt_q8_gemm_rope_t (weights in lt_q8_tiles_rope's order) equals lt_q8_gemm_t (bias) on
    the plain tile copy followed by lt_rope_append_seqs: the q|k|v buffer and both caches
    byte for byte, with positions spread over the cache and one past its end (no append);
    both leaf-split schedules (LT_GEMM_LS_STATIC)."""
    from llamatov_amd import q8 as hq8
    monkeypatch.setenv("LT_GEMM_LS_STATIC", static)
    case(f"gemm_rope nh={nh} nkv={nkv} hd={hd} K={K} T={T} kv={kv_dtype} static={static}")
    rng = np.random.default_rng(T * 5 + nh + kv_dtype)
    N, maxt = (nh + 2 * nkv) * hd, 40
    W = dr.DevTensor.from_host(hq8.quantize_rows((rng.standard_normal((N, K)) * 0.05).astype(np.float32)), gpu)
    n = int(dr._lib.raw("lt_q8_tiles_bytes")(N, K))
    Wt, Wr = dr.DevTensor.empty((n,), np.uint8, gpu), dr.DevTensor.empty((n,), np.uint8, gpu)
    call("lt_q8_tiles", gpu.handle, W.vp, Wt.vp, N, K)
    call("lt_q8_tiles_rope", gpu.handle, W.vp, Wr.vp, N, K, nh, nkv, hd)
    X = dr.DevTensor.from_host((rng.standard_normal((T, K)) * 2.0).astype(np.float32), gpu)
    xq, xd = dr.DevTensor.empty((T * K,), np.int8, gpu), dr.DevTensor.empty((T * K // 32,), np.uint16, gpu)
    call("lt_quant_q8_bm", gpu.handle, X.vp, xq.vp, xd.vp, T, K)
    bias = dr.DevTensor.from_host((rng.standard_normal(N) * 0.1).astype(np.float32), gpu)
    pos = rng.integers(0, maxt, T).astype(np.int32)
    if T > 2:
        pos[1] = maxt          # past the cache: rotated q, no append
    lens = dr.DevTensor.from_host(pos, gpu)
    freqs = dr.DevTensor.from_host((10000.0 ** (-np.arange(hd // 2) * 2.0 / hd)).astype(np.float32), gpu)
    eb = 2 if kv_dtype == LT_KV_F16 else 4
    init = rng.integers(0, 255, T * maxt * nkv * hd * eb, dtype=np.int64).astype(np.uint8)
    outs = []
    for fused in (False, True):
        qkv = dr.DevTensor.empty((T, N), np.float32, gpu)
        kc, vc = dr.DevTensor.from_host(init, gpu), dr.DevTensor.from_host(init[::-1].copy(), gpu)
        if fused:
            call("lt_q8_gemm_rope_t", gpu.handle, Wr.vp, xq.vp, xd.vp, T, bias.vp, qkv.vp, N, K, lens.vp, nh, nkv,
                 hd, freqs.vp, kc.vp, vc.vp, maxt, kv_dtype)
        else:
            call("lt_q8_gemm_t", gpu.handle, Wt.vp, xq.vp, xd.vp, bias.vp, None, qkv.vp, T, N, K)
            call("lt_rope_append_seqs", gpu.handle, qkv.vp, T, N, lens.vp, nh, nkv, hd, freqs.vp, kc.vp, vc.vp, maxt,
                 kv_dtype)
        outs.append((qkv.to_host(), kc.to_host(), vc.to_host()))
        for t in (qkv, kc, vc):
            t.free()
    assert bitexact(outs[0][0], outs[1][0]), "q|k|v rows"
    assert np.array_equal(outs[0][1], outs[1][1]) and np.array_equal(outs[0][2], outs[1][2]), "caches"
    for t in (W, Wt, Wr, X, xq, xd, bias, lens, freqs):
        t.free()


def test_argmax_rows_tie_rule(gpu):
    case("argmax rows")
    rng = np.random.default_rng(5)
    R, V = 5, 151936
    x = np.round(rng.standard_normal((R, V)), 1).astype(np.float32)
    x[2, [7, 100, 150000]] = 50.0
    x[3, :] = -np.inf
    x[4, 9000:] = np.float32(3.5)
    x[4, :9000] = np.float32(-1)
    d = dr.DevTensor.from_host(x, gpu)
    out = dr.DevTensor.empty((R,), np.int32, gpu)
    call("lt_argmax_rows", gpu.handle, d.vp, R, V, out.vp, None, None, 0)
    exp = [int(np.argmax(r)) for r in x]
    assert list(out.to_host()) == exp
    # the sliced variant: ties across slice boundaries (19456 elements a slice here), a row of
    # -inf, NaN never chosen, small rows (most slices empty), and the history append
    x[1, [19455, 19456, 140000]] = 60.0
    x[0, 3] = np.nan
    x[0, 5] = 70.0
    d = dr.DevTensor.from_host(x, gpu)
    exp = [int(np.argmax(np.where(np.isnan(r), -np.inf, r))) for r in x]
    from llamatov_amd import _lib
    for n in (V, 100):
        ws_n = int(_lib.raw("lt_argmax_rows_workspace_size")(R))
        ws = dr.DevTensor.empty((ws_n,), np.uint8, gpu)
        hist = dr.DevTensor.from_host(np.full((R, 4), -7, np.int32), gpu)
        cnt = dr.DevTensor.from_host(np.array([0, 1, 3, 4, 2], np.int32), gpu)
        xs = d if n == V else dr.DevTensor.from_host(np.ascontiguousarray(x[:, :n]), gpu)
        call("lt_argmax_rows_ws", gpu.handle, xs.vp, R, n, out.vp, hist.vp, cnt.vp, 4, ws.vp, ws_n)
        want = exp if n == V else [int(np.argmax(np.where(np.isnan(r), -np.inf, r))) for r in x[:, :n]]
        assert list(out.to_host()) == want, n
        h = hist.to_host()
        for r, c in enumerate([0, 1, 3, 4, 2]):
            assert (h[r, c] == want[r]) if c < 4 else (h[r] == -7).all()
        assert list(cnt.to_host()) == [1, 2, 4, 4, 3]


@pytest.mark.parametrize("nh,nkv,hd", [(14, 2, 64), (32, 8, 128), (8, 2, 32)])
@pytest.mark.parametrize("kv_dtype,nsplit", [(LT_KV_F16, 1), (LT_KV_F32, 1), (LT_KV_F16, 4)])
def test_attn_rows_q8_equals_attn_then_quant(gpu, nh, nkv, hd, kv_dtype, nsplit):
    """lt_attn_decode_rows_q8 (the attention writing the O projection's activation quants):
    bit-identical to lt_attn_decode_rows followed by lt_quant_q8 over the rows, with and
    without the fp32 rows, over ragged lengths (hd 32 runs the 256-thread kernel)."""
    from llamatov_amd import _lib
    import ctypes
    case(f"attn rows q8 nh={nh} nkv={nkv} hd={hd} kv={kv_dtype} nsplit={nsplit}")
    rng = np.random.default_rng(nh * hd + nsplit)
    B, maxt = 5, 96
    qs = nh * hd + 2 * nkv * hd   # q|k|v rows
    q = rng.standard_normal((B, qs)).astype(np.float32)
    dt = np.float16 if kv_dtype == LT_KV_F16 else np.float32
    kc = rng.standard_normal((B, maxt, nkv * hd)).astype(dt)
    vc = rng.standard_normal((B, maxt, nkv * hd)).astype(dt)
    lens = np.array([1, 17, 96, 40, 63], np.int32)
    dq, dk, dv, dl = (dr.DevTensor.from_host(a, gpu) for a in (q, kc, vc, lens))
    ws_n = max(_lib.raw("lt_attn_workspace_size")(B, nh, hd, nsplit), 16)
    ws = dr.DevTensor.empty((ws_n,), np.uint8, gpu)
    QD = nh * hd
    ref = dr.DevTensor.empty((B * QD,), np.float32, gpu)
    common = (B, nh, nkv, hd, ctypes.c_float(hd ** -0.5), maxt, nsplit, kv_dtype, ws.vp, ws_n)
    call("lt_attn_decode_rows", gpu.handle, dq.vp, qs, dk.vp, dv.vp, dl.vp, ref.vp, *common)
    rq = dr.DevTensor.empty((B * QD,), np.int8, gpu)
    rd = dr.DevTensor.empty((B * QD // 32,), np.uint16, gpu)
    call("lt_quant_q8", gpu.handle, ref.vp, rq.vp, rd.vp, B * QD)
    for with_out in (False, True):
        out = dr.DevTensor.empty((B * QD,), np.float32, gpu) if with_out else None
        oq = dr.DevTensor.empty((B * QD,), np.int8, gpu)
        od = dr.DevTensor.empty((B * QD // 32,), np.uint16, gpu)
        call("lt_attn_decode_rows_q8", gpu.handle, dq.vp, qs, dk.vp, dv.vp, dl.vp, out.vp if out else None, oq.vp,
             od.vp, *common)
        assert np.array_equal(oq.to_host(), rq.to_host())
        assert np.array_equal(od.to_host(), rd.to_host())
        if out is not None:
            assert bitexact(out.to_host(), ref.to_host())
    if nsplit == 1:
        # the block-major variant: lt_quant_q8_bm of the fp32 rows
        bq = dr.DevTensor.empty((B * QD,), np.int8, gpu)
        bd = dr.DevTensor.empty((B * QD // 32,), np.uint16, gpu)
        call("lt_quant_q8_bm", gpu.handle, ref.vp, bq.vp, bd.vp, B, QD)
        oq = dr.DevTensor.empty((B * QD,), np.int8, gpu)
        od = dr.DevTensor.empty((B * QD // 32,), np.uint16, gpu)
        call("lt_attn_decode_rows_q8_bm", gpu.handle, dq.vp, qs, dk.vp, dv.vp, dl.vp, None, oq.vp, od.vp, B, nh, nkv,
             hd, ctypes.c_float(hd ** -0.5), maxt, kv_dtype)
        assert np.array_equal(oq.to_host(), bq.to_host()), "block-major quants"
        assert np.array_equal(od.to_host(), bd.to_host()), "block-major scales"

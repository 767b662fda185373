"""The planar weight layout: lt_q8_to_planar's bytes against a numpy restatement of the
layout, every *_pl GEMV against its namesake over the GGUF blocks (outputs equal bit for bit,
and against the oracle where the namesake's tests do not already pin it), rows whose last
32-block group is partial (K % 1024 != 0), the K % 32 refusal, and decode through planar
copies equal to decode through the blocks and to the oracle."""
import ctypes

import numpy as np
import pytest

from llamatov_amd import _lib
from llamatov_amd import engine as dr
from llamatov_amd import model as M
from llamatov_amd._lib import LT_KV_F16, LT_KV_F32, call

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[gpu-case] {msg}", flush=True)


def bits(a):
    return np.asarray(a).view(np.uint32)


def rand_blocks(rng, N, K):
    nb = K // 32
    blk = np.empty((N, nb, 34), np.uint8)
    blk[..., 2:] = rng.integers(-127, 128, size=(N, nb, 32), dtype=np.int8).view(np.uint8)
    blk[..., :2] = (rng.standard_normal((N, nb)) * 0.02).astype(np.float16).view(np.uint8).reshape(N, nb, 2)
    return blk.reshape(N, nb * 34)


def planar_host(blocks, N, K):
    """The layout restated: per row, per group of up to 32 blocks (the last group of a row
    may hold fewer), the leading 16 quants of the group's blocks, then their trailing 16;
    then the scales [N][nb]."""
    nb = K // 32
    b = blocks.reshape(N, nb, 34)
    rows = []
    for k0 in range(0, nb, 32):
        q = b[:, k0:k0 + 32, 2:]                          # [N][m blocks][32 quants]
        m = q.shape[1]
        rows.append(np.concatenate([q[..., :16].reshape(N, 16 * m), q[..., 16:].reshape(N, 16 * m)], axis=1))
    quant = np.concatenate(rows, axis=1)                  # [N][nb * 32]
    scales = b[..., :2].reshape(N, nb * 2)
    return np.concatenate([quant.reshape(-1), scales.reshape(-1)])


def up(a):
    return dr.DevTensor.from_host(np.ascontiguousarray(a))


def planar_copy(gpu, W, N, K):
    t = dr.DevTensor.empty((W.nbytes,), np.uint8)
    call("lt_q8_to_planar", gpu.handle, W.vp, t.vp, N, K)
    return t


@pytest.mark.parametrize("N,K", [(37, 1024), (8, 14336), (300, 4096), (33, 896), (5, 4864), (7, 32)])
def test_planar_repack_layout(gpu, N, K):
    case(f"planar repack {N}x{K}")
    blk = rand_blocks(np.random.default_rng(N), N, K)
    W = up(blk)
    P = planar_copy(gpu, W, N, K)
    assert np.array_equal(P.to_host(), planar_host(blk, N, K))
    W.free()
    P.free()


def test_planar_refuses_k_outside_the_layout(gpu):
    case("planar refusal")
    W = dr.DevTensor.empty((64 * 28 * 34,), np.uint8)
    y = dr.DevTensor.empty((64 * 28 * 34,), np.uint8)
    xq = dr.DevTensor.empty((896,), np.int8)
    xd = dr.DevTensor.empty((28,), np.uint16)
    rc = _lib.raw("lt_q8_to_planar")(gpu.handle, W.vp, y.vp, 64, 880)
    assert rc == -1 and "multiple of 32" in _lib.last_error()
    rc = _lib.raw("lt_q8_gemv_pl")(gpu.handle, W.vp, xq.vp, xd.vp, None, y.vp, 64, 880)
    assert rc == -1 and "multiple of 32" in _lib.last_error()
    for t in (W, y, xq, xd):
        t.free()


SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336), (6144, 4096), (333, 1024), (1000, 2048), (151936, 896),
          (896, 4864), (1152, 896), (70, 96)]


@pytest.mark.parametrize("N,K", SHAPES)
def test_planar_gemv_stage_equals_blocks(gpu, oracle, N, K):
    """lt_q8_gemv_pl against lt_q8_gemv (staged quantized activation), with and without the
    residual, and against the oracle's GEMV."""
    case(f"planar gemv {N}x{K}")
    rng = np.random.default_rng(K + N)
    blk = rand_blocks(rng, N, K)
    W = up(blk)
    P = planar_copy(gpu, W, N, K)
    xq_h = rng.integers(-127, 128, K, dtype=np.int64).astype(np.int8)
    xd_h = (rng.standard_normal(K // 32) * 0.05).astype(np.float16).view(np.uint16)
    xq, xd = up(xq_h), up(xd_h)
    res = up(rng.standard_normal(N).astype(np.float32))
    ya, yb = dr.DevTensor.empty((N,), np.float32), dr.DevTensor.empty((N,), np.float32)
    for r in (None, res):
        call("lt_q8_gemv", gpu.handle, W.vp, xq.vp, xd.vp, None if r is None else r.vp, ya.vp, N, K)
        call("lt_q8_gemv_pl", gpu.handle, P.vp, xq.vp, xd.vp, None if r is None else r.vp, yb.vp, N, K)
        a, b = ya.to_host(), yb.to_host()
        assert np.array_equal(bits(a), bits(b))
    exp = oracle.q8_gemv(blk, xq_h, xd_h, K)
    call("lt_q8_gemv_pl", gpu.handle, P.vp, xq.vp, xd.vp, None, yb.vp, N, K)
    assert np.array_equal(bits(yb.to_host()), bits(exp))
    for t in (W, P, xq, xd, res, ya, yb):
        t.free()


@pytest.mark.parametrize("N,K", [(6144, 4096), (4096, 4096), (1000, 2048), (5000, 14336), (1152, 896), (96, 4864)])
def test_planar_rms_and_embed_equal_blocks(gpu, N, K):
    """lt_q8_gemv_rms_pl (with a bias and without) and lt_q8_gemv_embed_rms_pl against their
    namesakes."""
    case(f"planar rms / embed {N}x{K}")
    rng = np.random.default_rng(7 + N)
    blk = rand_blocks(rng, N, K)
    W = up(blk)
    P = planar_copy(gpu, W, N, K)
    x = up(rng.standard_normal(K).astype(np.float32))
    nw = up((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    bias = up(rng.standard_normal(N).astype(np.float32))
    ya, yb = dr.DevTensor.empty((N,), np.float32), dr.DevTensor.empty((N,), np.float32)
    eps = ctypes.c_float(1e-5)
    for bv in (None, bias):
        call("lt_q8_gemv_rms", gpu.handle, x.vp, nw.vp, eps, W.vp, None if bv is None else bv.vp, ya.vp, N, K)
        call("lt_q8_gemv_rms_pl", gpu.handle, x.vp, nw.vp, eps, P.vp, None if bv is None else bv.vp, yb.vp, N, K)
        assert np.array_equal(bits(ya.to_host()), bits(yb.to_host()))
    if K <= 4096:
        vocab = 50
        emb = up(rand_blocks(rng, vocab, K))
        xo = dr.DevTensor.empty((K,), np.float32)
        err = up(np.zeros(1, np.int32))
        for t in (7, 49):
            tok = up(np.array([t], np.int32))
            call("lt_q8_gemv_embed_rms", gpu.handle, emb.vp, tok.vp, vocab, xo.vp, err.vp, nw.vp, eps, W.vp,
                 bias.vp, ya.vp, N, K)
            call("lt_q8_gemv_embed_rms_pl", gpu.handle, emb.vp, tok.vp, vocab, xo.vp, err.vp, nw.vp, eps, P.vp,
                 bias.vp, yb.vp, N, K)
            assert np.array_equal(bits(ya.to_host()), bits(yb.to_host()))
            tok.free()
        assert err.to_host()[0] == 0
        for t in (emb, xo, err):
            t.free()
    for t in (W, P, x, nw, bias, ya, yb):
        t.free()


@pytest.mark.parametrize("F,K", [(14336, 4096), (2048, 1024), (4864, 896)])
def test_planar_rms_silu_equals_blocks(gpu, F, K):
    case(f"planar rms_silu F={F} K={K}")
    rng = np.random.default_rng(F)
    blk = rand_blocks(rng, 2 * F, K)
    W = up(blk)
    P = planar_copy(gpu, W, 2 * F, K)
    x = up(rng.standard_normal(K).astype(np.float32))
    nw = up((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    eps = ctypes.c_float(1e-5)
    outs = []
    for name, w in (("lt_q8_gemv_rms_silu", W), ("lt_q8_gemv_rms_silu_pl", P)):
        vq = dr.DevTensor.empty((F,), np.int8)
        vd = dr.DevTensor.empty((F // 32,), np.uint16)
        call(name, gpu.handle, x.vp, nw.vp, eps, w.vp, vq.vp, vd.vp, F, K)
        outs.append((vq.to_host(), vd.to_host()))
        vq.free()
        vd.free()
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    for t in (W, P, x, nw):
        t.free()


@pytest.mark.parametrize("nsplit", [1, 4])
def test_planar_attn_out_equals_blocks(gpu, nsplit):
    """lt_q8_gemv_attn_out_pl: the quantized attention (nsplit 1) or the split partials merged
    in the prologue, O GEMV + residual, the length bump."""
    nh, hd, N = 32, 128, 4096
    K = nh * hd
    case(f"planar attn_out nsplit={nsplit}")
    rng = np.random.default_rng(nsplit)
    blk = rand_blocks(rng, N, K)
    W = up(blk)
    P = planar_copy(gpu, W, N, K)
    xq = up(rng.integers(-127, 128, K, dtype=np.int64).astype(np.int8))
    xd = up((rng.standard_normal(K // 32) * 0.05).astype(np.float16).view(np.uint16))
    res = up(rng.standard_normal(N).astype(np.float32))
    wsn = int(_lib.raw("lt_attn_workspace_size")(1, nh, hd, nsplit))
    ws = None
    if nsplit > 1:
        # partials: finite maxima, positive sums, random outputs (the workspace layout's
        # regions filled as one float array)
        ws = up(np.abs(rng.standard_normal(wsn // 4)).astype(np.float32) + 0.5)
    outs = []
    for name, w in (("lt_q8_gemv_attn_out", W), ("lt_q8_gemv_attn_out_pl", P)):
        y = dr.DevTensor.empty((N,), np.float32)
        ln = up(np.array([5], np.int32))
        call(name, gpu.handle, xq.vp, xd.vp, None if ws is None else ws.vp, wsn, nsplit, nh, hd, w.vp, res.vp,
             y.vp, N, K, ln.vp, 100)
        outs.append((y.to_host(), ln.to_host()[0]))
        y.free()
        ln.free()
    assert np.array_equal(bits(outs[0][0]), bits(outs[1][0]))
    assert outs[0][1] == outs[1][1] == 6
    for t in (W, P, xq, xd, res) + ((ws,) if ws is not None else ()):
        t.free()


@pytest.mark.parametrize("N,K", [(128256, 4096), (3000, 1024), (151936, 896)])
def test_planar_rms_argmax_equals_blocks(gpu, N, K):
    case(f"planar rms_argmax {N}x{K}")
    rng = np.random.default_rng(3)
    blk = rand_blocks(rng, N, K)
    W = up(blk)
    P = planar_copy(gpu, W, N, K)
    x = up(rng.standard_normal(K).astype(np.float32))
    nw = up((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    eps = ctypes.c_float(1e-6)
    wsn = int(_lib.raw("lt_q8_gemv_argmax_workspace_size")(N))
    ws = dr.DevTensor.empty((wsn,), np.uint8)
    outs = []
    for name, w in (("lt_q8_gemv_rms_argmax", W), ("lt_q8_gemv_rms_argmax_pl", P)):
        lg = dr.DevTensor.empty((N,), np.float32)
        out = up(np.array([-1], np.int32))
        hist = up(np.zeros(4, np.int32))
        cnt = up(np.zeros(1, np.int32))
        call(name, gpu.handle, x.vp, nw.vp, eps, w.vp, lg.vp, N, K, out.vp, hist.vp, cnt.vp, 4, ws.vp, wsn)
        outs.append((lg.to_host(), out.to_host()[0], hist.to_host()[0], cnt.to_host()[0]))
        for t in (lg, out, hist, cnt):
            t.free()
    assert np.array_equal(bits(outs[0][0]), bits(outs[1][0]))
    assert outs[0][1:] == outs[1][1:] and outs[1][1] == int(np.argmax(outs[1][0])) and outs[1][3] == 1
    for t in (W, P, x, nw, ws):
        t.free()


# a small geometry whose every K is a multiple of 1024: n_embd 1024, 16 heads of 64, FFN 2048
PLANAR_SMALL = M.SMALL_QWEN.replace(name="small-planar", n_embd=1024, n_ff=2048, n_head=16, n_head_kv=4,
                                    n_layers=3, vocab=3000)


@pytest.mark.parametrize("kv_dtype,nsplit", [(LT_KV_F32, 1), (LT_KV_F16, 4)])
def test_planar_decode_equals_blocks_and_oracle(gpu, oracle, kv_dtype, nsplit):
    """The five-launch step over planar copies: eager steps and graph replays, logits equal to
    the step over the blocks and to the oracle."""
    cfg = PLANAR_SMALL
    case(f"planar decode kv={kv_dtype} nsplit={nsplit}")
    w = M.synth_weights(cfg, seed=11)
    m = dr.ResidentModel(cfg, w, gpu, layouts="fused")
    prof = dr.Profile(kv_dtype=kv_dtype, attn_nsplit=nsplit, persistent_step=False)
    pp = dr.DecodePlan(m, prof)
    pb = dr.DecodePlan(m, dr.Profile(kv_dtype=kv_dtype, attn_nsplit=nsplit, persistent_step=False, planar=False))
    assert pp.planar and not pb.planar
    orc = oracle.OracleModel(cfg, w, kv_f16=kv_dtype == LT_KV_F16, attn_nsplit=nsplit)
    toks = M.random_prompt(cfg, 6, seed=2)
    for i in range(14):
        t = toks[i] if i < len(toks) else int(np.argmax(exp))
        pp.step(t)
        pb.step(t)
        exp = orc.step(t)
        got = pp.read_logits()
        assert np.array_equal(bits(got), bits(pb.read_logits())), f"step {i}: planar vs blocks"
        assert np.array_equal(bits(got), bits(exp)), f"step {i}: planar vs oracle"
        assert pp.read_token() == oracle.argmax(exp)
    gr = dr.StepGraph(pp)
    gr.capture()
    for i in range(6):
        t = int(np.argmax(exp))
        lg = gr.replay_logits(t)
        exp = orc.step(t)
        assert np.array_equal(bits(lg), bits(exp)), f"replay {i}"
    assert pp.error() == 0
    gr.free()
    pp.free()
    pb.free()
    m.free()

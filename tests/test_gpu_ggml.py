"""The ggml-compatible numerics profile on the device (lt_ggml.hip) against the oracle's
ggml restatement (pinned against the reference's compiled CPU substrate in
test_oracle_ggml.py): quantizer, both dot orders, the two qmatmul drivers and the decode
step under numerics="ggml", bit for bit."""
import ctypes

import numpy as np
import pytest

from llamatov_amd import _lib
from llamatov_amd import engine as dr
from llamatov_amd import model as M
from llamatov_amd import q8 as hq8
from llamatov_amd._lib import LT_GGML_LLAMAFILE, LT_GGML_VEC, LT_KV_F16, LT_KV_F32, call

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
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]}"


def activations(rng, n, K):
    """Mixed magnitudes, exact zeros, a zero block, exact .5 ties under id = 1."""
    X = rng.standard_normal((n, K)) * np.repeat(np.exp(rng.uniform(-6, 6, (n, K // 32))), 32, axis=1)
    X = X.astype(np.float32)
    X[:, 5] = 0.0
    if K >= 64:
        X[0, 32:64] = 0.0
    X[-1, 0] = 127.0
    X[-1, 1:32] = np.float32(22.5) * np.sign(np.arange(1, 32) - 16)
    return X


def rand_weight(rng, N, K):
    return hq8.quantize_rows((rng.standard_normal((N, K)) * 0.05).astype(np.float32))


@pytest.mark.parametrize("K", [32, 896, 4864, 14336])
def test_quant_ggml(gpu, oracle, K):
    case(f"ggml quant K={K}")
    rng = np.random.default_rng(K)
    for x in activations(rng, 3, K):
        xq, xd = empty((K,), np.int8), empty((K // 32,), np.uint16)
        call("lt_quant_q8_ggml", gpu.handle, up(x).vp, xq.vp, xd.vp, K)
        eq, ed = oracle.quant_q8_ggml(x)
        assert_bitexact(xq.to_host(), eq, "quants")
        assert_bitexact(xd.to_host(), ed, "scales")
        yb = empty((K // 32 * 34,), np.uint8)
        call("lt_quant_q8_0_ggml", gpu.handle, up(x).vp, yb.vp, K)
        assert_bitexact(yb.to_host(), oracle.quant_q8_0_ggml_blocks(x), "blocks")


@pytest.mark.parametrize("order", [LT_GGML_VEC, LT_GGML_LLAMAFILE])
@pytest.mark.parametrize("N,K,bias", [(16, 32, False), (40, 96, True), (33, 928, False), (896, 896, True),
                                      (4864, 896, False), (896, 4864, True), (1152, 896, True),
                                      (151936, 896, False), (300, 14336, False), (4096, 4096, True)])
def test_q8_gemv_ggml(gpu, oracle, order, N, K, bias):
    case(f"ggml gemv order={order} N={N} K={K} bias={bias}")
    rng = np.random.default_rng(N + K)
    W = rand_weight(rng, N, K)
    xq, xd = oracle.quant_q8_ggml(activations(rng, 1, K)[0])
    b = (rng.standard_normal(N) * 0.1).astype(np.float32) if bias else None
    exp = oracle.q8_gemv_ggml(W, xq, xd, K, order, b)
    y = empty((N,), np.float32)
    call("lt_q8_gemv_ggml", gpu.handle, up(W).vp, up(xq).vp, up(xd).vp, up(b).vp if bias else None, y.vp,
         N, K, order)
    assert_bitexact(y.to_host(), exp, f"gemv order {order}")


@pytest.mark.parametrize("M_", [1, 2, 3, 5, 8])
def test_qmatmul_drivers(gpu, oracle, M_):
    rng = np.random.default_rng(40 + M_)
    N, K = 1152, 896
    W = rand_weight(rng, N, K)
    X = activations(rng, M_, K)
    dW, dX = up(W), up(X)
    ws_n = _lib.raw("lt_qmatmul_q8_0_workspace_size")(M_, K)
    ws = empty((ws_n,), np.uint8)
    case(f"qmatmul ggml M={M_}")
    out = empty((M_, N), np.float32)
    call("lt_qmatmul_q8_0_ggml", gpu.handle, dW.vp, dX.vp, out.vp, M_, N, K, ws.vp, ws_n)
    assert_bitexact(out.to_host(), oracle.qmatmul_q8_0_ggml(W, X, N, K), "qmatmul vec")
    case(f"qmatmul llamafile M={M_}")
    out2 = empty((M_, N), np.float32)
    call("lt_qmatmul_q8_0_llamafile", gpu.handle, dW.vp, dX.vp, out2.vp, N, M_, K, ws.vp, ws_n)
    assert_bitexact(out2.to_host(), oracle.qmatmul_q8_0_llamafile(W, X, N, K), "qmatmul llamafile")
    # a short workspace is refused before any launch
    assert _lib.raw("lt_qmatmul_q8_0_ggml")(gpu.handle, dW.vp, dX.vp, out.vp, M_, N, K, ws.vp, ws_n - 1) == -1


def test_ggml_gemv_limits(gpu):
    case("ggml gemv limits")
    W, xq, xd, y = empty((34 * 2,), np.uint8), empty((64,), np.int8), empty((2,), np.uint16), empty((1,), np.float32)
    f = _lib.raw("lt_q8_gemv_ggml")
    assert f(gpu.handle, W.vp, xq.vp, xd.vp, None, y.vp, 1, 20480 + 32, LT_GGML_LLAMAFILE) == -1
    assert f(gpu.handle, W.vp, xq.vp, xd.vp, None, y.vp, 1, 40960 + 32, LT_GGML_VEC) == -1
    assert f(gpu.handle, W.vp, xq.vp, xd.vp, None, y.vp, 1, 64, 7) == -1
    assert f(gpu.handle, W.vp, xq.vp, xd.vp, None, y.vp, 1, 48, LT_GGML_VEC) == -1


_W = {}


def weights(cfg):
    if cfg.name not in _W:
        _W[cfg.name] = M.synth_weights(cfg, 1234)
    return _W[cfg.name]


@pytest.mark.parametrize("cfg_name,kv_dtype", [("tiny", LT_KV_F32), ("small-qwen-arch", LT_KV_F16)])
def test_decode_step_ggml_numerics(gpu, oracle, cfg_name, kv_dtype):
    """The decode step under numerics="ggml" against the oracle's ggml-numerics step, logits
    bit for bit, eager and graph-replayed; the engine numerics give different logits."""
    cfg = M.CONFIGS[cfg_name]
    case(f"ggml decode {cfg_name} kv={kv_dtype}")
    w = weights(cfg)
    model = dr.ResidentModel(cfg, w, gpu)
    prof = dr.Profile(fused_step=False, numerics="ggml", kv_dtype=kv_dtype)
    plan = dr.DecodePlan(model, prof)
    orc = oracle.OracleModel(cfg, w, kv_f16=kv_dtype == LT_KV_F16, numerics="ggml")
    eng = oracle.OracleModel(cfg, w, kv_f16=kv_dtype == LT_KV_F16)
    toks = M.random_prompt(cfg, 6, seed=5)
    differs = False
    for i in range(16):
        t = toks[i] if i < len(toks) else int(np.argmax(exp))
        plan.step(t)
        exp = orc.step(t)
        differs |= not np.array_equal(exp, eng.step(t))
        assert_bitexact(plan.read_logits(), exp, f"step {i}")
    assert differs
    with pytest.raises(ValueError):
        dr.forward_prefill(plan, toks)
    gr = dr.StepGraph(plan)
    gr.capture()
    t = int(np.argmax(exp))
    for i in range(6):
        lg = gr.replay_logits(t)
        exp = orc.step(t)
        assert_bitexact(lg, exp, f"replay {i}")
        t = int(np.argmax(exp))
    gr.free()
    plan.free()
    model.free()


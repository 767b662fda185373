"""The batched prefill path: the int8-MFMA Q8_0 GEMM against the oracle's GEMV per token,
and a batched prefill against the token-by-token prefill (the reference's device-uniform
requirement, bpd/lib/dev_residency.py:1338-1356): KV cache, logits and the continued greedy
stream bit-identical."""
import numpy as np
import pytest

from llamatov_amd import dev_residency as dr
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
    la = dr.forward_pass_resident(a, prompt)
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
    gb = dr.GraphRunner(b)
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

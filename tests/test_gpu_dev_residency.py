"""The reference's host surface (llamatov_amd.dev_residency, llamatov_amd.llamatov_run) driven
in the reference's own call order, on the reference's kind of inputs (an fp32 weight dict in
GGUF [ne0, ne1] orientation, a cfg dict, torch tensors), checked against the oracle.

The driver sequence follows the reference's referee (bpd/kernelgen/referee/
rms_quant_prod_ab.py:21-35): apply_production_profile(); kv = [None] * n_layers;
gr = GraphRunner(w, cfg, kv); gr.seed(prompt, arange); t = argmax; gr.capture([t], [len]);
t = gr.replay_token([t]) ...
"""
import ctypes

import numpy as np
import pytest
import torch

from llamatov_amd import dev_residency as dr
from llamatov_amd import model as M
from llamatov_amd import q8 as hq8
from llamatov_amd._lib import LT_KV_F16

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[gpu-case] {msg}", flush=True)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def reference_w(cfg, qw):
    """The reference loader's view of a Q8_0 model: fp32 tensors, 2-D as [ne0, ne1]
    (inputs x outputs; token_embd n_embd x vocab), as torch tensors."""
    w = {}
    for name, kind, shape in M.weight_specs(cfg):
        a = qw[name]
        if kind == "q8":
            a = hq8.dequantize_rows(a, shape[1]).T
        w[name] = torch.from_numpy(np.ascontiguousarray(a, np.float32))
    return w


@pytest.fixture(autouse=True)
def _profile():
    dr.apply_production_profile()
    yield
    dr.apply_production_profile()
    dr._KV_ELEM_BYTES = 4


@pytest.mark.parametrize("cfg_name,elem_bytes,split", [("tiny", 4, False), ("small-qwen-arch", 4, False),
                                                      ("small-qwen-arch", 2, True)])
def test_graph_runner_reference_call_order(gpu, oracle, cfg_name, elem_bytes, split):
    cfg = M.CONFIGS[cfg_name]
    case(f"reference GraphRunner order {cfg_name} elem_bytes={elem_bytes} split={split}")
    qw = M.synth_weights(cfg, seed=77)
    w = reference_w(cfg, qw)
    c = cfg.as_cfg()
    dr._KV_ELEM_BYTES = elem_bytes
    dr._ATTN_SPLIT_K = split
    seed = M.random_prompt(cfg, 3, seed=4)
    kv = [None] * c["n_layers"]
    gr = dr.GraphRunner(w, c, kv)
    lg = gr.seed(torch.tensor(seed), torch.arange(3))
    assert isinstance(lg, torch.Tensor) and tuple(lg.shape) == (1, 1, cfg.vocab)
    t = int(lg[0, -1].argmax())
    out = [t]
    gr.capture(torch.tensor([t]), torch.tensor([3]))
    cur = t
    for _ in range(20):
        cur = gr.replay_token(torch.tensor([cur]))
        out.append(int(cur))
    orc = oracle.OracleModel(cfg, qw, kv_f16=elem_bytes == 2, attn_nsplit=16 if split else 1)
    exp, _ = orc.generate(seed, 21)
    assert out == exp
    # the caches live in the caller's list, with the reference's DeviceKVCache interface
    assert all(k is not None and k.length == 3 + 20 for k in kv)
    ks = kv[0].k_slice_host()
    assert ks.shape == (23, cfg.n_head_kv, cfg.head_dim) and ks.dtype == np.float32
    ref_k = orc.kv_rows(0, "k", 23)
    ref_k = ref_k.view(np.float16).astype(np.float32) if elem_bytes == 2 else ref_k
    assert np.array_equal(ks.reshape(23, -1), ref_k)
    # replay_logits of one more token equals the oracle's step
    exp_lg = orc.step(out[-1])
    got = gr.replay_logits(torch.tensor([out[-1]]))
    assert np.array_equal(bits(got.numpy().reshape(-1)), bits(exp_lg))
    gr.free()


def test_forward_pass_resident_matches_oracle(gpu, oracle):
    cfg = M.TINY
    case("forward_pass_resident")
    qw = M.synth_weights(cfg, seed=78)
    w = reference_w(cfg, qw)
    c = cfg.as_cfg()
    toks = M.random_prompt(cfg, 7, seed=9)
    kv = [None] * cfg.n_layers
    orc = oracle.OracleModel(cfg, qw)
    lg = dr.forward_pass_resident(w, c, torch.tensor(toks[:5]), torch.arange(5), kv)   # batched
    for t in toks[:5]:
        e = orc.step(t)
    assert np.array_equal(bits(lg.numpy().reshape(-1)), bits(e))
    for i in (5, 6):                                                                   # one at a time
        lg = dr.forward_pass_resident(w, c, torch.tensor([toks[i]]), torch.tensor([i]), kv)
        assert np.array_equal(bits(lg.numpy().reshape(-1)), bits(orc.step(toks[i])))
    with pytest.raises(ValueError):   # a position that does not continue the cache
        dr.forward_pass_resident(w, c, torch.tensor([1]), torch.tensor([3]), kv)
    kv[0]._plan.free()


def test_host_embedding_rows(gpu, oracle):
    """A token_embd that does not round-trip through Q8_0 (an fp32 row of an unused token
    perturbed) makes the step take its input row from the host, as the reference does; the
    used rows are unchanged, so the tokens still equal the oracle's."""
    cfg = M.TINY
    case("host embedding rows")
    qw = M.synth_weights(cfg, seed=79)
    w = reference_w(cfg, qw)
    emb = w["token_embd.weight"].numpy().copy()
    prompt = [5, 9, 11]
    emb[0, cfg.vocab - 1] += np.float32(1e-7)   # token vocab-1's row, never fed below
    w["token_embd.weight"] = torch.from_numpy(emb)
    kv = [None] * cfg.n_layers
    gr = dr.GraphRunner(w, cfg.as_cfg(), kv)
    lg = gr.seed(torch.tensor(prompt), torch.arange(3))
    assert kv[0]._plan.host_embed
    orc = oracle.OracleModel(cfg, qw)
    exp, _ = orc.generate(prompt, 8)
    out = [int(lg[0, -1].argmax())]
    gr.capture(torch.tensor([out[0]]), torch.tensor([3]))
    for _ in range(7):
        out.append(gr.replay_token(torch.tensor([out[-1]])))
    assert out == exp
    gr.free()
    kv[0]._plan.free()


def test_op_functions_match_oracle(gpu, oracle):
    """rms_norm_dev, q8_linear_dev (+ rms_src), q8_linear_add_residual_dev (+ silu_src),
    q8_linear_dev_bias, silu_mul_dev, add_dev, rope_dev_qk_fused, DeviceKVCache appends,
    attn_decode_from_cache_masked and argmax_dev on the reference's argument kinds."""
    case("op functions")
    rng = np.random.default_rng(5)
    K, N = 896, 1152
    x = rng.standard_normal(K).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    Wq = hq8.quantize_rows((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    W = torch.from_numpy(hq8.dequantize_rows(Wq, K).T.copy())        # [K, N] fp32
    xd = dr.DevTensor.from_host(x)
    h = dr.rms_norm_dev(xd, nw, 1e-6)
    assert np.array_equal(bits(h.to_host()), bits(oracle.rmsnorm(x, nw, 1e-6)))
    xq_, xd_ = oracle.quant_q8(oracle.rmsnorm(x, nw, 1e-6))
    exp = oracle.q8_gemv(Wq, xq_, xd_, K)
    assert np.array_equal(bits(dr.q8_linear_dev(h, W).to_host()), bits(exp))
    y = dr.q8_linear_dev(None, W, rms_src=(xd, dr._dev_const(nw), 1e-6))
    assert np.array_equal(bits(y.to_host()), bits(exp))
    b = (rng.standard_normal(N) * 0.02).astype(np.float32)
    yb = dr.q8_linear_dev_bias(h, W, torch.from_numpy(b))
    assert np.array_equal(bits(yb.to_host()), bits(oracle.q8_gemv(Wq, xq_, xd_, K, b)))
    # SiLU(g)*u: elementwise, and quantized into the down GEMV with the residual
    F = 4864
    g = (2 * rng.standard_normal(F)).astype(np.float32)
    u = rng.standard_normal(F).astype(np.float32)
    gd, ud = dr.DevTensor.from_host(g), dr.DevTensor.from_host(u)
    assert np.array_equal(bits(dr.silu_mul_dev(gd, ud).to_host()), bits(oracle.silu_mul(g, u)))
    assert np.array_equal(bits(dr.add_dev(gd, ud).to_host()), bits(g + u))
    Wdq = hq8.quantize_rows((rng.standard_normal((K, F)) * 0.02).astype(np.float32))
    Wd = torch.from_numpy(hq8.dequantize_rows(Wdq, F).T.copy())
    r = rng.standard_normal(K).astype(np.float32)
    out = dr.DevTensor.empty((K,))
    dr.q8_linear_add_residual_dev(None, Wd, dr.DevTensor.from_host(r), out=out, silu_src=(gd, ud))
    sq, sd = oracle.silu_mul_quant(g, u)
    assert np.array_equal(bits(out.to_host()), bits(oracle.q8_gemv(Wdq, sq, sd, F, r)))
    # RoPE of q|k at a device position, append, masked attention, argmax
    nh, nkv, hd = 14, 2, 64
    qk = rng.standard_normal((nh + nkv) * hd).astype(np.float32)
    for elem_bytes in (4, 2):
        cache = dr.DeviceKVCache(64, nkv, hd, elem_bytes)
        kvrows = []
        for pos in range(5):
            qkd = dr.DevTensor.from_host(qk + pos)
            lp = cache._ensure_len_ptr(seed=True)
            dr.rope_dev_qk_fused(qkd.ptr, lp, nh, nkv, hd, 1e6)
            kd = dr._slice_dev(qkd, nh * hd, nkv * hd)
            vd = dr.DevTensor.from_host(rng.standard_normal(nkv * hd).astype(np.float32))
            if pos % 2:
                assert cache.append_at_len_incr(kd.ptr, vd.ptr) is True
            else:
                cache.append_at_len(kd.ptr, vd.ptr)
                cache.incr_len_dev()
            cache.length += 1
            kvrows.append((oracle.rope(qk + pos, pos, nh + nkv, hd, 1e6), vd.to_host()))
            q_roped = kvrows[-1][0]
            assert np.array_equal(bits(qkd.to_host()[:nh * hd]), bits(q_roped[:nh * hd]))
        assert cache.device_length() == 5
        f16 = elem_bytes == 2
        conv = (lambda a: a.astype(np.float16).view(np.uint16)) if f16 else (lambda a: a)
        kc = np.stack([conv(kr[0][nh * hd:]) for kr in kvrows])
        vc = np.stack([conv(kr[1]) for kr in kvrows])
        qd = dr.DevTensor.from_host(kvrows[-1][0])
        att = dr.attn_decode_from_cache_masked(qd.ptr, cache, nh, hd ** -0.5, cache._ensure_len_ptr(False), 64)
        exp = oracle.attn_decode(kvrows[-1][0], kc, vc, 5, nh, nkv, hd, float(hd ** -0.5), f16)
        assert np.array_equal(bits(att.to_host()), bits(exp))
        assert np.array_equal(cache.k_slice_host().reshape(5, -1),
                              kc.view(np.float16).astype(np.float32) if f16 else kc)
        cache.free()
    lg = rng.standard_normal(5000).astype(np.float32)
    lg[[17, 4000]] = 9.0
    p = dr.argmax_dev(dr.DevTensor.from_host(lg).ptr, 5000)
    got = np.zeros(1, np.int32)
    gpu.sync()
    gpu.d2h(got, p.value)
    assert int(got[0]) == 17


def test_composition_gate_refuses(gpu):
    dr._KV_QUANT_Q8 = True
    with pytest.raises(RuntimeError):
        dr.assert_certified_composition()
    dr.apply_production_profile()
    dr._QFUSED = True
    with pytest.raises(RuntimeError):
        dr.assert_certified_composition()
    dr.apply_production_profile()
    dr.assert_certified_composition()
    assert dr.attest_profile()["_FUSE_QKV"] is True


def test_llamatov_run_generate(gpu, oracle, tmp_path):
    """generate(path, ids, n) from a Q8_0 GGUF file, and with preloaded=(cfg, w) from
    load_model(): (prompt + tokens, tok/s), tokens equal to the oracle's."""
    from llamatov_amd import gguf
    from llamatov_amd import llamatov_run as R
    cfg = M.TINY
    case("llamatov_run.generate")
    qw = M.synth_weights(cfg, seed=80)
    path = tmp_path / "tiny.gguf"
    gguf.save_q8_model(path, cfg, qw)
    ids = [3, 1, 4, 1, 5]
    exp, _ = oracle.OracleModel(cfg, qw).generate(ids, 6)
    gen, tps = R.generate(str(path), ids, 6)
    assert gen == ids + exp and tps > 0
    c, w = R.load_model(str(path))
    gen2, _ = R.generate(str(path), ids, 6, device="cuda", preloaded=(c, w))
    assert gen2 == ids + exp

"""BASELINE config 5 on the GPU: the random-init Llama-3-8B-architecture Q8_0 model (32 layers,
hidden 4096, FFN 14336, 32 Q / 8 KV heads, head_dim 128, vocab 128256, untied head), fp16 KV.

* The 512-token batched prefill (int8-MFMA GEMMs on the tiled layouts, the grouped walks at
  K = 4096 / 14336, the row-merged causal attention with 16 splits, the fused RoPE + append)
  leaves the same KV caches, last-token logits and greedy token, bit for bit, as the
  single-token device path fed the 512 tokens one at a time -- the reference's
  device-uniformity requirement for a batched prefill (bpd/lib/dev_residency.py:1344-1350).
* 256 greedy decode tokens by graph replay equal 256 eager steps (the reference's GR gate).
* The full 32-layer model matches the CPU oracle in the logits, bit for bit, over a short
  prompt and 4 greedy graph replays; a truncated model (2 layers at the full widths, the
  untied 128256 x 4096 head) does so over a longer continuation.
"""
import numpy as np
import pytest

from llamatov_amd import engine as dr
from llamatov_amd import model as M
from llamatov_amd._lib import LT_KV_F16

pytestmark = pytest.mark.gpu

C5_NSPLIT = 16
N_PREFILL, N_DECODE = 512, 256


def case(msg):
    print(f"[gpu-case] {msg}", flush=True)


def bits(a):
    return np.asarray(a).view(np.uint32)


@pytest.fixture(scope="module")
def c5_weights():
    case("C5 weights")
    return M.synth_weights(M.LLAMA3_8B, seed=4321)


@pytest.fixture(scope="module")
def c5_model(gpu, c5_weights):
    m = dr.ResidentModel(M.LLAMA3_8B, c5_weights, gpu, layouts="fused")
    yield m
    m.free()


def _kv(plan, n, layers):
    return {(il, which): plan.caches[il].rows_host(which, n).copy() for il in layers for which in "kv"}


def test_c5_prefill_512_equals_stepwise(gpu, c5_model):
    cfg = M.LLAMA3_8B
    prof = dr.Profile(kv_dtype=LT_KV_F16, attn_nsplit=C5_NSPLIT)
    prompt = M.random_prompt(cfg, N_PREFILL, seed=17)
    plan = dr.DecodePlan(c5_model, prof, max_ctx=N_PREFILL + N_DECODE + 8, hist_cap=N_PREFILL + N_DECODE + 8)
    layers = range(cfg.n_layers)
    case("C5 batched prefill 512")
    dr.forward_prefill(plan, prompt)
    lb, tb = plan.read_logits().copy(), plan.read_token()
    kvb = _kv(plan, N_PREFILL, layers)
    assert list(plan.lengths()) == [N_PREFILL] * cfg.n_layers
    case("C5 token-by-token 512")
    plan.reset()
    la = dr.forward_tokens(plan, prompt)
    assert np.array_equal(bits(la), bits(lb))
    assert plan.read_token() == tb == int(np.argmax(la))
    for key, rows in _kv(plan, N_PREFILL, layers).items():
        assert np.array_equal(rows, kvb[key]), key
    plan.free()


def test_c5_graph_replay_equals_eager_256(gpu, c5_model):
    cfg = M.LLAMA3_8B
    prof = dr.Profile(kv_dtype=LT_KV_F16, attn_nsplit=C5_NSPLIT)
    prompt = M.random_prompt(cfg, N_PREFILL, seed=17)
    plan = dr.DecodePlan(c5_model, prof, max_ctx=N_PREFILL + N_DECODE + 8, hist_cap=N_PREFILL + N_DECODE + 8)
    case("C5 prefill + 256 graph replays")
    dr.forward_prefill(plan, prompt)
    first = plan.read_token()
    gr = dr.StepGraph(plan)
    gr.capture()
    seq_g = [first] + gr.replay_tokens(N_DECODE - 1)
    lg = plan.read_logits().copy()
    kv_g = _kv(plan, N_PREFILL + N_DECODE - 1, (0, 15, 31))
    case("C5 prefill + 256 eager steps")
    plan.reset()
    dr.forward_prefill(plan, prompt)
    seq_e = [plan.read_token()]
    for _ in range(N_DECODE - 1):
        plan.step()
        seq_e.append(plan.read_token())
    assert seq_g == seq_e
    assert np.array_equal(bits(plan.read_logits()), bits(lg))
    for key, rows in _kv(plan, N_PREFILL + N_DECODE - 1, (0, 15, 31)).items():
        assert np.array_equal(rows, kv_g[key]), key
    gr.free()
    plan.free()


def test_c5_full_depth_matches_oracle(gpu, oracle, c5_model, c5_weights):
    """All 32 layers against the oracle: the last prompt position's logits after the batched
    prefill and the logits of 4 greedy graph replays, bit for bit, and the greedy tokens."""
    cfg = M.LLAMA3_8B
    case("C5 32-layer oracle")
    orc = oracle.OracleModel(cfg, c5_weights, kv_f16=True, attn_nsplit=C5_NSPLIT, max_ctx=64)
    prompt = M.random_prompt(cfg, 6, seed=23)
    for t in prompt:
        exp = orc.step(t)
    plan = dr.DecodePlan(c5_model, dr.Profile(kv_dtype=LT_KV_F16, attn_nsplit=C5_NSPLIT), max_ctx=64)
    case("C5 32-layer prefill + 4 replays")
    dr.forward_prefill(plan, prompt)
    assert np.array_equal(bits(plan.read_logits()), bits(exp))
    got, want = [plan.read_token()], [oracle.argmax(exp)]
    gr = dr.StepGraph(plan)
    gr.capture()
    for i in range(4):
        exp = orc.step(want[-1])
        lg = gr.replay_logits(got[-1])
        assert np.array_equal(bits(lg), bits(exp)), f"replay {i}: max |d| {np.abs(lg - exp).max()}"
        got.append(plan.read_token())
        want.append(oracle.argmax(exp))
    assert got == want
    for il in (0, 31):
        for which in "kv":
            assert np.array_equal(plan.caches[il].rows_host(which, len(prompt) + 4),
                                  orc.kv_rows(il, which, len(prompt) + 4)), (il, which)
    gr.free()
    plan.free()


def test_c5_truncated_matches_oracle(gpu, oracle):
    """Two layers at the full 8B widths with the untied 128256 x 4096 head: logits bit for
    bit against the oracle over a short prompt and greedy continuation, through the batched
    prefill and the graph."""
    cfg = M.LLAMA3_8B.replace(name="llama-3-8b-arch-2l", n_layers=2, max_ctx=64)
    case("C5 truncated 2-layer weights")
    w = M.synth_weights(cfg, seed=99)
    orc = oracle.OracleModel(cfg, w, kv_f16=True, attn_nsplit=C5_NSPLIT)
    prompt = M.random_prompt(cfg, 9, seed=5)
    exp_tokens, _ = orc.generate(prompt, 5)
    m = dr.ResidentModel(cfg, w, gpu, layouts="fused")
    plan = dr.DecodePlan(m, dr.Profile(kv_dtype=LT_KV_F16, attn_nsplit=C5_NSPLIT))
    case("C5 truncated prefill + steps")
    dr.forward_prefill(plan, prompt)
    got = [plan.read_token()]
    orc2 = oracle.OracleModel(cfg, w, kv_f16=True, attn_nsplit=C5_NSPLIT)
    for t in prompt:
        exp_logits = orc2.step(t)
    assert np.array_equal(bits(plan.read_logits()), bits(exp_logits))
    gr = dr.StepGraph(plan)
    gr.capture()
    for _ in range(4):
        t = got[-1]
        exp_logits = orc2.step(t)
        lg = gr.replay_logits(t)
        assert np.array_equal(bits(lg), bits(exp_logits))
        got.append(plan.read_token())
    assert got == exp_tokens
    for il in range(cfg.n_layers):
        for which in "kv":
            assert np.array_equal(plan.caches[il].rows_host(which, len(prompt) + 4),
                                  orc2.kv_rows(il, which, len(prompt) + 4)), (il, which)
    gr.free()
    plan.free()
    m.free()

"""Decode-level parity: the device decode step against the oracle's step, graph replay
against eager (the reference's GR gate, gr_referee.py), prefill KV against incremental KV
(A1, decode_referee.py), and greedy token identity (long_run_referee.py) at the
BASELINE configuration 2 geometry."""
import numpy as np
import pytest

from llamatov_amd import engine as dr
from llamatov_amd import model as M
from llamatov_amd._lib import LT_KV_F16, LT_KV_F32

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[gpu-case] {msg}", flush=True)


_WEIGHTS = {}


def weights(cfg, seed=1234):
    key = (cfg.name, seed)
    if key not in _WEIGHTS:
        _WEIGHTS[key] = M.synth_weights(cfg, seed)
    return _WEIGHTS[key]


_RESIDENT = {}


def resident(cfg, gpu):
    if cfg.name not in _RESIDENT:
        _RESIDENT[cfg.name] = dr.ResidentModel(cfg, weights(cfg), gpu)
    return _RESIDENT[cfg.name]


def bitexact(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


@pytest.mark.parametrize("step", ["fused", "fused_swiglu_fp32", "per_op"])
@pytest.mark.parametrize("kv_dtype,nsplit,fused", [(LT_KV_F32, 1, False), (LT_KV_F16, 1, True),
                                                   (LT_KV_F32, 4, True), (LT_KV_F16, 2, False),
                                                   (LT_KV_F16, 16, False)])
def test_tiny_stepwise_logits_bitexact(gpu, oracle, step, kv_dtype, nsplit, fused):
    cfg = M.TINY
    case(f"tiny stepwise {step} kv={kv_dtype} nsplit={nsplit} fused_rms={fused}")
    prof = dr.Profile(kv_dtype=kv_dtype, attn_nsplit=nsplit, fused_rms_quant=fused,
                      fused_step=step != "per_op", swiglu_fp32=step == "fused_swiglu_fp32")
    plan = dr.DecodePlan(resident(cfg, gpu), prof)
    orc = oracle.OracleModel(cfg, weights(cfg), kv_f16=kv_dtype == LT_KV_F16, attn_nsplit=nsplit)
    toks = M.random_prompt(cfg, 6, seed=3)
    for i in range(30):
        t = toks[i] if i < len(toks) else int(np.argmax(exp))
        plan.step(t)
        got = plan.read_logits()
        exp = orc.step(t)
        assert bitexact(got, exp), f"step {i}: max |d| = {np.abs(got - exp).max()}"
        assert plan.read_token() == oracle.argmax(exp)
    assert list(plan.lengths()) == [30] * cfg.n_layers
    for il in range(cfg.n_layers):
        for which in "kv":
            assert np.array_equal(plan.caches[il].rows_host(which, 30), orc.kv_rows(il, which, 30))
    plan.free()


@pytest.mark.parametrize("kv_dtype", [LT_KV_F32, LT_KV_F16])
@pytest.mark.parametrize("four", [True, False])
def test_small_qwen_four_launch_step_bitexact(gpu, oracle, kv_dtype, four):
    """The four-launch step (attention inside the O GEMV, RoPE + KV append in the QKV GEMV)
    and the five-launch step against the oracle's step, logits and KV rows, over 40 steps
    (head dim 64: the fused attention applies)."""
    cfg = M.SMALL_QWEN
    case(f"small-qwen stepwise four={four} kv={kv_dtype}")
    plan = dr.DecodePlan(resident(cfg, gpu), dr.Profile(kv_dtype=kv_dtype, attn_in_o=four, persistent_step=False))
    assert plan.four_launch == four
    orc = oracle.OracleModel(cfg, weights(cfg), kv_f16=kv_dtype == LT_KV_F16)
    toks = M.random_prompt(cfg, 5, seed=13)
    for i in range(40):
        t = toks[i] if i < len(toks) else int(np.argmax(exp))
        plan.step(t)
        exp = orc.step(t)
        assert bitexact(plan.read_logits(), exp), f"step {i}"
    assert list(plan.lengths()) == [40] * cfg.n_layers
    for il in range(cfg.n_layers):
        for which in "kv":
            assert np.array_equal(plan.caches[il].rows_host(which, 40), orc.kv_rows(il, which, 40))
    # graph replays of the same step continue the oracle's greedy chain, bit for bit (the
    # four-launch graph while the cache is short enough, the five-launch one after)
    gr = dr.StepGraph(plan)
    gr.capture()
    seq = gr.replay_tokens(6)
    ref = []
    t = int(np.argmax(exp))
    for _ in range(6):
        exp = orc.step(t)
        t = int(np.argmax(exp))
        ref.append(t)
    assert seq == ref
    assert bitexact(plan.read_logits(), exp)
    gr.free()
    plan.free()


@pytest.mark.parametrize("nsplit", [1, 8])
def test_graph_replay_equals_eager(gpu, nsplit):
    """GR gate: graph replay is bit-identical to the eager step, device length advances,
    and the token chain from replay_tokens equals replay_token one by one (also with the
    split-K attention and its merge launch in the graph)."""
    cfg = M.TINY
    case(f"tiny graph vs eager nsplit={nsplit}")
    m = resident(cfg, gpu)
    prompt = M.random_prompt(cfg, 5, seed=8)
    prof = dr.Profile(kv_dtype=LT_KV_F16, attn_nsplit=nsplit)
    eager = dr.DecodePlan(m, prof)
    graph = dr.DecodePlan(m, prof)
    dr.forward_tokens(eager, prompt)
    gr = dr.StepGraph(graph)
    gr.seed(prompt)
    gr.capture()
    for i in range(12):
        t = eager.read_token()
        eager.step(t)
        lg = gr.replay_logits(t)
        assert bitexact(lg, eager.read_logits()), f"replay {i}"
        assert list(graph.lengths()) == list(eager.lengths())
    for il in range(cfg.n_layers):
        n = int(eager.lengths()[il])
        assert np.array_equal(graph.caches[il].rows_host("k", n), eager.caches[il].rows_host("k", n))
    # back-to-back replays with the device-side token chain
    seq1 = [gr.replay_token() for _ in range(8)]
    ref = [eager.read_token()]
    for _ in range(8):
        eager.step(ref[-1])
        ref.append(eager.read_token())
    assert seq1 == ref[1:]
    seq2 = gr.replay_tokens(8)
    for t in seq2:
        eager.step(eager.read_token())
    assert seq2[-1] == eager.read_token()
    gr.free()
    eager.free()
    graph.free()


def test_prefill_kv_equals_incremental(gpu):
    """A1: a fresh prefill over gen[:t] reproduces the incremental KV cache bit for bit."""
    cfg = M.TINY
    case("tiny A1")
    m = resident(cfg, gpu)
    prompt = M.random_prompt(cfg, 4, seed=9)
    inc = dr.DecodePlan(m)
    dr.forward_tokens(inc, prompt)
    seq = list(prompt)
    for _ in range(10):
        seq.append(inc.read_token())
        inc.step(seq[-1])
    fresh = dr.DecodePlan(m)
    lg = dr.forward_tokens(fresh, seq)
    assert bitexact(lg, inc.read_logits())
    for il in range(cfg.n_layers):
        assert np.array_equal(fresh.caches[il].rows_host("k", len(seq)), inc.caches[il].rows_host("k", len(seq)))
        assert np.array_equal(fresh.caches[il].rows_host("v", len(seq)), inc.caches[il].rows_host("v", len(seq)))
    inc.free()
    fresh.free()


@pytest.mark.parametrize("cfg_name,n_prompt,n_gen,kv_dtype,step", [
    ("small-qwen-arch", 32, 32, LT_KV_F32, "fused"),
    ("small-qwen-arch", 32, 32, LT_KV_F32, "per_op"),
    ("small-qwen-arch", 32, 32, LT_KV_F16, "persistent"),
    ("qwen2.5-0.5b-arch", 32, 128, LT_KV_F32, "fused"),
    ("qwen2.5-0.5b-arch", 32, 128, LT_KV_F16, "fused"),
    ("qwen2.5-0.5b-arch", 32, 128, LT_KV_F32, "persistent"),
    ("qwen2.5-0.5b-arch", 32, 128, LT_KV_F16, "persistent"),
    ("qwen2.5-0.5b-arch", 32, 128, LT_KV_F16, "per_op"),
    ("qwen2.5-0.5b-arch", 32, 128, LT_KV_F16, "fused_swiglu_fp32"),
])
def test_greedy_tokens_identical(gpu, oracle, cfg_name, n_prompt, n_gen, kv_dtype, step):
    """Greedy token identity with the oracle, through the captured graph ("fused": the
    five-launch step; "persistent": the one-launch step)."""
    cfg = M.CONFIGS[cfg_name]
    case(f"greedy {cfg_name} {n_prompt}+{n_gen} kv={kv_dtype} {step}")
    prompt = M.random_prompt(cfg, n_prompt, seed=7)
    orc = oracle.OracleModel(cfg, weights(cfg), kv_f16=kv_dtype == LT_KV_F16)
    exp, margins = orc.generate(prompt, n_gen)
    plan = dr.DecodePlan(resident(cfg, gpu), dr.Profile(kv_dtype=kv_dtype, fused_step=step != "per_op",
                                                        swiglu_fp32=step == "fused_swiglu_fp32",
                                                        persistent_step=step == "persistent"))
    assert (plan.persistent_len > 0) == (step == "persistent")
    gr = dr.StepGraph(plan)
    gr.seed(prompt)
    first = plan.read_token()
    gr.capture()
    got = [first] + gr.replay_tokens(n_gen - 1)
    print(f"[margins] min top1-top2 margin {float(margins.min()):.3e}", flush=True)
    assert plan.error() == 0
    assert got == exp
    gr.free()
    plan.free()


def test_step_switches_from_four_to_five_launches(gpu, oracle):
    """A decode that crosses the four-launch step's length limit: the graph replays switch to
    the five-launch graph there, and every token's logits equal the oracle's."""
    cfg = M.SMALL_QWEN.replace(max_ctx=512)
    case("four -> five launch switch")
    w = weights(M.SMALL_QWEN)
    plan = dr.DecodePlan(dr.ResidentModel(cfg, w, gpu, layouts="fused"),
                         dr.Profile(kv_dtype=LT_KV_F16, attn_in_o=True, persistent_step=False))
    lim = plan.four_launch_len
    assert 0 < lim < 400
    orc = oracle.OracleModel(cfg, w, kv_f16=True)
    prompt = M.random_prompt(cfg, lim - 5, seed=3)
    dr.forward_prefill(plan, prompt)
    for t in prompt:
        exp = orc.step(t)
    gr = dr.StepGraph(plan)
    gr.capture()
    for i in range(12):     # lengths lim-5 .. lim+6: both graphs
        t = int(np.argmax(exp))
        lg = gr.replay_logits(t)
        exp = orc.step(t)
        assert bitexact(lg, exp), f"replay {i} at length {plan.caches[0].length}"
    gr.free()
    plan.free()

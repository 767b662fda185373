"""The persistent step (lt_decode_step: every layer in one launch, phases exchanged through
step-tagged words) against the oracle and against the five-launch step: logits bit for bit
at every step, KV rows, lengths, graph replays, the switch to five launches past the step's
length limit, host embedding rows and the error word."""
import numpy as np
import pytest

from llamatov_amd import engine as dr
from llamatov_amd import model as M
from llamatov_amd._lib import LT_KV_F16, LT_KV_F32

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[gpu-case] {msg}", flush=True)


_WEIGHTS = {}
_RESIDENT = {}


def weights(cfg, seed=1234):
    key = (cfg.name, seed)
    if key not in _WEIGHTS:
        _WEIGHTS[key] = M.synth_weights(cfg, seed)
    return _WEIGHTS[key]


def resident(cfg, gpu):
    if cfg.name not in _RESIDENT:
        _RESIDENT[cfg.name] = dr.ResidentModel(cfg, weights(cfg), gpu)
    return _RESIDENT[cfg.name]


def bitexact(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


@pytest.mark.parametrize("kv_dtype", [LT_KV_F32, LT_KV_F16])
def test_persistent_step_logits_bitexact(gpu, oracle, kv_dtype):
    """40 eager steps of SMALL_QWEN through the persistent step: every step's logits, the
    greedy token, the KV rows and the lengths equal the oracle's; no device error."""
    cfg = M.SMALL_QWEN
    case(f"persistent small-qwen stepwise kv={kv_dtype}")
    plan = dr.DecodePlan(resident(cfg, gpu), dr.Profile(kv_dtype=kv_dtype))
    assert plan.persistent_len > 0 and plan.persistent
    orc = oracle.OracleModel(cfg, weights(cfg), kv_f16=kv_dtype == LT_KV_F16)
    toks = M.random_prompt(cfg, 5, seed=21)
    for i in range(40):
        t = toks[i] if i < len(toks) else int(np.argmax(exp))
        plan.step(t)
        got = plan.read_logits()
        exp = orc.step(t)
        assert plan.error() == 0, f"step {i}: device error {plan.error()}"
        assert bitexact(got, exp), f"step {i}: max |d| = {np.abs(got - exp).max()}"
        assert plan.read_token() == oracle.argmax(exp)
    assert list(plan.lengths()) == [40] * cfg.n_layers
    for il in range(cfg.n_layers):
        for which in "kv":
            assert np.array_equal(plan.caches[il].rows_host(which, 40), orc.kv_rows(il, which, 40))
    plan.free()


@pytest.mark.parametrize("kv_dtype", [LT_KV_F32, LT_KV_F16])
def test_persistent_graph_equals_five_launch_graph(gpu, kv_dtype):
    """At the C2 geometry (24 layers): the persistent step's graph and the five-launch graph,
    replayed from the same prefilled cache, give the same logits at every replay and the same
    caches and lengths."""
    cfg = M.QWEN25_05B
    case(f"persistent vs five-launch graphs, C2 kv={kv_dtype}")
    m = resident(cfg, gpu)
    prompt = M.random_prompt(cfg, 20, seed=4)
    p5 = dr.DecodePlan(m, dr.Profile(kv_dtype=kv_dtype, persistent_step=False))
    pp = dr.DecodePlan(m, dr.Profile(kv_dtype=kv_dtype))
    assert pp.persistent and not p5.persistent
    g5, gp = dr.StepGraph(p5), dr.StepGraph(pp)
    g5.seed(prompt, batched=True)
    gp.seed(prompt, batched=True)
    g5.capture()
    gp.capture()
    assert gp.graphp.value and not g5.graphp.value
    t = p5.read_token()
    for i in range(24):
        a = g5.replay_logits(t)
        b = gp.replay_logits(t)
        assert pp.error() == 0
        assert bitexact(a, b), f"replay {i}"
        t = int(np.argmax(a))
    assert list(pp.lengths()) == list(p5.lengths()) == [44] * cfg.n_layers
    for il in (0, 11, 23):
        for which in "kv":
            assert np.array_equal(pp.caches[il].rows_host(which, 44), p5.caches[il].rows_host(which, 44))
    # the device token chain
    assert gp.replay_tokens(10) == g5.replay_tokens(10)
    g5.free()
    gp.free()
    p5.free()
    pp.free()


def test_persistent_switches_to_five_launches(gpu, oracle):
    """fp32 caches stage at most 256 rows in the persistent step: a decode that crosses that
    length switches graphs there, and every replay's logits equal the oracle's."""
    cfg = M.SMALL_QWEN.replace(max_ctx=512)
    case("persistent -> five-launch switch")
    w = weights(M.SMALL_QWEN)
    plan = dr.DecodePlan(dr.ResidentModel(cfg, w, gpu, layouts="fused"), dr.Profile(kv_dtype=LT_KV_F32))
    lim = plan.persistent_len
    assert 0 < lim < 512
    orc = oracle.OracleModel(cfg, w)
    prompt = M.random_prompt(cfg, lim - 6, seed=3)
    dr.forward_prefill(plan, prompt)
    for t in prompt:
        exp = orc.step(t)
    gr = dr.StepGraph(plan)
    gr.capture()
    seen = set()
    for i in range(12):     # lengths lim-6 .. lim+5: both graphs
        seen.add(plan.persistent)
        t = int(np.argmax(exp))
        lg = gr.replay_logits(t)
        exp = orc.step(t)
        assert plan.error() == 0
        assert bitexact(lg, exp), f"replay {i} at length {plan.caches[0].length}"
    assert seen == {True, False}
    gr.free()
    plan.free()


def test_persistent_host_embedding_rows(gpu, oracle):
    """A host_embed plan: layer 0 takes the host row instead of gathering token_embd."""
    cfg = M.SMALL_QWEN
    case("persistent host embedding rows")
    w = weights(cfg)
    plan = dr.DecodePlan(resident(cfg, gpu), dr.Profile(kv_dtype=LT_KV_F16), host_embed=True)
    assert plan.persistent
    orc = oracle.OracleModel(cfg, w, kv_f16=True)
    toks = M.random_prompt(cfg, 12, seed=31)
    for i, t in enumerate(toks):
        plan.step(embedding=oracle.embed_row(w["token_embd.weight"], t, cfg.n_embd))
        assert bitexact(plan.read_logits(), orc.step(t)), f"step {i}"
    assert plan.error() == 0
    plan.free()


def test_persistent_bad_token(gpu):
    """A token outside the vocabulary: the error word says so and the step runs on a zero row,
    as the five-launch step does (same logits)."""
    cfg = M.SMALL_QWEN
    case("persistent bad token")
    m = resident(cfg, gpu)
    a = dr.DecodePlan(m, dr.Profile(kv_dtype=LT_KV_F16, persistent_step=False))
    b = dr.DecodePlan(m, dr.Profile(kv_dtype=LT_KV_F16))
    for t in (3, cfg.vocab + 7, 5):
        a.step(t)
        b.step(t)
        assert bitexact(a.read_logits(), b.read_logits())
    assert a.error() == 1 and b.error() == 1
    a.free()
    b.free()


def test_persistent_many_steps_and_reset(gpu, oracle):
    """Step tags keep advancing over many steps and across reset(): 200 graph replays, a
    reset, then a fresh generation, each equal to the oracle's tokens."""
    cfg = M.SMALL_QWEN
    case("persistent 200 replays + reset")
    w = weights(cfg)
    plan = dr.DecodePlan(resident(cfg, gpu), dr.Profile(kv_dtype=LT_KV_F16))
    for seed in (5, 6):
        prompt = M.random_prompt(cfg, 8, seed=seed)
        orc = oracle.OracleModel(cfg, w, kv_f16=True)
        exp, _ = orc.generate(prompt, 200 if seed == 5 else 20)
        plan.reset()
        gr = dr.StepGraph(plan)
        gr.seed(prompt)
        first = plan.read_token()
        gr.capture()
        got = [first] + gr.replay_tokens(len(exp) - 1)
        assert plan.error() == 0
        assert got == exp
        gr.free()
    plan.free()

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


@pytest.mark.parametrize("kv_dtype,nsplit", [(LT_KV_F32, 1), (LT_KV_F16, 1), (LT_KV_F16, 4)])
def test_batch_rows_equal_lone_sequences(gpu, oracle, kv_dtype, nsplit):
    cfg = M.SMALL_QWEN
    case(f"batch vs lone sequences kv={kv_dtype} nsplit={nsplit}")
    w = weights(cfg)
    model = dr.ResidentModel(cfg, w, gpu)
    lens = [3, 9, 1, 14]
    prompts = [M.random_prompt(cfg, n, seed=40 + i) for i, n in enumerate(lens)]
    plan = dr.BatchDecodePlan(model, len(prompts), dr.Profile(kv_dtype=kv_dtype, attn_nsplit=nsplit), max_ctx=64)
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


def test_batch_generate_c2_geometry(gpu):
    """batch_generate at the C2 model (Qwen2.5-0.5B geometry, 8 sequences of 32-token
    prompts) equals generate per sequence."""
    cfg = M.QWEN25_05B
    case("batch_generate C2 x8")
    w = weights(cfg)
    model = dr.ResidentModel(cfg, w, gpu)
    prompts = [M.random_prompt(cfg, 32 - 3 * b, seed=70 + b) for b in range(8)]
    prof = dr.Profile(kv_dtype=LT_KV_F16)
    got = dr.batch_generate(model, prompts, 24, prof)
    for b, pr in enumerate(prompts):
        assert got[b] == dr.generate(model, pr, 24, prof), f"sequence {b}"
    model.free()


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

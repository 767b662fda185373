"""Pins of the oracle's SiLU*mul and of its whole-step composition (oracle/lt_oracle.c
or_silu_mul, or_silu_mul_quant, or_decode_step, or_generate) by checks that do not restate it.

* SiLU*mul (reference formula v = (g / (1 + expf(-g))) * u, bpd/lib/dev_residency.py:583):
  a float64 bound, exact special cases, and constructed inputs on which the reference's
  operation order gives different bits from the other plausible orders.
* The decode step (bpd/lib/dev_residency.py:1328-1623; the equations of the reference's own
  torch model, bpd/llamatov_run.py:513-550, 845-857): compared with tests/f64_model.py, a
  float64 restatement written from the model equations on dequantized weights.  At the small
  TINY sizes the two agree to float32 rounding (no activation-quantization code flips at the
  seeds used); at SMALL_QWEN size, where flips at rounding boundaries do occur, within a bound
  derived from the quantization step.  The KV rows are compared too: RoPE is relative, so an
  absolute-position error is invisible in the logits with an fp32 cache but not in the cached K.
  Planted wiring mistakes (bias after RoPE, RoPE at pos + 1, gate/up swapped, no attention
  residual, attention without the new row, wrong head) exceed the tolerances.
* An invariant: with every layer's matrices zero, the embedding reaches the final norm unchanged,
  so the logits are the head GEMV of the normalized embedding, bit for bit.
"""
import numpy as np
import pytest

from llamatov_amd import model as M
from llamatov_amd import q8 as hq8

from f64_model import F64Model


def ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, np.int64(-2**31) - a, a)
    b = np.where(b < 0, np.int64(-2**31) - b, b)
    return np.abs(a - b)


# ---- SiLU * mul ----------------------------------------------------------------------
def test_silu_mul_float64_bound(oracle):
    rng = np.random.default_rng(41)
    g = np.concatenate([rng.uniform(-100, 100, 40000), rng.uniform(-8, 8, 40000),
                        rng.standard_normal(20000) * 1e-3]).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32) * np.float32(3.0)
    v = oracle.silu_mul(g, u)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    with np.errstate(over="ignore"):
        ref = gd / (1.0 + np.exp(-gd)) * ud
    # where e^-g exceeds the float32 range (g < -88.72) the float32 exp is +inf and the
    # quotient is a signed zero
    ovf = np.exp(-gd) > np.finfo(np.float32).max
    assert ovf.sum() > 1000
    assert np.all(v[ovf] == 0.0)
    assert np.array_equal(np.signbit(v[ovf]), np.signbit(g[ovf]) != np.signbit(u[ovf]))
    # four roundings (exp <= 1 ulp, add, divide, multiply): at most 3 ulp of the exact value
    # for normal results; results below the normal range to within 4 subnormal steps
    normal = (np.abs(ref) >= 2.0 ** -126) & ~ovf
    assert ulp_diff(v[normal], ref[normal].astype(np.float32)).max() <= 3
    sub = ~normal & ~ovf
    assert np.all(np.abs(v[sub].astype(np.float64) - ref[sub]) <= 4 * 2.0 ** -149)


def test_silu_mul_special_cases(oracle):
    g = np.array([0.0, -0.0, 3.0, -3.0, 20.0, 50.0, 88.0, 1e4, -1e4, -100.0, 7.25], np.float32)
    u = np.array([5.0, 5.0, 0.0, 0.0, 1.5, -2.25, 3.0, 0.5, 2.0, 1.0, -0.0], np.float32)
    v = oracle.silu_mul(g, u)
    assert v[0] == 0.0 and v[1] == 0.0                       # g = +-0 -> 0
    assert v[2] == 0.0 and v[3] == 0.0 and v[10] == 0.0      # u = 0 -> 0
    # large positive g: 1 + e^-g rounds to 1, so v = fl(g * u) exactly
    for i in (4, 5, 6, 7):
        assert v[i] == np.float32(g[i]) * np.float32(u[i])
    # very negative g: e^-g overflows (or nearly), g / (1 + e^-g) -> -0, then * u
    assert v[8] == 0.0 and np.signbit(v[8])
    assert v[9] == np.float32(-100.0 / (1.0 + np.exp(100.0))) * np.float32(1.0) or v[9] == 0.0
    # the quantizing variant is quant(silu_mul)
    rng = np.random.default_rng(3)
    G = rng.standard_normal(4864).astype(np.float32) * 3
    U = rng.standard_normal(4864).astype(np.float32)
    xq, xd = oracle.silu_mul_quant(G, U)
    rq, rd = oracle.quant_q8(oracle.silu_mul(G, U))
    assert np.array_equal(xq, rq) and np.array_equal(xd, rd)


def test_silu_mul_operation_order_is_pinned(oracle):
    """(g / (1 + e)) * u differs in the last bit from g * (u / (1 + e)), (g * u) / (1 + e) and
    g * (1 / (1 + e)) * u on some inputs; the oracle must give the reference order's bits
    everywhere (e = expf(-g) from the oracle's exp, pinned separately to <= 1 ulp)."""
    rng = np.random.default_rng(77)
    g = rng.uniform(-6, 6, 20000).astype(np.float32)
    u = rng.uniform(-4, 4, 20000).astype(np.float32)
    v = oracle.silu_mul(g, u)
    e = np.array([oracle.expf(float(-x)) for x in g], np.float32)
    one = np.float32(1.0)
    den = (one + e).astype(np.float32)
    ref = ((g / den).astype(np.float32) * u).astype(np.float32)
    alts = [(g * (u / den).astype(np.float32)).astype(np.float32),
            ((g * u).astype(np.float32) / den).astype(np.float32),
            ((g * (one / den).astype(np.float32)).astype(np.float32) * u).astype(np.float32)]
    assert np.array_equal(v.view(np.uint32), ref.view(np.uint32))
    for a in alts:
        assert np.count_nonzero(a.view(np.uint32) != ref.view(np.uint32)) > 100


# ---- the decode step against the float64 restatement --------------------------------
def _weights(cfg, seed, bias_std=0.5):
    """Synthetic weights with large q/k/v biases, so that where the bias is added matters."""
    w = M.synth_weights(cfg, seed=seed)
    rng = np.random.default_rng(seed)
    for k in list(w):
        if k.endswith(".bias"):
            w[k] = (rng.standard_normal(w[k].shape) * bias_std).astype(np.float32)
    return w


def _run(oracle, cfg, w, prompt, kv_f16, mistake=None):
    o = oracle.OracleModel(cfg, w, kv_f16=kv_f16)
    f = F64Model(cfg, w, kv_f16=kv_f16, mistake=mistake)
    logit_err, kv_err = [], []
    for i, t in enumerate(prompt):
        a = o.step(t).astype(np.float64)
        b = f.step(t)
        logit_err.append(np.abs(a - b).max() / np.abs(b).max())
        e = 0.0
        for il in range(cfg.n_layers):
            for which, rows in (("k", f.K[il]), ("v", f.V[il])):
                got = o.kv_rows(il, which, i + 1)
                got = got.view(np.float16).astype(np.float64) if kv_f16 else got.astype(np.float64)
                ref = np.stack(rows)
                e = max(e, np.abs(got - ref).max() / np.abs(ref).max())
        kv_err.append(e)
    return max(logit_err), max(kv_err)


TINY_UNTIED = M.TINY.replace(name="tiny-untied", tied=False, qkv_bias=False)
TINY_GQA4 = M.TINY.replace(name="tiny-gqa4", n_head=8, n_head_kv=2, n_embd=256, n_ff=512)
# float32 rounding of a TINY step stays near 1e-7 of the logits' scale; the fp16 KV rows
# agree to one fp16 rounding (2^-11) where a float32 and a float64 value straddle a midpoint
TIGHT_LOGITS, TIGHT_KV32, TIGHT_KV16 = 1e-6, 1e-6, 2.0 ** -10


@pytest.mark.parametrize("cfg", [M.TINY, TINY_UNTIED, TINY_GQA4], ids=lambda c: c.name)
@pytest.mark.parametrize("kv_f16", [False, True])
def test_step_composition_matches_float64_equations(oracle, cfg, kv_f16):
    w = _weights(cfg, 31)
    prompt = M.random_prompt(cfg, 8, seed=31)
    le, ke = _run(oracle, cfg, w, prompt, kv_f16)
    assert le <= TIGHT_LOGITS, le
    assert ke <= (TIGHT_KV16 if kv_f16 else TIGHT_KV32), ke


def _quant_step_bound(cfg) -> float:
    # one code flip moves a dequantized activation element by one step (1/127 of its block's
    # amax, about 1/254 of the block's scale on average); four quantized activations per
    # layer, each able to flip, and the effects add across layers
    return 4 * cfg.n_layers / 254.0


@pytest.mark.parametrize("kv_f16", [False, True])
def test_step_composition_small_qwen_within_quant_bound(oracle, kv_f16):
    cfg = M.SMALL_QWEN
    w = _weights(cfg, 33)
    prompt = M.random_prompt(cfg, 6, seed=33)
    le, ke = _run(oracle, cfg, w, prompt, kv_f16)
    assert le <= _quant_step_bound(cfg), le
    assert ke <= _quant_step_bound(cfg), ke


@pytest.mark.parametrize("mistake,cfg", [
    ("bias_after_rope", M.TINY), ("rope_pos_plus1", M.TINY), ("gate_up_swapped", M.TINY),
    ("no_attn_residual", M.TINY), ("attend_without_new", M.TINY), ("head_from_embd", TINY_UNTIED),
    ("gate_up_swapped", M.SMALL_QWEN), ("no_attn_residual", M.SMALL_QWEN),
    ("attend_without_new", M.SMALL_QWEN)])
def test_planted_wiring_mistakes_exceed_the_tolerances(oracle, mistake, cfg):
    """Each plausible misreading, planted in the float64 restatement, is caught by the
    comparison above: the oracle and the mistaken model differ beyond the tolerance used."""
    w = _weights(cfg, 31 if cfg is not M.SMALL_QWEN else 33)
    prompt = M.random_prompt(cfg, 6, seed=31 if cfg is not M.SMALL_QWEN else 33)
    le, ke = _run(oracle, cfg, w, prompt, False, mistake=mistake)
    if cfg is M.SMALL_QWEN:
        assert max(le, ke) > 4 * _quant_step_bound(cfg), (le, ke)
    else:
        assert le > 1e3 * TIGHT_LOGITS or ke > 1e3 * TIGHT_KV32, (le, ke)


def test_zeroed_layers_pass_the_embedding_to_the_final_norm(oracle):
    """With every layer matrix zero (biases kept), each GEMV adds 0 to its residual, so the
    embedding reaches the final norm unchanged: logits == head(Q8(rmsnorm(embed(tok))))."""
    cfg = M.TINY
    w = _weights(cfg, 5)
    for k in list(w):
        if k.startswith("blk.") and k.endswith(".weight") and "norm" not in k:
            N, nbytes = w[k].shape
            w[k] = hq8.quantize_rows(np.zeros((N, nbytes // 34 * 32), np.float32))
    o = oracle.OracleModel(cfg, w)
    for tok in (0, 7, 311):
        got = o.step(tok)
        x = oracle.embed_row(w["token_embd.weight"], tok, cfg.n_embd)
        xq, xd = oracle.quant_q8(oracle.rmsnorm(x, w["output_norm.weight"], cfg.norm_eps))
        exp = oracle.q8_gemv(w["token_embd.weight"], xq, xd, cfg.n_embd)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_generate_is_greedy_over_steps(oracle):
    """or_generate feeds the prompt through or_decode_step and each argmax back in."""
    cfg = M.TINY
    w = _weights(cfg, 8)
    prompt = M.random_prompt(cfg, 5, seed=8)
    o = oracle.OracleModel(cfg, w)
    toks, margins = o.generate(prompt, 6)
    o2 = oracle.OracleModel(cfg, w)
    for t in prompt:
        lg = o2.step(t)
    exp = []
    for _ in range(6):
        t = int(np.argmax(lg))
        s = np.sort(lg)
        exp.append(t)
        assert margins[len(exp) - 1] == s[-1] - s[-2]
        lg = o2.step(t)
    assert toks == exp

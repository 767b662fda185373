"""Long-run check at C2 (the reference's long-run referee, bpd/kernelgen/referee/
long_run_referee.py:150-212): six prompts of different lengths, 128 greedy tokens each,
through the production profile's captured step (the persistent step while the cache fits it,
the five-launch step past that), against the oracle.

Per prompt it reports token agreement, the largest |device logit - oracle logit| over the
steps (the drift), and the min and median top-1/top-2 margin of the oracle's logits; over all
decisions it reports the margin statistics, the safety factor min margin / max drift and the
near-flip census (steps whose margin is within 5x the drift).  The pass condition is the
reference's "token-exact at scale" plus this build's own bar: zero drift, i.e. logits equal
bit for bit at every one of the 768 steps."""
import statistics

import numpy as np
import pytest

from llamatov_amd import engine as dr
from llamatov_amd import model as M

pytestmark = pytest.mark.gpu

PROMPT_LENS = (5, 17, 32, 64, 100, 150)
N_GEN = 128


def case(msg):
    print(f"[gpu-case] {msg}", flush=True)


def top2(x):
    i = int(np.argmax(x))
    second = np.partition(x, -2)[-2]
    return i, float(x[i] - second)


def test_long_run_six_prompts_128_tokens(gpu, oracle):
    cfg = M.QWEN25_05B
    case("long-run C2 weights")
    w = M.synth_weights(cfg, seed=2024)
    m = dr.ResidentModel(cfg, w, gpu)
    plan = dr.DecodePlan(m, dr.PRODUCTION_PROFILE, max_ctx=cfg.max_ctx)
    all_margins, near_flips, max_drift, persistent_seen = [], [], 0.0, set()
    try:
        for pi, n in enumerate(PROMPT_LENS):
            case(f"long-run prompt {pi} ({n} tokens + {N_GEN})")
            prompt = M.random_prompt(cfg, n, seed=100 + pi)
            orc = oracle.OracleModel(cfg, w)
            for t in prompt:
                exp = orc.step(t)
            plan.reset()
            gr = dr.StepGraph(plan)
            gr.seed(prompt)
            got = plan.read_logits().copy()
            gr.capture()
            gen_dev, gen_orc, margins, drifts = [], [], [], []
            for step in range(N_GEN):
                tok, margin = top2(exp)
                d = float(np.abs(got - exp).max())
                drifts.append(d)
                margins.append(margin)
                if d > 0 and margin < 5 * d:
                    near_flips.append((pi, step, margin, d))
                gen_orc.append(tok)
                gen_dev.append(int(np.argmax(got)))
                if step + 1 < N_GEN:
                    persistent_seen.add(plan.persistent)
                    got = gr.replay_logits(gen_dev[-1]).copy()
                    exp = orc.step(tok)
            assert plan.error() == 0
            gr.free()
            agree = gen_dev == gen_orc
            print(f"prompt {pi}: agree={'FULL' if agree else 'DIVERGED'}  max_drift={max(drifts):.3e}  "
                  f"min_margin={min(margins):.4f}  median={statistics.median(margins):.4f}", flush=True)
            assert agree, f"prompt {pi}: tokens diverge at step {next(i for i, (a, b) in enumerate(zip(gen_dev, gen_orc)) if a != b)}"
            max_drift = max(max_drift, max(drifts))
            all_margins += margins
    finally:
        plan.free()
        m.free()
    sf = min(all_margins) / max_drift if max_drift > 0 else float("inf")
    print(f"margin statistics over {len(all_margins)} decisions: min={min(all_margins):.4f}  "
          f"median={statistics.median(all_margins):.4f}  max={max(all_margins):.4f}", flush=True)
    print(f"max_drift={max_drift:.3e}  safety factor (min margin / max drift) = {sf}  "
          f"near-flip census: {len(near_flips)} steps within 5x", flush=True)
    assert len(all_margins) == len(PROMPT_LENS) * N_GEN
    assert persistent_seen == {True, False}      # both step forms took part
    assert max_drift == 0.0 and not near_flips

"""Generation from a Q8_0 GGUF file on the device:

    python -m llamatov_amd.generate MODEL.gguf --ids 1,415,6557 -n 6
    python -m llamatov_amd.generate MODEL.gguf --prompt "Once upon a time" -n 32 --temperature 0.8

prints one JSON line with the generated ids (and text, when the prompt is text) and the
decode rate.  The command-line counterpart of the reference's decode entry points
(bpd/decode_fact.py:54-111, bpd/llamatov_run.py:863-1196); a text prompt goes through the
GGUF's own byte-level BPE vocabulary (llamatov_amd.tokenizer, the reference's qwen_bpe.py).
Greedy by default; --temperature > 0 draws with the device sampler (top-k, top-p, seed).
"""
from __future__ import annotations

import argparse
import json
import time


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("model", help="Q8_0 GGUF file")
    src = ap.add_mutually_exclusive_group(required=True)
    src.add_argument("--ids", help="prompt token ids, comma separated")
    src.add_argument("--prompt", help="prompt text (needs tokenizer.ggml.tokens/merges in the GGUF)")
    ap.add_argument("--temperature", type=float, default=0.0, help="0 = greedy")
    ap.add_argument("--top-k", type=int, default=40)
    ap.add_argument("--top-p", type=float, default=1.0)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("-n", "--n-tokens", type=int, default=16)
    ap.add_argument("--kv", choices=("f32", "f16"), default="f32",
                    help="KV cache element type (f32 = the reference's cache)")
    ap.add_argument("--nsplit", type=int, default=1, help="attention split-K factor")
    ap.add_argument("--max-ctx", type=int, default=1024)
    ap.add_argument("--token-by-token", action="store_true",
                    help="prefill one token at a time instead of the batched GEMM (same bits)")
    a = ap.parse_args(argv)

    from . import engine as dr
    tok = None
    if a.prompt is not None:
        from .tokenizer import QwenBPE
        tok = QwenBPE(a.model)
        ids = tok.encode(a.prompt)
    else:
        ids = [int(t) for t in a.ids.split(",") if t.strip()]
    sampling = None
    if a.temperature > 0:
        sampling = dict(temperature=a.temperature, top_k=a.top_k, top_p=a.top_p, seed=a.seed)
    t0 = time.perf_counter()
    model = dr.ResidentModel.from_gguf(a.model, max_ctx=a.max_ctx)
    t1 = time.perf_counter()
    prof = dr.Profile(kv_dtype=dr.LT_KV_F16 if a.kv == "f16" else dr.LT_KV_F32, attn_nsplit=a.nsplit)
    try:
        out = dr.generate(model, ids, a.n_tokens, prof, batched_prefill=not a.token_by_token,
                          max_ctx=a.max_ctx, sampling=sampling)
    finally:
        t2 = time.perf_counter()
        model.free()
    rep = model.load_report
    rec = {"text": tok.decode(out)} if tok is not None else {}
    print(json.dumps({"model": a.model, "config": model.cfg.name, "prompt": ids, "tokens": out, **rec,
                      "load_s": round(t1 - t0, 3), "generate_s": round(t2 - t1, 3),
                      "load": {"verbatim": rep.verbatim, "canonicalized": rep.canonicalized,
                               "blocks_replaced": rep.blocks_replaced,
                               "requantized": rep.requantized}}))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

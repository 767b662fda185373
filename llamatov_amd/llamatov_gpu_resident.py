"""The reference's GPU-resident decode loop, bpd/llamatov_gpu_resident.py: run(path, input_ids,
n_tokens=10) (:20-235) and its command line (:237-246), over this build's device engine.

The reference's run() keeps activations on the GPU between its ops, moves attention through
the host and prints the tokens it decodes: the prompt's greedy continuation (its "first
token", :207-211) and then n_tokens more (:212-217), n_tokens + 1 new tokens in all, with the
throughput over the n_tokens decode steps.  Here the whole step stays on the device (Q8_0
weights uploaded verbatim from the file, batched prefill, then one graph replay per token),
and the same lines are printed.  run() also returns prompt + new tokens, which the reference
leaves in a local list.
"""
from __future__ import annotations

import sys
import time

from .gguf import parse_gguf


def _tok_str(tokens, t: int) -> str:
    return repr(tokens[t]) if t < len(tokens) else "?"


def run(path, input_ids, n_tokens=10):
    """Greedy decode of n_tokens + 1 tokens after input_ids from the Q8_0 GGUF at `path`, on
    GPU 0; prints the reference's report lines and returns input_ids + the new tokens."""
    from . import engine
    t0 = time.time()
    print("=== LlamaTov GPU-Resident Inference ===")
    md, _, _ = parse_gguf(path)
    arch = md.get("general.architecture", "llama")
    g = lambda k, dflt: md.get(f"{arch}.{k}", dflt)
    print(f"Arch: {arch}, layers: {g('block_count', 16)}, heads: {g('attention.head_count', 32)}/"
          f"{g('attention.head_count_kv', 8)}, embd: {g('embedding_length', 2048)}")
    ids = [int(t) for t in input_ids]
    if not ids:
        raise ValueError("run: empty prompt")
    n_new = int(n_tokens) + 1
    max_ctx = max(1024, len(ids) + n_new)
    print("Uploading weights to GPU...")
    model = engine.ResidentModel.from_gguf(path, max_ctx=max_ctx)
    try:
        print(f"Loaded and uploaded in {time.time() - t0:.1f}s")
        print(f"Running ({len(ids)} prefill + {n_tokens} decode)...")
        t_gen = time.time()
        out = engine.generate(model, ids, n_new, max_ctx=max_ctx)
        gen_time = time.time() - t_gen
    finally:
        model.free()
    tokens = md.get("tokenizer.ggml.tokens", [])
    print(f"  Prefill → first token: {out[0]} = {_tok_str(tokens, out[0])}")
    for i, t in enumerate(out[1:]):
        if i < 3 or i == n_tokens - 1:
            print(f"  Step {i}: token {t} = {_tok_str(tokens, t)}")
    tok_s = n_tokens / gen_time if gen_time > 0 else float("inf")
    print("\n=== RESULTS ===")
    print(f"Generated: {n_tokens} tokens in {gen_time:.2f}s")
    print(f"Throughput: {tok_s:.1f} tok/s")
    return ids + out


def main(argv=None) -> int:
    """`python -m llamatov_amd.llamatov_gpu_resident MODEL.gguf [N]`: [BOS, 'Hello'] and N
    tokens, as the reference's command line does."""
    argv = sys.argv[1:] if argv is None else argv
    if not argv:
        print("usage: python -m llamatov_amd.llamatov_gpu_resident MODEL.gguf [N_TOKENS]")
        return 2
    path = argv[0]
    n = int(argv[1]) if len(argv) > 1 else 10
    md, _, _ = parse_gguf(path)
    bos = md.get("tokenizer.ggml.bos_token_id", 1)
    tokens = md.get("tokenizer.ggml.tokens", [])
    hello = next((i for i, t in enumerate(tokens) if t == "Hello"), None)
    if hello is None:
        print("No 'Hello' token")
        return 1
    print(f"BOS={bos}, Hello={hello}")
    run(path, [bos, hello], n)
    return 0


if __name__ == "__main__":
    sys.exit(main())

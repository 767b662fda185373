"""The reference's model-file and generation entry points, bpd/llamatov_run.py, with its
signatures: parse_gguf(path) (:9-40), lt(path, data_offset, info) (:497-511),
load_model(path, device) (:933-953) and generate(path, input_ids, n_tokens, device, preloaded)
(:955-1177).

generate() runs the device decode path on the MI355X: the reference's engine semantics
(Q8_0 weights and activations, bpd/lib/dev_residency.py), not the fp32 torch model of the
reference's own generate().  `device` names where a torch caller keeps tensors in the
reference; this build has no CPU path and runs on one GPU, so "cpu", "cuda" and "cuda:0"
all decode on GPU 0 ("cuda:N" with N > 0 is refused).  The return value is the reference's:
(prompt + generated token ids, tok/s).
"""
from __future__ import annotations

import time

import numpy as np

from .gguf import parse_gguf, lt  # noqa: F401  (the reference's names, re-exported)


def _gpu_index(device) -> int:
    d = str(device)
    if ":" in d:
        return int(d.split(":", 1)[1])
    return 0


def load_model(path, device="cpu"):
    """(cfg, w): the reference's config dict and its fp32 weight dict ([ne0, ne1] orientation,
    torch tensors when torch is importable, else numpy arrays)."""
    md, ts, do = parse_gguf(path)
    arch = md.get("general.architecture", "llama")
    g = lambda k, dflt: md.get(f"{arch}.{k}", dflt)
    cfg = {
        "arch": arch,
        "n_layers": g("block_count", 12),
        "n_head": g("attention.head_count", 12),
        "n_head_kv": g("attention.head_count_kv", g("attention.head_count", 12)),
        "head_dim": g("attention.key_length", None),
        "moe_top_k": g("expert_used_count", 8),
        "n_embd": g("embedding_length", 768),
        "rope_theta": g("rope.freq_base", 500000.0),
        "norm_eps": g("attention.layer_norm_rms_epsilon", g("attention.layer_norm_epsilon", 1e-5)),
    }
    w = {n: lt(path, do, info) for n, info in ts.items()}
    try:
        import torch
        w = {n: torch.from_numpy(np.ascontiguousarray(a)) for n, a in w.items()}
    except ImportError:
        pass
    return cfg, w


def generate(path, input_ids, n_tokens=20, device="cpu", preloaded=None):
    """Greedy generation of n_tokens after input_ids on the device decode path; returns
    (input_ids + generated ids, tokens per second).  preloaded=(cfg, w) reuses a loaded model
    (its fp32 weights are quantized to Q8_0 at first use, as the reference's device path
    does); otherwise the Q8_0 blocks of the GGUF file go to the device verbatim."""
    from . import engine
    if _gpu_index(device) != 0:
        raise ValueError(f"generate: device {device!r}: this build decodes on GPU 0")
    ids = [int(t) for t in np.asarray(input_ids).reshape(-1)]
    if not ids:
        raise ValueError("generate: empty prompt")
    if n_tokens < 1:
        return ids, 0.0
    t0 = time.time()
    print(f"=== LlamaTov Generate ===\nModel: {path}")
    if preloaded is not None:
        from . import dev_residency as dr
        cfg, w = preloaded
        saved = dr._KV_MAX_SEQ
        dr._KV_MAX_SEQ = max(saved, len(ids) + n_tokens)
        kv = [None] * int(cfg["n_layers"])
        gr = dr.GraphRunner(w, cfg, kv)
        try:
            t_gen = time.time()
            lg = gr.seed(np.asarray(ids), np.arange(len(ids)))
            out = [int(np.asarray(lg).reshape(-1).argmax())]
            if n_tokens > 1:
                gr.capture([out[-1]], [len(ids)])
                for _ in range(n_tokens - 1):
                    out.append(gr.replay_token([out[-1]]))
            out = out[:n_tokens]
            gen_time = time.time() - t_gen
        finally:
            gr.free()
            plan = getattr(kv[0], "_plan", None)
            if plan is not None:
                plan.free()
            dr.release_resident(w)   # the device copy of this dict's weights
            dr._KV_MAX_SEQ = saved
    else:
        model = engine.ResidentModel.from_gguf(path, max_ctx=max(1024, len(ids) + n_tokens))
        try:
            t_gen = time.time()
            out = engine.generate(model, ids, n_tokens, max_ctx=max(1024, len(ids) + n_tokens))
            gen_time = time.time() - t_gen
        finally:
            model.free()
    generated = ids + out
    tok_per_sec = n_tokens / gen_time if gen_time > 0 else float("inf")
    print(f"Generated {n_tokens} tokens in {gen_time:.2f}s")
    print(f"Throughput: {tok_per_sec:.1f} tok/s")
    print(f"Total (load + gen): {time.time() - t0:.2f}s")
    print(f"Tokens: {generated}")
    return generated, tok_per_sec

"""Model configurations and seeded synthetic Q8_0 weights.

Tensor names and orientations follow GGUF as the reference loader reads them
(bpd/llamatov_run.py:9-40, 497-511; names used by forward_pass_resident,
bpd/lib/dev_residency.py:1380-1477): a linear weight is stored as N output rows of K
inputs, i.e. Q8_0 blocks [N][K/32].  The lm_head is tied to token_embd when
`tied` (Qwen2, dev_residency.py:1057); Qwen2 carries q/k/v biases
(dev_residency.py:1177-1193); head_dim = n_embd // n_head (dev_residency.py:1337).

Synthetic weights: numpy default_rng(seed + crc32(name)), N(0, 0.02) fp32 quantized to
Q8_0 with the engine quantizer; norm weights 1.0 (or 1 + 0.1 N(0,1) for the test
configurations, to exercise the multiply); q/k/v biases N(0, 0.02).
"""
from __future__ import annotations

import dataclasses
import zlib
from dataclasses import dataclass

import numpy as np

from . import q8


@dataclass(frozen=True)
class ModelConfig:
    name: str
    n_layers: int
    n_embd: int
    n_ff: int
    n_head: int
    n_head_kv: int
    vocab: int
    rope_theta: float
    norm_eps: float
    tied: bool = True
    qkv_bias: bool = False
    max_ctx: int = 1024
    norm_init: str = "ones"        # "ones" | "random"

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_head

    @property
    def q_dim(self) -> int:
        return self.n_head * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_head_kv * self.head_dim

    @property
    def n_qkv(self) -> int:
        return self.q_dim + 2 * self.kv_dim

    def replace(self, **kw) -> "ModelConfig":
        return dataclasses.replace(self, **kw)

    def as_cfg(self) -> dict:
        """The reference's cfg dict keys (decode_fact.load_model, bpd/decode_fact.py:39-51)."""
        return {"n_layers": self.n_layers, "n_embd": self.n_embd, "n_head": self.n_head,
                "n_head_kv": self.n_head_kv, "rope_theta": self.rope_theta,
                "norm_eps": self.norm_eps, "n_ff": self.n_ff, "vocab": self.vocab}

    def weight_bytes(self) -> int:
        """Q8_0 weight bytes streamed per decode token (tied lm_head counted once)."""
        rb = q8.row_bytes
        E, F = self.n_embd, self.n_ff
        per_layer = (self.n_qkv * rb(E) + E * rb(self.q_dim) + 2 * F * rb(E) + E * rb(F))
        lm = self.vocab * rb(E)
        return self.n_layers * per_layer + lm


# Qwen2.5-0.5B architecture.
QWEN25_05B = ModelConfig("qwen2.5-0.5b-arch", n_layers=24, n_embd=896, n_ff=4864, n_head=14,
                         n_head_kv=2, vocab=151936, rope_theta=1e6, norm_eps=1e-6, tied=True,
                         qkv_bias=True, max_ctx=1024)
# Llama-3-8B architecture.
LLAMA3_8B = ModelConfig("llama-3-8b-arch", n_layers=32, n_embd=4096, n_ff=14336, n_head=32,
                        n_head_kv=8, vocab=128256, rope_theta=5e5, norm_eps=1e-5, tied=False,
                        qkv_bias=False, max_ctx=1024)
# Small configurations for tests (same code paths, seconds on the CPU oracle).
TINY = ModelConfig("tiny", n_layers=2, n_embd=128, n_ff=256, n_head=4, n_head_kv=2, vocab=512,
                   rope_theta=1e4, norm_eps=1e-6, tied=True, qkv_bias=True, max_ctx=64,
                   norm_init="random")
SMALL_QWEN = ModelConfig("small-qwen-arch", n_layers=4, n_embd=896, n_ff=4864, n_head=14,
                         n_head_kv=2, vocab=4096, rope_theta=1e6, norm_eps=1e-6, tied=True,
                         qkv_bias=True, max_ctx=256, norm_init="random")

CONFIGS = {c.name: c for c in (QWEN25_05B, LLAMA3_8B, TINY, SMALL_QWEN)}


def tensor_seed(base: int, name: str) -> int:
    return (base + zlib.crc32(name.encode())) & 0xFFFFFFFF


def _normal(base: int, name: str, shape, std: float) -> np.ndarray:
    rng = np.random.default_rng(tensor_seed(base, name))
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def _q8_normal(base: int, name: str, N: int, K: int, std: float = 0.02,
               chunk_rows: int = 4096) -> np.ndarray:
    rng = np.random.default_rng(tensor_seed(base, name))
    out = np.empty((N, q8.row_bytes(K)), dtype=np.uint8)
    for r0 in range(0, N, chunk_rows):
        n = min(chunk_rows, N - r0)
        w = rng.standard_normal((n, K), dtype=np.float32) * np.float32(std)
        out[r0:r0 + n] = q8.quantize_rows(w)
    return out


def _norm_weight(cfg: ModelConfig, base: int, name: str, n: int) -> np.ndarray:
    if cfg.norm_init == "ones":
        return np.ones(n, dtype=np.float32)
    return (np.float32(1.0) + _normal(base, name, (n,), 0.1)).astype(np.float32)


def weight_specs(cfg: ModelConfig) -> list[tuple[str, str, tuple]]:
    """(name, kind, shape) of every tensor: kind 'q8' (N, K), 'norm' (n,), 'bias' (n,)."""
    E, F = cfg.n_embd, cfg.n_ff
    specs = [("token_embd.weight", "q8", (cfg.vocab, E))]
    if not cfg.tied:
        specs.append(("output.weight", "q8", (cfg.vocab, E)))
    specs.append(("output_norm.weight", "norm", (E,)))
    for il in range(cfg.n_layers):
        p = f"blk.{il}"
        specs += [(f"{p}.attn_norm.weight", "norm", (E,)),
                  (f"{p}.attn_q.weight", "q8", (cfg.q_dim, E)),
                  (f"{p}.attn_k.weight", "q8", (cfg.kv_dim, E)),
                  (f"{p}.attn_v.weight", "q8", (cfg.kv_dim, E))]
        if cfg.qkv_bias:
            specs += [(f"{p}.attn_q.bias", "bias", (cfg.q_dim,)),
                      (f"{p}.attn_k.bias", "bias", (cfg.kv_dim,)),
                      (f"{p}.attn_v.bias", "bias", (cfg.kv_dim,))]
        specs += [(f"{p}.attn_output.weight", "q8", (E, cfg.q_dim)),
                  (f"{p}.ffn_norm.weight", "norm", (E,)),
                  (f"{p}.ffn_gate.weight", "q8", (F, E)),
                  (f"{p}.ffn_up.weight", "q8", (F, E)),
                  (f"{p}.ffn_down.weight", "q8", (E, F))]
    return specs


def synth_weights(cfg: ModelConfig, seed: int = 1234, workers: int | None = None) -> dict[str, np.ndarray]:
    """GGUF-named tensors: Q8_0 blocks (uint8 [N, K/32*34]) and fp32 vectors.  Each tensor
    has its own seeded generator, so the result does not depend on the worker count."""
    import os
    from concurrent.futures import ThreadPoolExecutor

    def make(spec):
        name, kind, shape = spec
        if kind == "q8":
            return name, _q8_normal(seed, name, shape[0], shape[1])
        if kind == "norm":
            return name, _norm_weight(cfg, seed, name, shape[0])
        return name, _normal(seed, name, shape, 0.02)

    specs = weight_specs(cfg)
    n = workers or min(16, len(os.sched_getaffinity(0)))
    with ThreadPoolExecutor(max_workers=n) as ex:
        return dict(ex.map(make, specs))


def fused_layer_tensors(cfg: ModelConfig, w: dict, il: int) -> dict[str, np.ndarray]:
    """The concatenations the reference builds at first use: q|k|v rows with their biases
    (_fused_qkv_weight, bpd/lib/dev_residency.py:1283-1306) and gate|up rows
    (_fused_gateup_weight)."""
    p = f"blk.{il}"
    out = {
        "attn_norm": w[f"{p}.attn_norm.weight"],
        "wqkv": np.ascontiguousarray(np.concatenate(
            [w[f"{p}.attn_q.weight"], w[f"{p}.attn_k.weight"], w[f"{p}.attn_v.weight"]], axis=0)),
        "wo": w[f"{p}.attn_output.weight"],
        "ffn_norm": w[f"{p}.ffn_norm.weight"],
        "wgu": np.ascontiguousarray(np.concatenate(
            [w[f"{p}.ffn_gate.weight"], w[f"{p}.ffn_up.weight"]], axis=0)),
        "wdown": w[f"{p}.ffn_down.weight"],
    }
    if f"{p}.attn_q.bias" in w:
        out["bqkv"] = np.ascontiguousarray(np.concatenate(
            [w[f"{p}.attn_q.bias"], w[f"{p}.attn_k.bias"], w[f"{p}.attn_v.bias"]]).astype(np.float32))
    else:
        out["bqkv"] = None
    return out


def interleave_gateup(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """gate [F, rb] and up [F, rb] Q8_0 block rows -> [2F, rb] with row 2j = gate j and
    row 2j+1 = up j: the layout of the fused gate|up GEMV, whose workgroups hold a gate row
    and its up row on the two halves of one wave.  Each row's dot product is unchanged."""
    F = gate.shape[0]
    out = np.empty((2 * F, gate.shape[1]), dtype=gate.dtype)
    out[0::2] = gate
    out[1::2] = up
    return out


def random_prompt(cfg: ModelConfig, n: int, seed: int = 7) -> list[int]:
    rng = np.random.default_rng(seed)
    return [int(t) for t in rng.integers(0, cfg.vocab, size=n)]

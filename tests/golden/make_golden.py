#!/usr/bin/env python3
"""Writes the committed golden fixtures of the Q8_0 decode path (tests/golden/*.npz).

The reference holds no value fixtures for this path: its bpd/tests/fixtures/*.npy cover
activation functions and row reductions only, and its gates store seeds and shapes, not
outputs.  These fixtures are the outputs of the CPU restatement (oracle/lt_oracle.c) on
the reference gates' shapes, seeds and distributions:
  gemv_canonical: gemv_canonical_pairgate.py:36-42 / q8_referee.py:23-93 (64x256, seed 11);
  quant_q8:       gate_quant_par.py:21-45 (x = 2*N(0,1), seed 7, K = 896);
  rmsnorm:        rms_canonical_pairgate.py:22-48 (N=896, eps 1e-6, seed 7);
  rope:           rope_from_facts.pl:40-69 (hd 64, theta 1e6, 16 heads);
  attention:      masked single pass and split-K (dev_residency.py:1955-2031,
                  attn_decode_split.cu:14-91), fp32 and fp16 caches;
  decode_tiny:    16 greedy tokens + final logits of the TINY synthetic model.
The oracle itself is pinned independently (closed forms, float64 bounds, order pins) by
tests/test_oracle_pins.py; these files freeze its values so that any later change to the
oracle or the kernels that moves a bit is caught.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from llamatov_amd import model as M  # noqa: E402
from llamatov_amd import q8 as hq8  # noqa: E402
from oracle import oracle as orc  # noqa: E402

OUT = Path(__file__).resolve().parent


def weights_digest(w: dict) -> str:
    h = hashlib.sha256()
    for k in sorted(w):
        h.update(k.encode())
        h.update(np.ascontiguousarray(w[k]).tobytes())
    return h.hexdigest()


def main() -> None:
    # GEMV (canonical order) + residual epilogue + per-block int32 dots
    rng = np.random.default_rng(11)
    N, K = 64, 256
    q = rng.integers(-127, 128, size=(N, K), dtype=np.int64).astype(np.int8)
    d = (rng.standard_normal((N, K // 32)) * 0.1).astype(np.float16).view(np.uint16)
    W = hq8.join_blocks(q, d)
    xq = rng.integers(-127, 128, size=K, dtype=np.int64).astype(np.int8)
    xd = (rng.standard_normal(K // 32) * 0.1).astype(np.float16).view(np.uint16)
    resid = rng.standard_normal(N).astype(np.float32)
    np.savez_compressed(OUT / "gemv_canonical_64x256.npz", W=W, xq=xq, xd=xd, resid=resid,
                        y=orc.q8_gemv(W, xq, xd, K), y_resid=orc.q8_gemv(W, xq, xd, K, resid),
                        isum=orc.block_dots(W, xq, K))

    # activation quant (and silu*mul + quant)
    rng = np.random.default_rng(7)
    x = (2.0 * rng.standard_normal(896)).astype(np.float32)
    x[:32] = 0.0
    u = rng.standard_normal(896).astype(np.float32)
    xq, xd = orc.quant_q8(x)
    sq, sd = orc.silu_mul_quant(x, u)
    np.savez_compressed(OUT / "quant_q8_896.npz", x=x, u=u, xq=xq, xd=xd, silu_xq=sq, silu_xd=sd)

    # RMSNorm
    rng = np.random.default_rng(7)
    x = (2.0 * rng.standard_normal(896)).astype(np.float32)
    w = (0.5 * rng.standard_normal(896) + 1.0).astype(np.float32)
    np.savez_compressed(OUT / "rmsnorm_896.npz", x=x, w=w, eps=np.float32(1e-6),
                        y=orc.rmsnorm(x, w, 1e-6))

    # RoPE
    rng = np.random.default_rng(4)
    x = rng.standard_normal(16 * 64).astype(np.float32)
    pos = np.array([0, 1, 31, 159, 1023], np.int32)
    ys = np.stack([orc.rope(x, int(p), 16, 64, 1e6) for p in pos])
    np.savez_compressed(OUT / "rope_hd64.npz", x=x, pos=pos, theta=np.float32(1e6),
                        freqs=orc.rope_freqs(64, 1e6), y=ys)

    # attention: nh 4, nkv 2, hd 32, L 20 of maxt 24
    rng = np.random.default_rng(6)
    nh, nkv, hd, L, maxt = 4, 2, 32, 20, 24
    qv = rng.standard_normal(nh * hd).astype(np.float32)
    kc = rng.standard_normal((maxt, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((maxt, nkv * hd)).astype(np.float32)
    kh, vh = kc.astype(np.float16).view(np.uint16), vc.astype(np.float16).view(np.uint16)
    scale = np.float32(hd ** -0.5)
    np.savez_compressed(OUT / "attn_small.npz", q=qv, kc=kc, vc=vc, kc16=kh, vc16=vh,
                        L=np.int32(L), scale=scale,
                        out_f32_s1=orc.attn_decode(qv, kc, vc, L, nh, nkv, hd, scale, False, 1),
                        out_f32_s3=orc.attn_decode(qv, kc, vc, L, nh, nkv, hd, scale, False, 3),
                        out_f16_s1=orc.attn_decode(qv, kh, vh, L, nh, nkv, hd, scale, True, 1),
                        out_f16_s3=orc.attn_decode(qv, kh, vh, L, nh, nkv, hd, scale, True, 3))

    # whole-model greedy decode on the TINY config (weights regenerated from the seed;
    # their digest is stored so a generator change is detected)
    cfg = M.TINY
    wts = M.synth_weights(cfg, seed=99)
    prompt = np.array(M.random_prompt(cfg, 6, seed=5), np.int32)
    om = orc.OracleModel(cfg, wts)
    toks, margins = om.generate(prompt.tolist(), 16)
    final = om.step(toks[-1])
    om16 = orc.OracleModel(cfg, wts, kv_f16=True, attn_nsplit=4)
    toks16, _ = om16.generate(prompt.tolist(), 16)
    np.savez_compressed(OUT / "decode_tiny.npz", prompt=prompt, tokens=np.array(toks, np.int32),
                        margins=margins, final_logits=final,
                        tokens_f16_split4=np.array(toks16, np.int32),
                        weights_sha256=np.array(weights_digest(wts)))
    for p in sorted(OUT.glob("*.npz")):
        print(f"{p.name}: {p.stat().st_size} bytes")


if __name__ == "__main__":
    main()

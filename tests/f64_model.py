"""A float64 numpy restatement of one decode step of a Qwen2 / Llama model, written from the
model equations, not from the oracle's C code.  It is the independent check of the oracle's
step composition (oracle/lt_oracle.c or_decode_step / or_generate).

Equations (the reference's own torch model, bpd/llamatov_run.py:513-550 rms_norm / apply_rope
and :845-857 qwen2_layer; the engine's device chain bpd/lib/dev_residency.py:1328-1593):

    x      = dequant(token_embd[tok])
    per layer:
      h    = attn_norm * x / sqrt(mean(x^2) + eps)
      qkv  = Wqkv . Q8(h) + bqkv                         (bias before RoPE)
      q, k = rope(q, pos), rope(k, pos)                  (NeoX half split, pos = cache length)
      K[pos], V[pos] = k, v                              (fp16 rounding when the cache is fp16)
      a_h  = softmax(scale * K[:pos+1] . q_h) . V[:pos+1]  (kv head h // (nh / nkv))
      xres = x + Wo . Q8(a)
      h2   = ffn_norm * xres / sqrt(mean(xres^2) + eps)
      g, u = Wgate . Q8(h2), Wup . Q8(h2)
      x    = xres + Wdown . Q8(silu(g) * u)
    logits = Wout . Q8(output_norm * x / sqrt(mean(x^2) + eps))   (Wout = token_embd when tied)

Q8 is the engine's activation quantizer (d = fp16(amax/127), 1 if amax = 0; q = clip(rint(x/d),
+-127)), evaluated in float64 here; weights are the dequantized Q8_0 blocks (exact).  Every
other operation is float64, so the difference from the oracle is float32 rounding plus the
rare quantization code that flips at a rounding boundary.

`mistake` plants one plausible wiring error (for the tests that show the comparison's
tolerance would catch it): "bias_after_rope", "rope_pos_plus1", "gate_up_swapped",
"no_attn_residual", "attend_without_new", "head_from_embd" (untied models only).
"""
from __future__ import annotations

import numpy as np


def dequant(B: np.ndarray, K: int) -> np.ndarray:
    nb = K // 32
    blk = np.asarray(B, np.uint8).reshape(-1, nb, 34)
    d = blk[..., 0:2].copy().view(np.float16).astype(np.float64)
    q = blk[..., 2:].view(np.int8).astype(np.float64)
    return (q * d).reshape(-1, K)


def q8_f64(x: np.ndarray, tol: float | None = None) -> tuple[np.ndarray, bool]:
    """Quantize -> dequantize an activation with the engine's Q8_0 rule, in float64.

    With tol, also report whether every rounding decision is robust: whether moving any
    element by tol * max|x| (the size of a float32 evaluation's error) could change a block
    scale's fp16 rounding or an element's integer code.  A float32 implementation of the
    same arithmetic must make the same decisions wherever this holds."""
    b = np.asarray(x, np.float64).reshape(-1, 32)
    amax = np.abs(b).max(axis=1)
    r = np.where(amax > 0, amax / 127.0, 1.0)
    d = r.astype(np.float16).astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = np.where(d[:, None] > 0, b / d[:, None], 0.0)
    q = np.clip(np.rint(t), -127, 127)
    robust = True
    if tol is not None:
        e = tol * float(np.abs(b).max()) + 1e-300
        nz = amax > 0
        # a zero block stays zero (its elements are exact zeros); a non-zero block must keep
        # its fp16 scale under +-e on amax, and every code under +-e on its element
        scale_ok = np.all(((amax[nz] - e) / 127.0).astype(np.float16) == ((amax[nz] + e) / 127.0).astype(np.float16))
        scale_ok = scale_ok and np.all(amax[nz] > e)
        et = e / d[:, None]
        code_ok = np.all(np.rint(t - et) == np.rint(t + et))
        robust = bool(scale_ok and code_ok)
    return (q * d[:, None]).reshape(-1), robust


def rms(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.asarray(x, np.float64)
    return np.asarray(w, np.float64) * (x / np.sqrt(np.mean(x * x) + eps))


def rope(x: np.ndarray, pos: int, nheads: int, hd: int, theta: float) -> np.ndarray:
    half = hd // 2
    freq = 1.0 / (theta ** (np.arange(0, hd, 2, dtype=np.float64) / hd))
    ang = pos * freq
    c, s = np.cos(ang), np.sin(ang)
    y = np.asarray(x, np.float64).reshape(nheads, hd)
    x1, x2 = y[:, :half], y[:, half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=1).reshape(-1)


class F64Model:
    """Greedy decoding state of the float64 restatement (a growing KV cache per layer)."""

    def __init__(self, cfg, weights: dict, kv_f16: bool = False, mistake: str | None = None,
                 tol: float = 1e-6):
        self.cfg, self.kv_f16, self.mistake, self.tol = cfg, kv_f16, mistake, tol
        self.robust = True     # every rounding decision of the last step was robust (q8_f64)
        E, F = cfg.n_embd, cfg.n_ff
        self.emb = weights["token_embd.weight"]
        head = weights["token_embd.weight"] if cfg.tied or mistake == "head_from_embd" else weights["output.weight"]
        self.head = dequant(head, E)
        self.out_norm = weights["output_norm.weight"]
        self.layers = []
        for il in range(cfg.n_layers):
            p = f"blk.{il}"
            L = {
                "an": weights[f"{p}.attn_norm.weight"],
                "wq": dequant(weights[f"{p}.attn_q.weight"], E),
                "wk": dequant(weights[f"{p}.attn_k.weight"], E),
                "wv": dequant(weights[f"{p}.attn_v.weight"], E),
                "wo": dequant(weights[f"{p}.attn_output.weight"], cfg.q_dim),
                "fn": weights[f"{p}.ffn_norm.weight"],
                "wg": dequant(weights[f"{p}.ffn_gate.weight"], E),
                "wu": dequant(weights[f"{p}.ffn_up.weight"], E),
                "wd": dequant(weights[f"{p}.ffn_down.weight"], F),
            }
            for n in ("q", "k", "v"):
                b = weights.get(f"{p}.attn_{n}.bias")
                L["b" + n] = np.zeros(L["w" + n].shape[0]) if b is None else np.asarray(b, np.float64)
            self.layers.append(L)
        self.K = [[] for _ in range(cfg.n_layers)]
        self.V = [[] for _ in range(cfg.n_layers)]

    def _q8(self, x: np.ndarray) -> np.ndarray:
        y, ok = q8_f64(x, self.tol)
        self.robust &= ok
        return y

    def _store(self, v: np.ndarray) -> np.ndarray:
        if not self.kv_f16:
            return v
        e = self.tol * float(np.abs(v).max())
        self.robust &= bool(np.all((v - e).astype(np.float16) == (v + e).astype(np.float16)))
        return v.astype(np.float16).astype(np.float64)

    def step(self, tok: int) -> np.ndarray:
        cfg, mk = self.cfg, self.mistake
        nh, nkv, hd, E = cfg.n_head, cfg.n_head_kv, cfg.head_dim, cfg.n_embd
        pos = len(self.K[0])
        self.robust = True
        x = dequant(self.emb[tok:tok + 1], E)[0]
        for il, L in enumerate(self.layers):
            hq = self._q8(rms(x, L["an"], cfg.norm_eps))
            q, k, v = L["wq"] @ hq, L["wk"] @ hq, L["wv"] @ hq
            rpos = pos + 1 if mk == "rope_pos_plus1" else pos
            if mk == "bias_after_rope":
                q, k = rope(q, rpos, nh, hd, cfg.rope_theta), rope(k, rpos, nkv, hd, cfg.rope_theta)
                q, k, v = q + L["bq"], k + L["bk"], v + L["bv"]
            else:
                q, k, v = q + L["bq"], k + L["bk"], v + L["bv"]
                q, k = rope(q, rpos, nh, hd, cfg.rope_theta), rope(k, rpos, nkv, hd, cfg.rope_theta)
            self.K[il].append(self._store(k))
            self.V[il].append(self._store(v))
            Kc = np.stack(self.K[il]).reshape(-1, nkv, hd)
            Vc = np.stack(self.V[il]).reshape(-1, nkv, hd)
            if mk == "attend_without_new" and len(Kc) > 1:
                Kc, Vc = Kc[:-1], Vc[:-1]
            att = np.empty(nh * hd)
            for h in range(nh):
                g = h // (nh // nkv)
                s = Kc[:, g] @ q[h * hd:(h + 1) * hd] * hd ** -0.5
                p = np.exp(s - s.max())
                att[h * hd:(h + 1) * hd] = (p / p.sum()) @ Vc[:, g]
            o = L["wo"] @ self._q8(att)
            xres = o if mk == "no_attn_residual" else x + o
            h2 = self._q8(rms(xres, L["fn"], cfg.norm_eps))
            gate, up = L["wg"] @ h2, L["wu"] @ h2
            if mk == "gate_up_swapped":
                gate, up = up, gate
            act = gate / (1.0 + np.exp(-gate)) * up
            x = xres + L["wd"] @ self._q8(act)
        return self.head @ self._q8(rms(x, self.out_norm, cfg.norm_eps))

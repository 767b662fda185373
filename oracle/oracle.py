"""ctypes wrapper of liblt_oracle.so, the CPU restatement of the reference arithmetic.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the llamatov_amd package.
"""
from __future__ import annotations

import ctypes
import subprocess
from ctypes import POINTER, c_float, c_int, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liblt_oracle.so"
_lib = None


REF_SRC = Path("/root/reference/bpd-substrate/bench/bpd_cpu.c")


def build() -> Path:
    """The oracle, and -- where the reference tree is present (not on the GPU box) -- the
    reference's own CPU substrate into _ref/ (`make ref`), the checker of the ggml numerics."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    if REF_SRC.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True, stdout=subprocess.DEVNULL,
                       stderr=subprocess.DEVNULL)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        P = c_void_p
        sigs = {
            "or_set_threads": (None, [c_int]),
            "or_max_threads": (c_int, []),
            "or_half_to_float": (c_float, [ctypes.c_uint16]),
            "or_float_to_half": (ctypes.c_uint16, [c_float]),
            "or_expf": (c_float, [c_float]),
            "or_expf_sel_mismatches": (ctypes.c_uint64, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64]),
            "or_sincosf": (None, [c_float, P, P]),
            "or_rsqrtf": (c_float, [c_float]),
            "or_dequant_rows": (None, [P, c_int, c_int, P]),
            "or_quantize_rows": (None, [P, c_int, c_int, P]),
            "or_quant_q8": (None, [P, c_int, P, P]),
            "or_silu_mul_quant": (None, [P, P, c_int, P, P]),
            "or_silu_mul": (None, [P, P, c_int, P]),
            "or_q8_block_dots": (None, [P, P, c_int, c_int, P]),
            "or_q8_gemv": (None, [P, P, P, P, P, c_int, c_int]),
            "or_quant_q8_ggml": (None, [P, c_int, P, P]),
            "or_philox4x32_10": (None, [P, P, P]),
            "or_sample": (c_int, [P, c_int, c_float, c_int, c_float, ctypes.c_uint64, ctypes.c_uint64]),
            "or_quant_q8_0_ggml_blocks": (None, [P, c_int, P]),
            "or_q8_gemv_ggml": (None, [P, P, P, P, P, c_int, c_int, c_int]),
            "or_qmatmul_q8_0_ggml": (None, [P, P, P, c_int, c_int, c_int]),
            "or_qmatmul_q8_0_llamafile": (None, [P, P, P, c_int, c_int, c_int]),
            "or_rmsnorm": (None, [P, P, P, c_int, c_float]),
            "or_rope_freqs": (None, [c_int, c_float, P]),
            "or_rope": (None, [P, c_int, c_int, c_int, P]),
            "or_attn_decode": (None, [P, P, P, c_int, P, c_int, c_int, c_int, c_float, c_int, c_int]),
            "or_argmax": (c_int, [P, c_int]),
            "or_embed_row": (None, [P, c_int, c_int, P]),
            "or_state_new": (P, [P]),
            "or_state_free": (None, [P, P]),
            "or_state_len": (c_int, [P]),
            "or_state_kv": (P, [P, c_int, c_int]),
            "or_decode_step": (c_int, [P, P, c_int, P]),
            "or_generate": (c_int, [P, P, P, c_int, c_int, P, P]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray | None) -> c_void_p:
    if a is None:
        return c_void_p(0)
    assert a.flags.c_contiguous
    return a.ctypes.data_as(c_void_p)


def set_threads(n: int) -> None:
    lib().or_set_threads(int(n))


def max_threads() -> int:
    return int(lib().or_max_threads())


# ---- scalar numerics ---------------------------------------------------------------
def expf(x: float) -> float:
    return lib().or_expf(x)


def expf_sel_mismatches(start: int, stride: int, count: int) -> int:
    """Bit patterns start + i*stride (mod 2^32), i < count, where the device's branch-free
    lt_expf_sel differs from lt_expf."""
    return int(lib().or_expf_sel_mismatches(start & 0xFFFFFFFF, stride, count))


def sincosf(x: float) -> tuple[float, float]:
    s, c = c_float(), c_float()
    lib().or_sincosf(x, ctypes.byref(s), ctypes.byref(c))
    return s.value, c.value


def rsqrtf(x: float) -> float:
    return lib().or_rsqrtf(x)


def float_to_half_bits(x: float) -> int:
    return lib().or_float_to_half(x)


def half_to_float(h: int) -> float:
    return lib().or_half_to_float(h)


# ---- ops -------------------------------------------------------------------------
def quantize_rows(W: np.ndarray) -> np.ndarray:
    W = np.ascontiguousarray(W, np.float32)
    N, K = W.shape
    out = np.empty((N, K // 32 * 34), np.uint8)
    lib().or_quantize_rows(_p(W), N, K, _p(out))
    return out


def dequant_rows(B: np.ndarray, K: int) -> np.ndarray:
    B = np.ascontiguousarray(B, np.uint8)
    out = np.empty((B.shape[0], K), np.float32)
    lib().or_dequant_rows(_p(B), B.shape[0], K, _p(out))
    return out


def quant_q8(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    K = x.size
    xq = np.empty(K, np.int8)
    xd = np.empty(K // 32, np.uint16)
    lib().or_quant_q8(_p(x), K, _p(xq), _p(xd))
    return xq, xd


def silu_mul_quant(g: np.ndarray, u: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    g = np.ascontiguousarray(g, np.float32).reshape(-1)
    u = np.ascontiguousarray(u, np.float32).reshape(-1)
    K = g.size
    xq = np.empty(K, np.int8)
    xd = np.empty(K // 32, np.uint16)
    lib().or_silu_mul_quant(_p(g), _p(u), K, _p(xq), _p(xd))
    return xq, xd


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32).reshape(-1)
    u = np.ascontiguousarray(u, np.float32).reshape(-1)
    v = np.empty_like(g)
    lib().or_silu_mul(_p(g), _p(u), g.size, _p(v))
    return v


def block_dots(W: np.ndarray, xq: np.ndarray, K: int) -> np.ndarray:
    W = np.ascontiguousarray(W, np.uint8)
    xq = np.ascontiguousarray(xq, np.int8)
    N = W.shape[0]
    out = np.empty((N, K // 32), np.int32)
    lib().or_q8_block_dots(_p(W), _p(xq), N, K, _p(out))
    return out


def q8_gemv(W: np.ndarray, xq: np.ndarray, xd: np.ndarray, K: int, resid: np.ndarray | None = None) -> np.ndarray:
    W = np.ascontiguousarray(W, np.uint8)
    xq = np.ascontiguousarray(xq, np.int8)
    xd = np.ascontiguousarray(xd, np.uint16)
    N = W.shape[0]
    y = np.empty(N, np.float32)
    r = None if resid is None else np.ascontiguousarray(resid, np.float32)
    lib().or_q8_gemv(_p(W), _p(xq), _p(xd), _p(r), _p(y), N, K)
    return y


# ---- ggml-compatible numerics ----------------------------------------------------------
GGML_VEC, GGML_LLAMAFILE = 0, 1


def quant_q8_ggml(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x, np.float32)
    xq = np.empty(x.size, np.int8)
    xd = np.empty(x.size // 32, np.uint16)
    lib().or_quant_q8_ggml(_p(x), x.size, _p(xq), _p(xd))
    return xq, xd


def quant_q8_0_ggml_blocks(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(x.size // 32 * 34, np.uint8)
    lib().or_quant_q8_0_ggml_blocks(_p(x), x.size, _p(y))
    return y


def q8_gemv_ggml(W: np.ndarray, xq: np.ndarray, xd: np.ndarray, K: int, order: int = GGML_VEC,
                 resid: np.ndarray | None = None) -> np.ndarray:
    W = np.ascontiguousarray(W, np.uint8)
    N = W.size // (K // 32 * 34)
    y = np.empty(N, np.float32)
    r = None if resid is None else np.ascontiguousarray(resid, np.float32)
    lib().or_q8_gemv_ggml(_p(W), _p(np.ascontiguousarray(xq, np.int8)), _p(np.ascontiguousarray(xd, np.uint16)),
                          _p(r), _p(y), N, K, order)
    return y


def qmatmul_q8_0_ggml(W: np.ndarray, X: np.ndarray, N: int, K: int) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32).reshape(-1, K)
    out = np.empty((X.shape[0], N), np.float32)
    lib().or_qmatmul_q8_0_ggml(_p(np.ascontiguousarray(W, np.uint8)), _p(X), _p(out), X.shape[0], N, K)
    return out


def qmatmul_q8_0_llamafile(W: np.ndarray, X: np.ndarray, m_weight: int, K: int) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32).reshape(-1, K)
    out = np.empty((X.shape[0], m_weight), np.float32)
    lib().or_qmatmul_q8_0_llamafile(_p(np.ascontiguousarray(W, np.uint8)), _p(X), _p(out), m_weight,
                                    X.shape[0], K)
    return out


# ---- sampling ------------------------------------------------------------------------------
def philox4x32_10(ctr, key) -> list[int]:
    c = np.ascontiguousarray(np.asarray(ctr, np.uint32))
    k = np.ascontiguousarray(np.asarray(key, np.uint32))
    out = np.zeros(4, np.uint32)
    lib().or_philox4x32_10(_p(c), _p(k), _p(out))
    return [int(v) for v in out]


def sample(logits: np.ndarray, temperature: float, top_k: int, top_p: float, seed: int, counter: int) -> int:
    x = np.ascontiguousarray(logits, np.float32).reshape(-1)
    return int(lib().or_sample(_p(x), x.size, temperature, top_k, top_p, seed, counter))


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    w = np.ascontiguousarray(w, np.float32).reshape(-1)
    y = np.empty_like(x)
    lib().or_rmsnorm(_p(x), _p(w), _p(y), x.size, eps)
    return y


def rope_freqs(hd: int, theta: float) -> np.ndarray:
    f = np.empty(hd // 2, np.float32)
    lib().or_rope_freqs(hd, theta, _p(f))
    return f


def rope(x: np.ndarray, pos: int, nheads: int, hd: int, theta: float) -> np.ndarray:
    y = np.ascontiguousarray(x, np.float32).reshape(-1).copy()
    f = rope_freqs(hd, theta)
    lib().or_rope(_p(y), pos, nheads, hd, _p(f))
    return y


def attn_decode(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, L: int, nh: int, nkv: int, hd: int,
                scale: float, kv_f16: bool, nsplit: int = 1) -> np.ndarray:
    """q [nh*hd] fp32; kc/vc position-major [>=L][nkv*hd] (fp32 or fp16 bits as uint16)."""
    q = np.ascontiguousarray(q, np.float32).reshape(-1)
    kc = np.ascontiguousarray(kc)
    vc = np.ascontiguousarray(vc)
    out = np.empty(nh * hd, np.float32)
    lib().or_attn_decode(_p(q), _p(kc), _p(vc), L, _p(out), nh, nkv, hd, scale, int(kv_f16), nsplit)
    return out


def argmax(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    return lib().or_argmax(_p(x), x.size)


def embed_row(emb: np.ndarray, tok: int, E: int) -> np.ndarray:
    out = np.empty(E, np.float32)
    lib().or_embed_row(_p(np.ascontiguousarray(emb, np.uint8)), tok, E, _p(out))
    return out


# ---- whole model -------------------------------------------------------------------
class _OrModel(ctypes.Structure):
    _fields_ = [
        ("n_layers", c_int), ("n_embd", c_int), ("n_ff", c_int), ("n_head", c_int),
        ("n_head_kv", c_int), ("head_dim", c_int), ("vocab", c_int), ("max_ctx", c_int),
        ("kv_f16", c_int), ("attn_nsplit", c_int), ("eps", c_float), ("theta", c_float),
        ("tok_embd", c_void_p), ("output", c_void_p), ("output_norm", c_void_p),
        ("attn_norm", POINTER(c_void_p)), ("wqkv", POINTER(c_void_p)), ("bqkv", POINTER(c_void_p)),
        ("wo", POINTER(c_void_p)), ("ffn_norm", POINTER(c_void_p)), ("wgu", POINTER(c_void_p)),
        ("wdown", POINTER(c_void_p)), ("numerics", c_int),
    ]


def _layer_tensors(w: dict, il: int) -> dict:
    """Per-layer inputs of or_decode_step from GGUF-named tensors: q|k|v rows (and biases)
    and gate|up rows concatenated, as the reference does at first use
    (bpd/lib/dev_residency.py:1283-1326)."""
    p = f"blk.{il}"
    cat = lambda names: np.concatenate([w[f"{p}.{n}"] for n in names], axis=0)
    has_bias = f"{p}.attn_q.bias" in w
    return {
        "attn_norm": w[f"{p}.attn_norm.weight"],
        "wqkv": cat(["attn_q.weight", "attn_k.weight", "attn_v.weight"]),
        "bqkv": cat(["attn_q.bias", "attn_k.bias", "attn_v.bias"]) if has_bias else None,
        "wo": w[f"{p}.attn_output.weight"],
        "ffn_norm": w[f"{p}.ffn_norm.weight"],
        "wgu": cat(["ffn_gate.weight", "ffn_up.weight"]),
        "wdown": w[f"{p}.ffn_down.weight"],
    }


class OracleModel:
    """The oracle's view of a synthetic model: keeps the numpy arrays alive."""

    def __init__(self, cfg, weights: dict, kv_f16: bool = False, attn_nsplit: int = 1,
                 max_ctx: int | None = None, numerics: str = "engine"):
        self.cfg = cfg
        self.keep = []
        nl = cfg.n_layers

        def arr(a, dt):
            a = np.ascontiguousarray(a, dt)
            self.keep.append(a)
            return a.ctypes.data

        def ptrs(vals):
            A = (c_void_p * nl)(*vals)
            self.keep.append(A)
            return ctypes.cast(A, POINTER(c_void_p))

        layers = [_layer_tensors(weights, il) for il in range(nl)]
        m = _OrModel()
        m.n_layers, m.n_embd, m.n_ff = nl, cfg.n_embd, cfg.n_ff
        m.n_head, m.n_head_kv, m.head_dim, m.vocab = cfg.n_head, cfg.n_head_kv, cfg.head_dim, cfg.vocab
        m.max_ctx = int(max_ctx or cfg.max_ctx)
        m.kv_f16, m.attn_nsplit = int(kv_f16), int(attn_nsplit)
        m.eps, m.theta = cfg.norm_eps, cfg.rope_theta
        m.tok_embd = arr(weights["token_embd.weight"], np.uint8)
        m.output = m.tok_embd if cfg.tied else arr(weights["output.weight"], np.uint8)
        m.output_norm = arr(weights["output_norm.weight"], np.float32)
        m.attn_norm = ptrs([arr(L["attn_norm"], np.float32) for L in layers])
        m.wqkv = ptrs([arr(L["wqkv"], np.uint8) for L in layers])
        if layers[0]["bqkv"] is not None:
            m.bqkv = ptrs([arr(L["bqkv"], np.float32) for L in layers])
        else:
            m.bqkv = ctypes.cast(c_void_p(0), POINTER(c_void_p))
        m.wo = ptrs([arr(L["wo"], np.uint8) for L in layers])
        m.ffn_norm = ptrs([arr(L["ffn_norm"], np.float32) for L in layers])
        m.wgu = ptrs([arr(L["wgu"], np.uint8) for L in layers])
        m.wdown = ptrs([arr(L["wdown"], np.uint8) for L in layers])
        if numerics not in ("engine", "ggml"):
            raise ValueError(f"numerics={numerics!r}")
        m.numerics = int(numerics == "ggml")
        self.m = m
        self.st = lib().or_state_new(ctypes.byref(m))

    def reset(self) -> None:
        lib().or_state_free(ctypes.byref(self.m), self.st)
        self.st = lib().or_state_new(ctypes.byref(self.m))

    def __del__(self):
        try:
            if self.st:
                lib().or_state_free(ctypes.byref(self.m), self.st)
                self.st = None
        except Exception:
            pass

    @property
    def length(self) -> int:
        return lib().or_state_len(self.st)

    def step(self, tok: int) -> np.ndarray:
        logits = np.empty(self.cfg.vocab, np.float32)
        rc = lib().or_decode_step(ctypes.byref(self.m), self.st, int(tok), _p(logits))
        if rc != 0:
            raise RuntimeError("oracle KV cache full")
        return logits

    def generate(self, prompt, n_gen: int) -> tuple[list[int], np.ndarray]:
        p = np.ascontiguousarray(np.asarray(prompt, np.int32))
        out = np.empty(n_gen, np.int32)
        margins = np.empty(n_gen, np.float32)
        rc = lib().or_generate(ctypes.byref(self.m), self.st, _p(p), p.size, n_gen, _p(out), _p(margins))
        if rc != 0:
            raise RuntimeError("oracle KV cache full")
        return [int(t) for t in out], margins

    def kv_rows(self, layer: int, which: str, n: int) -> np.ndarray:
        cfg = self.cfg
        width = cfg.kv_dim
        dt = np.uint16 if self.m.kv_f16 else np.float32
        ptr = lib().or_state_kv(self.st, layer, 1 if which == "v" else 0)
        buf = (ctypes.c_uint8 * (n * width * np.dtype(dt).itemsize)).from_address(ptr)
        return np.frombuffer(buf, dtype=dt).reshape(n, width).copy()

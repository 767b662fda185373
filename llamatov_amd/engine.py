"""The MI355X decode engine: device-resident Q8_0 weights, a fixed-buffer decode plan whose
launches are captured into one HIP graph per token, and the batched prefill, all driving
libllamatov_hip.so through ctypes.

Each piece replaces a part of the reference's bpd/lib/dev_residency.py, with buffers the caller
owns instead of module globals:
  DevTensor (dev_residency.py:387-415); KVCache (DeviceKVCache, :418-541); the op launchers
  rms_norm_into (rms_norm_dev, :746-781), q8_linear_into (q8_linear_dev, :905-985),
  q8_linear_add_residual_into (:988-1045), q8_linear_bias_into (q8_linear_dev_bias,
  :1177-1193), rope_qk_into (rope_dev_qk_fused, :722-741), attn_decode_into
  (attn_decode_from_cache_masked, :2016-2031), argmax_into (argmax_dev, :1074-1110);
  DecodePlan + forward_tokens (forward_pass_resident, :1328-1593); StepGraph (GraphRunner,
  :1626-1818); Profile (PRODUCTION_PROFILE / attest_profile / assert_certified_composition,
  :1209-1281).  llamatov_amd.dev_residency keeps the reference's own signatures on top of it.

Design differences (MI355X-first; results are the same bits):
  * Q8_0 weights are the GGUF 34-byte blocks, uploaded once at load (ResidentModel); the
    reference dequantizes to fp32 on the host and re-quantizes at first use.
  * Every buffer a decode step touches is allocated up front in a DecodePlan, so the
    step is capturable without a slab arena and graph pointers never move.
  * The token id lives on the device: the step gathers its embedding from the Q8_0
    token_embd and the argmax writes the next id back into the same buffer, so greedy
    decoding can replay the graph back to back with no host round trip per token.
"""
from __future__ import annotations

import ctypes
import dataclasses
import math
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import LT_GGML_VEC, LT_KV_F16, LT_KV_F32, LT_MULTI_RESID, LT_MULTI_SILU, LT_MULTI_STORE, LT_SAMPLE_MAX_K, call
from .model import ModelConfig, fused_layer_tensors, interleave_gateup


# ----------------------------------------------------------------------------------
# Device context and tensors
# ----------------------------------------------------------------------------------
class Device:
    """One lt_ctx (one HIP device + one stream).  The reference's fact_dispatch._ctx()."""

    def __init__(self, index: int = 0):
        _lib.load()
        h = ctypes.c_void_p()
        call("lt_init", index, ctypes.byref(h))
        self.handle = h
        self.index = index
        self.capturing = False

    def malloc(self, nbytes: int) -> int:
        p = ctypes.c_void_p()
        call("lt_malloc", self.handle, ctypes.byref(p), max(int(nbytes), 1))
        return int(p.value)

    def free(self, ptr: int) -> None:
        if ptr:
            call("lt_free", self.handle, ctypes.c_void_p(ptr))

    def h2d(self, ptr: int, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        call("lt_memcpy_h2d", self.handle, ctypes.c_void_p(ptr), a.ctypes.data_as(ctypes.c_void_p), a.nbytes)

    def d2h(self, arr: np.ndarray, ptr: int) -> np.ndarray:
        assert arr.flags.c_contiguous
        call("lt_memcpy_d2h", self.handle, arr.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(ptr), arr.nbytes)
        return arr

    def d2d(self, dst: int, src: int, nbytes: int) -> None:
        call("lt_memcpy_d2d", self.handle, ctypes.c_void_p(dst), ctypes.c_void_p(src), int(nbytes))

    def fill(self, ptr: int, value: int, nbytes: int) -> None:
        call("lt_fill_u8", self.handle, ctypes.c_void_p(ptr), value, int(nbytes))

    def sync(self) -> None:
        call("lt_sync", self.handle)


_DEVICE: Device | None = None


def get_device() -> Device:
    global _DEVICE
    if _DEVICE is None:
        _DEVICE = Device(0)
    return _DEVICE


class DevTensor:
    """A device buffer: raw pointer + shape + numpy dtype (reference DevTensor is fp32-only)."""
    __slots__ = ("ptr", "shape", "dtype", "n", "nbytes", "_owns", "dev")

    def __init__(self, ptr: int, shape, dtype=np.float32, owns: bool = True, dev: Device | None = None):
        self.ptr = int(ptr)
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.n = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = self.n * self.dtype.itemsize
        self._owns = owns
        self.dev = dev or get_device()

    @staticmethod
    def empty(shape, dtype=np.float32, dev: Device | None = None) -> "DevTensor":
        dev = dev or get_device()
        n = int(np.prod(shape)) if shape else 1
        return DevTensor(dev.malloc(n * np.dtype(dtype).itemsize), shape, dtype, True, dev)

    @staticmethod
    def zeros(shape, dtype=np.float32, dev: Device | None = None) -> "DevTensor":
        t = DevTensor.empty(shape, dtype, dev)
        t.dev.fill(t.ptr, 0, t.nbytes)
        return t

    @staticmethod
    def from_host(arr: np.ndarray, dev: Device | None = None) -> "DevTensor":
        a = np.ascontiguousarray(arr)
        t = DevTensor.empty(a.shape, a.dtype, dev)
        t.dev.h2d(t.ptr, a)
        return t

    def view(self, offset_elems: int, shape, dtype=None) -> "DevTensor":
        dt = np.dtype(dtype) if dtype is not None else self.dtype
        return DevTensor(self.ptr + offset_elems * self.dtype.itemsize, shape, dt, False, self.dev)

    def to_host(self) -> np.ndarray:
        self.dev.sync()
        out = np.empty(self.shape, self.dtype)
        return self.dev.d2h(out, self.ptr)

    def upload(self, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr, dtype=self.dtype)
        if a.nbytes != self.nbytes:
            raise ValueError(f"upload of {a.nbytes} bytes into a {self.nbytes}-byte tensor")
        self.dev.h2d(self.ptr, a)

    def free(self) -> None:
        if self._owns and self.ptr:
            self.dev.free(self.ptr)
            self.ptr = 0

    @property
    def vp(self) -> ctypes.c_void_p:
        return ctypes.c_void_p(self.ptr)


def _vp(x) -> ctypes.c_void_p:
    """A device pointer as a ctypes argument: None, an int address, a ctypes.c_void_p, a
    DevTensor, or any object whose .ptr is one of those (the reference's tensors)."""
    if x is None:
        return ctypes.c_void_p(0)
    if isinstance(x, ctypes.c_void_p):
        return ctypes.c_void_p(x.value or 0)
    if isinstance(x, DevTensor):
        return x.vp
    p = getattr(x, "ptr", None)
    if p is not None:
        return _vp(p)
    return ctypes.c_void_p(int(x))


# ----------------------------------------------------------------------------------
# Op launchers (thin mirrors of the reference op functions)
# ----------------------------------------------------------------------------------
class Q8Weight:
    """A Q8_0 weight resident on the device as GGUF blocks [N][K/32]: uploads its own copy,
    or wraps a slice of a DeviceArena (t=...)."""
    __slots__ = ("t", "N", "K")

    def __init__(self, blocks: np.ndarray | None, K: int, dev: Device | None = None,
                 t: "DevTensor | None" = None, N: int | None = None):
        if t is not None:
            self.t, self.N, self.K = t, int(N), K
            return
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        N = blocks.shape[0]
        if blocks.shape[1] != K // 32 * 34:
            raise ValueError(f"Q8Weight: {blocks.shape} is not [N, {K // 32 * 34}]")
        self.t = DevTensor.from_host(blocks, dev)
        self.N, self.K = N, K


class DeviceArena:
    """One device allocation holding a model's tensors back to back (256-byte aligned
    slices, 2 MiB-aligned base): a single mapping with large pages, so streaming the
    weights of a decode step never walks more page tables than it has to.  The slices
    are non-owning DevTensor views; free() releases the whole arena."""
    ALIGN = 256
    BASE_ALIGN = 2 << 20

    def __init__(self, dev: Device | None = None):
        self.dev = dev or get_device()
        self.items: list[tuple[np.ndarray, list]] = []
        self.ptr = 0

    def add(self, arr: np.ndarray) -> list:
        """Stage an array; the returned one-element list receives its DevTensor at commit()."""
        slot: list = []
        self.items.append((np.ascontiguousarray(arr), slot))
        return slot

    def commit(self) -> None:
        offs, total = [], 0
        for a, _ in self.items:
            offs.append(total)
            total += (a.nbytes + self.ALIGN - 1) // self.ALIGN * self.ALIGN
        self.ptr = self.dev.malloc(total + self.BASE_ALIGN)
        base = (self.ptr + self.BASE_ALIGN - 1) // self.BASE_ALIGN * self.BASE_ALIGN
        for (a, slot), off in zip(self.items, offs):
            t = DevTensor(base + off, a.shape, a.dtype, owns=False, dev=self.dev)
            self.dev.h2d(t.ptr, a)
            slot.append(t)
        self.nbytes = total
        self.items = []

    def free(self) -> None:
        if self.ptr:
            self.dev.free(self.ptr)
            self.ptr = 0


def quant_q8_into(x: DevTensor, xq: DevTensor, xd: DevTensor, K: int | None = None) -> None:
    K = K or x.n
    call("lt_quant_q8", x.dev.handle, x.vp, xq.vp, xd.vp, K)


def rms_norm_into(x: DevTensor, w: DevTensor, eps: float, out: DevTensor) -> DevTensor:
    """k_rmsnorm block_row into `out` (reference rms_norm_dev_into, dev_residency.py:1130)."""
    N = x.shape[-1]
    M = x.n // N
    call("lt_rmsnorm", x.dev.handle, x.vp, w.vp, out.vp, M, N, ctypes.c_float(eps))
    return out


def q8_gemv_into(W: Q8Weight, xq: DevTensor, xd: DevTensor, out: DevTensor,
                resid: DevTensor | None = None) -> DevTensor:
    call("lt_q8_gemv", out.dev.handle, W.t.vp, xq.vp, xd.vp, _vp(resid), out.vp, W.N, W.K)
    return out


def q8_linear_into(x: DevTensor, W: Q8Weight, out: DevTensor, xq: DevTensor, xd: DevTensor) -> DevTensor:
    """quant + GEMV into `out` (reference q8_linear_dev_into, dev_residency.py:1139-1172)."""
    quant_q8_into(x, xq, xd, W.K)
    return q8_gemv_into(W, xq, xd, out)


def q8_linear_add_residual_into(x: DevTensor, W: Q8Weight, resid: DevTensor, out: DevTensor,
                               xq: DevTensor, xd: DevTensor, silu_src=None) -> DevTensor:
    """quant (or SiLU*mul+quant when silu_src=(g, u)) + GEMV with the residual added at the
    store (reference q8_linear_add_residual_dev, dev_residency.py:988-1045)."""
    if silu_src is not None:
        g, u = silu_src
        call("lt_silu_mul_quant", out.dev.handle, g.vp, u.vp, xq.vp, xd.vp, W.K)
    else:
        quant_q8_into(x, xq, xd, W.K)
    return q8_gemv_into(W, xq, xd, out, resid)


def q8_linear_bias_into(x: DevTensor, W: Q8Weight, bias: DevTensor | None, out: DevTensor,
                       xq: DevTensor, xd: DevTensor) -> DevTensor:
    """Bias folded into the GEMV store (reference q8_linear_dev_bias, :1177-1193)."""
    if bias is None:
        return q8_linear_into(x, W, out, xq, xd)
    return q8_linear_add_residual_into(x, W, bias, out, xq, xd)


def rope_qk_into(qk: DevTensor, pos_ptr: int, nh: int, nkv: int, hd: int, freqs: DevTensor) -> None:
    call("lt_rope_qk", qk.dev.handle, qk.vp, _vp(pos_ptr), nh + nkv, hd, freqs.vp)


def attn_decode_into(q: DevTensor, cache: "KVCache", nh: int, scale: float,
                                  len_ptr: int, out: DevTensor, nsplit: int = 1,
                                  ws: DevTensor | None = None) -> DevTensor:
    call("lt_attn_decode", q.dev.handle, q.vp, cache.k.vp, cache.v.vp, _vp(len_ptr), out.vp, 1, nh,
         cache.nkv, cache.hd, ctypes.c_float(scale), cache.max_seq, nsplit, cache.kv_dtype,
         _vp(ws), ws.nbytes if ws is not None else 0)
    return out


def argmax_into(logits: DevTensor, n: int, out_ptr: int, ws: DevTensor) -> int:
    if n <= 0:
        raise ValueError(f"argmax_into: n={n} (must be > 0)")
    call("lt_argmax", logits.dev.handle, logits.vp, n, _vp(out_ptr), ws.vp, ws.nbytes)
    return out_ptr


def rope_freqs(hd: int, theta: float) -> np.ndarray:
    f = np.empty(hd // 2, dtype=np.float32)
    call("lt_rope_freqs", hd, ctypes.c_float(theta), f.ctypes.data_as(ctypes.c_void_p))
    return f


# ----------------------------------------------------------------------------------
# KV cache
# ----------------------------------------------------------------------------------
class KVCache:
    """Device KV cache for one layer: position-major [max_seq][nkv*hd] K and V and a device
    int length (reference DeviceKVCache, bpd/lib/dev_residency.py:418-541).  kv_dtype
    LT_KV_F32 (the reference's elem_bytes=4) or LT_KV_F16."""

    def __init__(self, max_seq: int, nkv: int, hd: int, kv_dtype: int = LT_KV_F32,
                 len_ptr: int | None = None, dev: Device | None = None):
        self.dev = dev or get_device()
        self.max_seq, self.nkv, self.hd = int(max_seq), int(nkv), int(hd)
        self.width = self.nkv * self.hd
        self.kv_dtype = kv_dtype
        self.elem_bytes = 2 if kv_dtype == LT_KV_F16 else 4
        dt = np.uint16 if kv_dtype == LT_KV_F16 else np.float32
        self.k = DevTensor.empty((self.max_seq, self.width), dt, self.dev)
        self.v = DevTensor.empty((self.max_seq, self.width), dt, self.dev)
        self._len_owned = len_ptr is None
        self.len_ptr = self.dev.malloc(4) if len_ptr is None else int(len_ptr)
        self.length = 0
        self.set_length(0)

    def set_length(self, n: int) -> None:
        self.length = int(n)
        self.dev.h2d(self.len_ptr, np.array([n], dtype=np.int32))

    def device_length(self) -> int:
        out = np.zeros(1, np.int32)
        self.dev.sync()
        self.dev.d2h(out, self.len_ptr)
        return int(out[0])

    # -- the reference DeviceKVCache interface (bpd/lib/dev_residency.py:418-541) --------
    @property
    def k_ptr(self) -> ctypes.c_void_p:
        return self.k.vp

    @property
    def v_ptr(self) -> ctypes.c_void_p:
        return self.v.vp

    def _ensure_len_ptr(self, seed: bool = True) -> ctypes.c_void_p:
        """The device length; seed=True writes the host mirror into it first (eager use,
        never under capture)."""
        if seed:
            self.set_length(self.length)
        return ctypes.c_void_p(self.len_ptr)

    def incr_len_dev(self) -> None:
        """*len += 1 on the device (capturable); the host mirror is the caller's."""
        call("lt_len_add", self.dev.handle, _vp(self.len_ptr), 1, self.max_seq)

    def append(self, k, v, count: int = 1) -> None:
        """Copy `count` rows of K and V (device pointers, fp32 rows of width elements) into
        the cache at the host length, then advance the host length (device len unchanged)."""
        if self.kv_dtype != LT_KV_F32:
            raise ValueError("KVCache.append copies raw rows into an fp32 cache; an fp16 cache "
                             "takes rows through append_at_len / append_at_len_incr")
        if self.length + count > self.max_seq:
            raise ValueError(f"KV cache full: {self.length} + {count} > {self.max_seq}")
        n = count * self.width * 4
        off = self.length * self.width * 4
        self.dev.d2d(self.k.ptr + off, _vp(k).value, n)
        self.dev.d2d(self.v.ptr + off, _vp(v).value, n)
        self.length += count

    def append_at_len(self, k, v) -> None:
        """Write one K and V row at the device length *len, leaving *len unchanged
        (capturable; fp16 caches round to nearest even)."""
        if getattr(self, "_stage", None) is None:
            self._stage = DevTensor.empty((2 * self.width,), np.float32, self.dev)
        st = self._stage
        self.dev.d2d(st.ptr, _vp(k).value, self.width * 4)
        self.dev.d2d(st.ptr + self.width * 4, _vp(v).value, self.width * 4)
        call("lt_kv_append_batch", self.dev.handle, self.k.vp, self.v.vp, st.vp, 0, 0, self.width, 1,
             _vp(self.len_ptr), self.width, self.max_seq, self.kv_dtype)

    def append_at_len_incr(self, k, v) -> bool:
        """Write one K and V row at *len and advance *len, in one launch; True (the
        increment is folded, as the reference's fused path reports)."""
        call("lt_kv_append_incr", self.dev.handle, self.k.vp, _vp(k), self.v.vp, _vp(v),
             _vp(self.len_ptr), self.width, self.max_seq, self.kv_dtype)
        return True

    def _slice_host(self, which: str) -> np.ndarray:
        rows = self.rows_host(which, self.length)
        if self.kv_dtype == LT_KV_F16:
            rows = rows.view(np.float16).astype(np.float32)
        return np.ascontiguousarray(rows, np.float32).reshape(self.length, self.nkv, self.hd)

    def k_slice_host(self) -> np.ndarray:
        """The valid K rows [length, nkv, hd] as fp32 on the host."""
        return self._slice_host("k")

    def v_slice_host(self) -> np.ndarray:
        return self._slice_host("v")

    def rows_host(self, which: str, n: int | None = None) -> np.ndarray:
        n = self.length if n is None else n
        t = self.k if which == "k" else self.v
        out = np.empty((self.max_seq, self.width), t.dtype)
        self.dev.sync()
        self.dev.d2h(out, t.ptr)
        return out[:n]

    def free(self) -> None:
        self.k.free()
        self.v.free()
        if getattr(self, "_stage", None) is not None:
            self._stage.free()
            self._stage = None
        if self._len_owned:
            self.dev.free(self.len_ptr)


# ----------------------------------------------------------------------------------
# Production profile (a frozen config object instead of the reference's env flags)
# ----------------------------------------------------------------------------------
@dataclass(frozen=True)
class Profile:
    """The certified ensemble.  Every variant below is bit-identical to the reference's
    per-op chain; the fields select kernels, not numerics, except attn_nsplit (> 1 selects
    the split-K declared order) and kv_dtype."""
    kv_dtype: int = LT_KV_F32
    attn_nsplit: int = 1
    fused_step: bool = True         # five fused launches per layer (lt_fused.hip)
    # fused step: True = the gate|up GEMV writes fp32 SiLU(g)*u and the down GEMV quantizes it
    # in its prologue (lt_q8_gemv_rms_swiglu + lt_q8_gemv_quant), so gate|up takes any row
    # mapping; False = gate|up quantizes in its epilogue, 64 staged rows per workgroup
    # (lt_q8_gemv_rms_silu).  Same bits; False is faster at C2 (gate|up 6.0 vs 7.6 us, down
    # 5.1 vs 6.1 us: more workgroups repeat the RMSNorm prologue, whose latency bounds them)
    swiglu_fp32: bool = False
    # fused step, nsplit 1: four launches per layer while the fused attention kernel applies
    # (head dim 64, at most lt_attn_o_max_len attended rows): QKV + RoPE + KV append
    # (lt_q8_gemv_rms_rope_kv), attention recomputed in the O GEMV's prologue
    # (lt_q8_gemv_attn_o), gate|up + the length bump, down; past that length, and otherwise,
    # the five launches (same bits).  Off by default: recomputing all heads' attention on
    # each workgroup's CU measured slower at C2 than the separate attention launch, which
    # spreads the heads over 14 CUs
    attn_in_o: bool = False
    # fused step, nsplit 1, engine numerics: the whole step (every layer) in one persistent
    # launch (lt_decode_step: workgroups exchange each phase's outputs through step-tagged
    # words, no kernel boundaries between layers) while the geometry allows it (head dim 64,
    # n_embd <= 1024, n_ff <= 5120) and the cache holds at most lt_decode_step_max_len rows;
    # otherwise the five launches (same bits)
    persistent_step: bool = True
    # fused step: the five launches stream planar copies of their matrices (lt_q8_to_planar,
    # *_pl GEMVs: whole aligned cache lines per load) when every K is a multiple of 1024
    # (the 8B geometry; same bits)
    planar: bool = True
    fused_rms_quant: bool = False   # per-op path only: k_rms_quant instead of k_rmsnorm + k_quant_q8
    graph: bool = True
    # "engine": the reference engine's quantizer and canonical GEMV order (every field above);
    # "ggml": ggml's dispatched quantizer (id = 127/amax, ties to even) and its vec_dot order
    # for every GEMV of the step (lt_ggml.hip), so that logits compare with llama.cpp on an
    # AVX1 host; per-op launches only (fused_step=False), prefill token by token
    numerics: str = "engine"


PRODUCTION_PROFILE = Profile()
GGML_PROFILE = Profile(fused_step=False, numerics="ggml")
_CERTIFIED_NSPLIT = {1, 2, 4, 8, 16, 32, 64, 128}


def attn_nsplit_for(batch: int, length: int, n_kv_heads: int, num_cus: int = 256) -> int:
    """A split count for decode attention over `length` cached positions (the reference fixes
    it per capture, ir_param_axes.pl:303-341): a power of two in 1 .. 128 with at least 64
    and at most 512 positions per split, and enough workgroups to fill the CUs --
      batch 1: two per CU of the small-grid kernel, whose workgroups hold one wave per query
        head of a KV group (4 waves at C4);
      batch > 1: eight single-wave workgroups per CU (one per split, KV group and sequence).
    Measured at C4 (32 q / 8 KV heads, hd 128, fp16; attention + merge, median of 5 runs):
    batch 1 at 4k / 16k / 32k takes 9.6-9.7 / 18.4-18.9 / 29.8-30.3 us at 64 splits against
    9.9-10.3 / 23.6-24.2 / 43.8 at 32 and 13.1 / 19.5-20.1 / 30.7-31.7 at 128;
    batch 8 picks 32 / 32 / 64 (61% / 63% / 61% of 8 TB/s)."""
    per_cu = 2 if batch == 1 else 8
    want = max((per_cu * num_cus + batch * n_kv_heads - 1) // (batch * n_kv_heads), (length + 511) // 512)
    cap = min(128, max(1, length // 64))
    n = 1
    while n * 2 <= cap and n < want:
        n *= 2
    return n


def attest_profile(p: Profile) -> dict:
    return dataclasses.asdict(p)


def assert_certified_composition(p: Profile) -> None:
    """Refuse uncertified ensembles (reference dev_residency.py:1268-1281)."""
    if p.kv_dtype not in (LT_KV_F32, LT_KV_F16):
        raise RuntimeError(f"uncertified kv_dtype {p.kv_dtype}")
    if p.attn_nsplit not in _CERTIFIED_NSPLIT:
        raise RuntimeError(f"uncertified attn_nsplit {p.attn_nsplit}")
    if p.numerics not in ("engine", "ggml"):
        raise RuntimeError(f"uncertified numerics {p.numerics!r}")
    if p.numerics == "ggml" and (p.fused_step or p.fused_rms_quant):
        raise RuntimeError("the ggml numerics profile runs the per-op step: fused_step=False, "
                           "fused_rms_quant=False")


# ----------------------------------------------------------------------------------
# Resident model and the fixed-buffer decode plan
# ----------------------------------------------------------------------------------
class ResidentModel:
    """All weights on the device, uploaded once: Q8_0 blocks verbatim, q|k|v and gate|up
    concatenated at load (the reference concatenates at first use, dev_residency.py:1283-1326),
    tied lm_head sharing token_embd's blocks.

    layouts selects the gate|up layouts uploaded: "fused" (rows interleaved gate j, up j, for
    lt_q8_gemv_rms_silu), "per_op" (gate rows then up rows, the reference's concatenation,
    for lt_q8_gemv + lt_silu_mul_quant) or "both"."""

    def __init__(self, cfg: ModelConfig, weights: dict, dev: Device | None = None, layouts: str = "both"):
        if layouts not in ("fused", "per_op", "both"):
            raise ValueError(f"layouts={layouts!r}")
        self.cfg = cfg
        self.dev = dev or get_device()
        self.layouts = layouts
        E, F = cfg.n_embd, cfg.n_ff
        arena = DeviceArena(self.dev)
        staged = []   # (kind, owner dict, key, slot, N, K)

        def q8(owner, key, blocks, K):
            staged.append(("q8", owner, key, arena.add(blocks), blocks.shape[0], K))

        def vec(owner, key, arr):
            if arr is None:
                owner[key] = None
                return
            staged.append(("vec", owner, key, arena.add(np.asarray(arr, np.float32)), 0, 0))

        top: dict = {}
        q8(top, "tok_embd", weights["token_embd.weight"], E)
        if not cfg.tied:
            q8(top, "output", weights["output.weight"], E)
        vec(top, "output_norm", weights["output_norm.weight"])
        vec(top, "freqs", rope_freqs(cfg.head_dim, cfg.rope_theta))
        self.layers = []
        for il in range(cfg.n_layers):
            t = fused_layer_tensors(cfg, weights, il)
            L: dict = {}
            vec(L, "attn_norm", t["attn_norm"])
            q8(L, "wqkv", t["wqkv"], E)
            vec(L, "bqkv", t["bqkv"])
            q8(L, "wo", t["wo"], cfg.q_dim)
            vec(L, "ffn_norm", t["ffn_norm"])
            q8(L, "wdown", t["wdown"], F)
            if layouts in ("per_op", "both"):
                q8(L, "wgu", t["wgu"], E)
            if layouts in ("fused", "both"):
                p = f"blk.{il}"
                q8(L, "wgu_il", interleave_gateup(weights[f"{p}.ffn_gate.weight"],
                                                  weights[f"{p}.ffn_up.weight"]), E)
            self.layers.append(L)
        arena.commit()
        for kind, owner, key, slot, N, K in staged:
            owner[key] = Q8Weight(None, K, t=slot[0], N=N) if kind == "q8" else slot[0]
        self.arena = arena
        self.load_report = None
        self.tiles = None   # the prefill GEMM's tile-major copies (prefill_tiles)
        self.output_t: Q8Weight | None = None   # the lm_head's tile-major copy (head_tiles)
        self.planar = None  # the planar copies of the decode GEMVs' matrices (planar_copies)
        self.output_pl: Q8Weight | None = None
        self._head_pl: DevTensor | None = None   # head_planar's own allocation
        self.qkv_rope = None  # the q|k|v matrices' rope-pair tile copies (qkv_rope_tiles)
        self.tok_embd = top["tok_embd"]
        self.output = top.get("output", self.tok_embd)
        self.output_norm = top["output_norm"]
        self.freqs = top["freqs"]

    @classmethod
    def from_gguf(cls, path, dev: Device | None = None, layouts: str = "both",
                  max_ctx: int = 1024) -> "ResidentModel":
        """Upload a Q8_0 GGUF file (the reference's load_model + first-use residency,
        decode_fact.py:39-51, fact_dispatch.py:255-299): Q8_0 blocks go from the mapped file
        to the device without a float32 copy.  `load_report` says how many tensors were used
        verbatim, canonicalized or quantized from another type."""
        from . import gguf
        cfg, w, reader, report = gguf.load_q8_model(path, max_ctx=max_ctx)
        try:
            m = cls(cfg, w, dev, layouts)
        finally:
            del w
            reader.close()
        m.load_report = report
        return m

    def prefill_tiles(self) -> None:
        """Tile-major copies of the prefill GEMM's matrices (q|k|v, o, interleaved gate|up,
        down), built on the device from the resident blocks at the first batched prefill:
        one allocation, lt_q8_tiles per matrix.  The decode path keeps reading the GGUF-layout
        blocks; the copies cost one more copy of those weights in HBM."""
        if self.tiles is not None:
            return
        if "wgu_il" not in self.layers[0]:
            raise ValueError("prefill needs the fused gate|up layout (ResidentModel layouts 'fused' or 'both')")
        nbytes = _lib.raw("lt_q8_tiles_bytes")
        names = ("wqkv", "wo", "wgu_il", "wdown")
        plan = []
        total = 0
        for L in self.layers:
            for k in names:
                W = L[k]
                n = int(nbytes(W.N, W.K))
                plan.append((L, k, W, total, n))
                total += (n + 255) // 256 * 256
        base = self.dev.malloc(total)
        for L, k, W, off, n in plan:
            t = DevTensor(base + off, (n,), np.uint8, owns=False, dev=self.dev)
            call("lt_q8_tiles", self.dev.handle, W.t.vp, t.vp, W.N, W.K)
            L[k + "_t"] = Q8Weight(None, W.K, t=t, N=W.N)
        self.tiles = base

    def qkv_rope_tiles(self) -> None:
        """Tile-major copies of every layer's q|k|v matrix in the rope-pair row order
        (lt_q8_tiles_rope), built on the device at first use: one allocation.  The batched
        step's q|k|v GEMM with the RoPE + KV-append epilogue (lt_q8_gemm_rope_t) reads them."""
        if self.qkv_rope is not None:
            return
        c = self.cfg
        n = int(_lib.raw("lt_q8_tiles_bytes")(c.n_qkv, c.n_embd))
        step = (n + 255) // 256 * 256
        base = self.dev.malloc(step * len(self.layers))
        for il, L in enumerate(self.layers):
            W = L["wqkv"]
            t = DevTensor(base + il * step, (n,), np.uint8, owns=False, dev=self.dev)
            call("lt_q8_tiles_rope", self.dev.handle, W.t.vp, t.vp, W.N, W.K, c.n_head, c.n_head_kv, c.head_dim)
            L["wqkv_rt"] = Q8Weight(None, W.K, t=t, N=W.N)
        self.qkv_rope = base

    def planar_eligible(self) -> bool:
        """Every matrix the five-launch step streams (q|k|v, o, interleaved gate|up, down, the
        lm_head) has K a multiple of 1024, the planar layout's condition."""
        c = self.cfg
        return "wgu_il" in self.layers[0] and all(k % 1024 == 0 for k in (c.n_embd, c.q_dim, c.n_ff))

    def planar_copies(self) -> bool:
        """Planar copies (lt_q8_to_planar) of the step's matrices, built on the device from the
        resident blocks at first use: one allocation, one more copy of those weights in HBM.
        The five-launch step then streams them through the *_pl GEMVs (same bits).  False when
        the geometry is not eligible."""
        if self.planar is not None:
            return True
        if not self.planar_eligible():
            return False
        names = ("wqkv", "wo", "wgu_il", "wdown")
        plan = []
        total = 0
        for L in self.layers:
            for k in names:
                W = L[k]
                plan.append((L, k, W, total))
                total += (W.t.nbytes + 255) // 256 * 256
        plan.append((None, "output", self.output, total))
        total += (self.output.t.nbytes + 255) // 256 * 256
        base = self.dev.malloc(total)
        for L, k, W, off in plan:
            t = DevTensor(base + off, (W.t.nbytes,), np.uint8, owns=False, dev=self.dev)
            call("lt_q8_to_planar", self.dev.handle, W.t.vp, t.vp, W.N, W.K)
            if L is None:
                self.output_pl = Q8Weight(None, W.K, t=t, N=W.N)
            else:
                L[k + "_pl"] = Q8Weight(None, W.K, t=t, N=W.N)
        self.planar = base
        return True

    def head_planar(self) -> Q8Weight | None:
        """Planar copy (lt_q8_to_planar) of the lm_head alone, built on the device at first use:
        the vocab GEMV of a step whose layers stream other layouts (the persistent step, the
        five-launch step of a geometry with K % 1024 != 0) reads it -- same bits, fewer bytes
        per load instruction (C2: 31.5 -> 29.1 us for the RMSNorm + GEMV + argmax launch).  The
        copy planar_copies made when there is one; None when K is not a multiple of 32."""
        if self.output_pl is not None:
            return self.output_pl
        W = self.output
        if W.K % 32 != 0:
            return None
        t = DevTensor.empty((W.t.nbytes,), np.uint8, self.dev)
        call("lt_q8_to_planar", self.dev.handle, W.t.vp, t.vp, W.N, W.K)
        self._head_pl = t
        self.output_pl = Q8Weight(None, W.K, t=t, N=W.N)
        return self.output_pl

    def head_tiles(self) -> Q8Weight:
        """Tile-major copy of the lm_head (the batched decode step's vocab GEMM), built on the
        device at first use."""
        if self.output_t is None:
            W = self.output
            n = int(_lib.raw("lt_q8_tiles_bytes")(W.N, W.K))
            t = DevTensor.empty((n,), np.uint8, self.dev)
            call("lt_q8_tiles", self.dev.handle, W.t.vp, t.vp, W.N, W.K)
            self.output_t = Q8Weight(None, W.K, t=t, N=W.N)
        return self.output_t

    def free(self) -> None:
        if self.tiles is not None:
            self.dev.free(self.tiles)
            self.tiles = None
        if self.planar is not None:
            self.dev.free(self.planar)
            self.planar = None
            self.output_pl = None
            for L in self.layers:
                for k in ("wqkv_pl", "wo_pl", "wgu_il_pl", "wdown_pl"):
                    L.pop(k, None)
        if self.qkv_rope is not None:
            self.dev.free(self.qkv_rope)
            self.qkv_rope = None
            for L in self.layers:
                L.pop("wqkv_rt", None)
        if self._head_pl is not None:
            self._head_pl.free()
            self._head_pl = None
            self.output_pl = None
        if self.output_t is not None:
            self.output_t.t.free()
            self.output_t = None
        self.arena.free()


class _StepLayer(ctypes.Structure):
    """lt_step_layer of include/llamatov_hip.h: one layer's device pointers."""
    _fields_ = [(n, ctypes.c_void_p) for n in ("attn_norm", "wqkv", "bqkv", "wo", "ffn_norm", "wgu", "wdown",
                                                "kc", "vc")]


class DecodePlan:
    """Fixed device buffers and the launch sequence of one decode token."""

    def __init__(self, model: ResidentModel, profile: Profile = PRODUCTION_PROFILE,
                 max_ctx: int | None = None, hist_cap: int = 4096, host_embed: bool = False):
        """host_embed: the step reads its input row from resid_in, written by the host before
        each step (set_embedding), as the reference's replay does with its fp32 host
        embedding (dev_residency.py:1371-1377, 1769-1772); otherwise the step gathers the
        row of the device token from the Q8_0 token_embd."""
        assert_certified_composition(profile)
        self.host_embed = bool(host_embed)
        need = "fused" if profile.fused_step else "per_op"
        if model.layouts not in (need, "both"):
            raise ValueError(f"DecodePlan: profile needs the {need!r} gate|up layout, model has {model.layouts!r}")
        self.model, self.cfg, self.profile = model, model.cfg, profile
        self.dev = model.dev
        cfg = self.cfg
        E, F, hd = cfg.n_embd, cfg.n_ff, cfg.head_dim
        self.max_ctx = int(max_ctx or cfg.max_ctx)
        kmax = max(E, F, cfg.q_dim)
        D = self.dev
        self.tok = DevTensor.empty((1,), np.int32, D)
        self.err = DevTensor.empty((1,), np.int32, D)
        self.hist = DevTensor.empty((hist_cap,), np.int32, D)
        self.hist_count = DevTensor.empty((1,), np.int32, D)
        self.hist_cap = hist_cap
        self.lens = DevTensor.empty((cfg.n_layers,), np.int32, D)
        self.resid_in = DevTensor.empty((E,), np.float32, D)
        self.carry = DevTensor.empty((E,), np.float32, D)
        self.xres = DevTensor.empty((E,), np.float32, D)
        self.h = DevTensor.empty((E,), np.float32, D)
        self.qkv = DevTensor.empty((cfg.n_qkv,), np.float32, D)
        self.att = DevTensor.empty((cfg.q_dim,), np.float32, D)
        self.gu = DevTensor.empty((2 * F,), np.float32, D)
        self.v = DevTensor.empty((F,), np.float32, D)
        self.logits = DevTensor.empty((cfg.vocab,), np.float32, D)
        self.xq = DevTensor.empty((kmax,), np.int8, D)
        self.xd = DevTensor.empty((kmax // 32,), np.uint16, D)
        ws_n = max(_lib.raw("lt_argmax_workspace_size")(), _lib.raw("lt_q8_gemv_argmax_workspace_size")(cfg.vocab))
        self.am_ws = DevTensor.empty((ws_n,), np.uint8, D)
        aw = _lib.raw("lt_attn_workspace_size")(1, cfg.n_head, hd, profile.attn_nsplit)
        self.attn_ws = DevTensor.empty((aw,), np.uint8, D) if aw else None
        self.caches = [KVCache(self.max_ctx, cfg.n_head_kv, hd, profile.kv_dtype,
                                     len_ptr=self.lens.ptr + 4 * il, dev=D)
                       for il in range(cfg.n_layers)]
        self.scale = float(hd ** -0.5)
        # planar copies for the five-launch step (engine numerics, SiLU-quant gate|up)
        self.planar = bool(profile.fused_step and profile.planar and profile.numerics == "engine"
                           and not profile.swiglu_fp32 and model.planar_copies())
        # the vocab GEMV of the fused steps over a planar copy of the lm_head (same bits)
        self.head_pl = (model.head_planar() if profile.fused_step and profile.planar and profile.numerics == "engine"
                        else None)
        self._setup_persistent()
        self._prefill: PrefillBuffers | None = None
        self.sampling = False
        self._sample_params: DevTensor | None = None
        self._sample_ws: DevTensor | None = None
        self.reset()

    def _setup_persistent(self) -> None:
        """The persistent step's workspace (zero-filled: its tags start above every stored
        word) and the device array of per-layer descriptors, when the profile and the
        geometry take it (lt_decode_step_max_len > 0)."""
        self.persistent_len = 0
        self.step_ws: DevTensor | None = None
        self.step_layers: DevTensor | None = None
        p, cfg, m = self.profile, self.cfg, self.model
        if not (p.fused_step and p.persistent_step and p.attn_nsplit == 1 and not p.swiglu_fp32
                and p.numerics == "engine"):
            return
        E, F, hd, nh, nkv = cfg.n_embd, cfg.n_ff, cfg.head_dim, cfg.n_head, cfg.n_head_kv
        n = int(_lib.raw("lt_decode_step_max_len")(self.dev.handle, cfg.n_layers, E, F, nh, nkv, hd, p.kv_dtype,
                                                    self.max_ctx))
        if n <= 0:
            return
        wsb = int(_lib.raw("lt_decode_step_workspace_size")(cfg.n_layers, E, F, nh, nkv, hd))
        self.step_ws = DevTensor.empty((wsb,), np.uint8, self.dev)
        self.dev.fill(self.step_ws.ptr, 0, wsb)
        self.step_layers = self.step_layer_descs()
        self.persistent_len = n

    @property
    def persistent(self) -> bool:
        """The next step (at the current host length) runs as one persistent launch."""
        return self.persistent_len > 0 and self.caches[0].length + 1 <= self.persistent_len

    def error(self) -> int:
        """The step's device error word: 0 = none, 1 = a token outside the vocabulary, 2 = a
        persistent step's exchange wait ran out, 3 = a persistent step past its length."""
        out = np.zeros(1, np.int32)
        self.dev.d2h(out, self.err.ptr)
        return int(out[0])

    def prefill_buffers(self, T: int) -> "PrefillBuffers":
        if self._prefill is None or self._prefill.T < T:
            if self._prefill is not None:
                self.dev.sync()
                self._prefill.free()
            self._prefill = PrefillBuffers(self, max(T, 32))
        return self._prefill

    # -- state --------------------------------------------------------------------
    def reset(self) -> None:
        """Empty caches (length 0), zero token history."""
        self.dev.h2d(self.lens.ptr, np.zeros(self.cfg.n_layers, np.int32))
        for c in self.caches:
            c.length = 0
        self.dev.h2d(self.hist_count.ptr, np.zeros(1, np.int32))
        self.dev.h2d(self.err.ptr, np.zeros(1, np.int32))
        if getattr(self, "step_ws", None) is not None:
            self.dev.h2d(self.step_ws.ptr + 8, np.zeros(1, np.uint32))   # StepState.fail

    def set_token(self, tok: int) -> None:
        self.dev.h2d(self.tok.ptr, np.array([tok], np.int32))

    def set_embedding(self, row: np.ndarray) -> None:
        """The next step's input row (host_embed plans), fp32 [n_embd]."""
        r = np.ascontiguousarray(row, np.float32).reshape(-1)
        if r.size != self.cfg.n_embd:
            raise ValueError(f"embedding row of {r.size} values, expected {self.cfg.n_embd}")
        self.dev.h2d(self.resid_in.ptr, r)

    def read_token(self) -> int:
        out = np.zeros(1, np.int32)
        self.dev.d2h(out, self.tok.ptr)
        return int(out[0])

    def read_logits(self) -> np.ndarray:
        return self.logits.to_host()

    def history_count(self) -> int:
        out = np.zeros(1, np.int32)
        self.dev.d2h(out, self.hist_count.ptr)
        return int(out[0])

    def history(self) -> list[int]:
        n = self.history_count()
        out = np.zeros(self.hist_cap, np.int32)
        self.dev.d2h(out, self.hist.ptr)
        return [int(t) for t in out[:n]]

    def lengths(self) -> np.ndarray:
        out = np.zeros(self.cfg.n_layers, np.int32)
        self.dev.sync()
        return self.dev.d2h(out, self.lens.ptr)

    # -- the step ----------------------------------------------------------------
    def enqueue_step(self, four: bool | None = None, persistent: bool | None = None) -> None:
        """Launch one decode token (fused or per-op, as the profile says).  persistent selects
        the one-launch step and four the four-launch fused step (default: each when the
        current length allows it; the persistent step first)."""
        if self.profile.fused_step:
            if persistent is None:
                persistent = self.persistent and not four
            if persistent:
                self._enqueue_persistent()
            else:
                self._enqueue_fused(self.four_launch if four is None else four)
        else:
            self._enqueue_per_op()

    def _enqueue_persistent(self) -> None:
        """Every layer in one launch (lt_decode_step), then the vocab GEMV with its argmax:
        the same arithmetic as _enqueue_fused, bit for bit."""
        if self.persistent_len <= 0:
            raise ValueError("the persistent step does not apply to this profile or geometry")
        cfg, m = self.cfg, self.model
        h = self.dev.handle
        eps = ctypes.c_float(cfg.norm_eps)
        self.enqueue_layers()
        hp = self.head_pl
        call("lt_q8_gemv_rms_argmax" + ("_pl" if hp else ""), h, self.carry.vp, m.output_norm.vp, eps,
             (hp or m.output).t.vp, self.logits.vp, cfg.vocab, cfg.n_embd, self.tok.vp, *self._hist_args(),
             self.am_ws.vp, self.am_ws.nbytes)
        self._enqueue_sample_if_on()

    def _enqueue_fused(self, four: bool = False) -> None:
        """Five launches per layer (lt_fused.hip), then the vocab GEMV with its argmax:
        the same arithmetic as _enqueue_per_op, bit for bit.
          QKV   rmsnorm -> quant -> GEMV + bias        (layer 0: from the embedding of tok)
          attn  RoPE -> KV append -> attention -> quant (split-K: partials, then a merge launch)
          O     GEMV + x, length += 1
          FFN1  rmsnorm -> quant -> gate|up GEMV -> SiLU(g)*u (-> quant, swiglu_fp32=False)
          FFN2  (quant ->) down GEMV + xres"""
        cfg, m, p = self.cfg, self.model, self.profile
        h = self.dev.handle
        E, F, hd, nh, nkv = cfg.n_embd, cfg.n_ff, cfg.head_dim, cfg.n_head, cfg.n_head_kv
        eps = ctypes.c_float(cfg.norm_eps)
        if four:
            if self.four_launch_len <= 0:
                raise ValueError("the four-launch step does not apply to this profile or geometry")
            self._enqueue_four()
            return
        ws, ws_n = _vp(self.attn_ws), (self.attn_ws.nbytes if self.attn_ws is not None else 0)
        pl = self.planar
        sfx = "_pl" if pl else ""

        def w(L, k):   # the matrix the step streams: its planar copy on planar plans
            return L[k + "_pl"].t.vp if pl else L[k].t.vp
        for il, L in enumerate(m.layers):
            cache = self.caches[il]
            x = self.resid_in if il == 0 else self.carry
            if il == 0 and not self.host_embed:
                call("lt_q8_gemv_embed_rms" + sfx, h, m.tok_embd.t.vp, self.tok.vp, cfg.vocab, self.resid_in.vp,
                     self.err.vp, L["attn_norm"].vp, eps, w(L, "wqkv"), _vp(L["bqkv"]), self.qkv.vp,
                     cfg.n_qkv, E)
            else:
                call("lt_q8_gemv_rms" + sfx, h, x.vp, L["attn_norm"].vp, eps, w(L, "wqkv"), _vp(L["bqkv"]),
                     self.qkv.vp, cfg.n_qkv, E)
            call("lt_attn_step", h, self.qkv.vp, m.freqs.vp, cache.k.vp, cache.v.vp, _vp(cache.len_ptr),
                 None, self.xq.vp, self.xd.vp, nh, nkv, hd, ctypes.c_float(self.scale), cache.max_seq,
                 p.attn_nsplit, p.kv_dtype, ws, ws_n)
            call("lt_q8_gemv_attn_out" + sfx, h, self.xq.vp, self.xd.vp, None, 0, 1, nh, hd, w(L, "wo"),
                 x.vp, self.xres.vp, E, cfg.q_dim, _vp(cache.len_ptr), cache.max_seq)
            if p.swiglu_fp32:
                call("lt_q8_gemv_rms_swiglu", h, self.xres.vp, L["ffn_norm"].vp, eps, L["wgu_il"].t.vp,
                     self.v.vp, F, E)
                call("lt_q8_gemv_quant", h, self.v.vp, L["wdown"].t.vp, self.xres.vp, self.carry.vp, E, F)
            else:
                call("lt_q8_gemv_rms_silu" + sfx, h, self.xres.vp, L["ffn_norm"].vp, eps, w(L, "wgu_il"),
                     self.xq.vp, self.xd.vp, F, E)
                call("lt_q8_gemv" + sfx, h, w(L, "wdown"), self.xq.vp, self.xd.vp, self.xres.vp, self.carry.vp,
                     E, F)
        hp = m.output_pl if pl else self.head_pl
        call("lt_q8_gemv_rms_argmax" + ("_pl" if hp else ""), h, self.carry.vp, m.output_norm.vp, eps,
             (hp or m.output).t.vp, self.logits.vp, cfg.vocab, E, self.tok.vp, *self._hist_args(),
             self.am_ws.vp, self.am_ws.nbytes)
        self._enqueue_sample_if_on()

    @property
    def four_launch_len(self) -> int:
        """Cache lengths up to which a step runs four launches per layer (the next token's
        attention covers length + 1 <= this many rows); 0 when the profile or the geometry
        keeps every step at five launches."""
        p, cfg = self.profile, self.cfg
        if not (p.fused_step and p.attn_in_o and p.attn_nsplit == 1 and not p.swiglu_fp32):
            return 0
        n = int(_lib.raw("lt_attn_o_max_len")(cfg.n_head, cfg.n_head_kv, cfg.head_dim, p.kv_dtype))
        return min(n, self.max_ctx) if n > 0 else 0

    @property
    def four_launch(self) -> bool:
        """The next step (at the current host length) runs four launches per layer."""
        return self.caches[0].length + 1 <= self.four_launch_len

    def enqueue_layers(self, layers: DevTensor | None = None) -> None:
        """The persistent step's launch alone (every layer; the last one's output row in
        carry), over the plan's layer descriptors or another array of them (`layers`: same
        caches and vectors, other weight copies -- the benchmark's rotation)."""
        cfg, m, p = self.cfg, self.model, self.profile
        gather = not self.host_embed
        call("lt_decode_step", self.dev.handle, (layers or self.step_layers).vp, cfg.n_layers, cfg.n_embd,
             cfg.n_ff, cfg.n_head, cfg.n_head_kv, cfg.head_dim, ctypes.c_float(cfg.norm_eps),
             ctypes.c_float(self.scale), m.freqs.vp, self.lens.vp, self.max_ctx, p.kv_dtype,
             m.tok_embd.t.vp if gather else None, self.tok.vp if gather else None, cfg.vocab,
             None if gather else self.resid_in.vp, self.carry.vp, self.err.vp, self.step_ws.vp,
             self.step_ws.nbytes)

    def step_layer_descs(self, weights: dict | None = None) -> DevTensor:
        """A device array of the persistent step's layer descriptors; `weights` maps
        (layer, name) for name in wqkv, wo, wgu_il, wdown to other device copies of those
        matrices (the plan's own otherwise)."""
        descs = (_StepLayer * self.cfg.n_layers)()
        for il, L in enumerate(self.model.layers):
            mat = lambda name: (weights or {}).get((il, name), L[name].t).ptr
            d = descs[il]
            d.attn_norm, d.bqkv = L["attn_norm"].ptr, (L["bqkv"].ptr if L["bqkv"] is not None else None)
            d.wqkv, d.wo, d.wgu, d.wdown = mat("wqkv"), mat("wo"), mat("wgu_il"), mat("wdown")
            d.ffn_norm = L["ffn_norm"].ptr
            d.kc, d.vc = self.caches[il].k.ptr, self.caches[il].v.ptr
        raw = np.frombuffer(bytes(descs), np.uint8).copy()
        t = DevTensor.empty((raw.size,), np.uint8, self.dev)
        self.dev.h2d(t.ptr, raw)
        return t

    def _enqueue_four(self) -> None:
        """Four launches per layer, the same bits as the five-launch step:
          QKV   rmsnorm -> quant -> GEMV + bias -> RoPE(q, k) -> k, v into the caches at *len
          O     attention over *len + 1 rows (every workgroup) -> quant -> O GEMV + x
          FFN1  rmsnorm -> quant -> gate|up GEMV -> SiLU(g)*u -> quant; *len += 1
          FFN2  down GEMV + xres"""
        cfg, m, p = self.cfg, self.model, self.profile
        h = self.dev.handle
        E, F, hd, nh, nkv = cfg.n_embd, cfg.n_ff, cfg.head_dim, cfg.n_head, cfg.n_head_kv
        eps = ctypes.c_float(cfg.norm_eps)
        scale = ctypes.c_float(self.scale)
        for il, L in enumerate(m.layers):
            cache = self.caches[il]
            lp = _vp(cache.len_ptr)
            x = self.resid_in if il == 0 else self.carry
            gather = il == 0 and not self.host_embed
            call("lt_q8_gemv_rms_rope_kv", h, None if gather else x.vp,
                 m.tok_embd.t.vp if gather else None, self.tok.vp if gather else None, cfg.vocab,
                 self.resid_in.vp if gather else None, self.err.vp, L["attn_norm"].vp, eps, L["wqkv"].t.vp,
                 _vp(L["bqkv"]), self.qkv.vp, E, m.freqs.vp, cache.k.vp, cache.v.vp, lp, nh, nkv, hd,
                 cache.max_seq, p.kv_dtype)
            call("lt_q8_gemv_attn_o", h, self.qkv.vp, cache.k.vp, cache.v.vp, lp, nh, nkv, hd, scale,
                 cache.max_seq, p.kv_dtype, L["wo"].t.vp, x.vp, self.xres.vp, E)
            call("lt_q8_gemv_rms_silu_len", h, self.xres.vp, L["ffn_norm"].vp, eps, L["wgu_il"].t.vp,
                 self.xq.vp, self.xd.vp, F, E, lp, cache.max_seq)
            call("lt_q8_gemv", h, L["wdown"].t.vp, self.xq.vp, self.xd.vp, self.xres.vp, self.carry.vp, E, F)
        call("lt_q8_gemv_rms_argmax", h, self.carry.vp, m.output_norm.vp, eps, m.output.t.vp, self.logits.vp,
             cfg.vocab, E, self.tok.vp, *self._hist_args(), self.am_ws.vp, self.am_ws.nbytes)
        self._enqueue_sample_if_on()

    def _enqueue_per_op(self) -> None:
        """Launch one token: embed(tok) -> layers -> logits -> argmax -> tok.
        The launch order is forward_pass_resident's fully-device branch
        (bpd/lib/dev_residency.py:1365-1477) followed by _compute_folded_logits (:1596-1623)
        and the device argmax of replay_token (:1795-1818).  Under numerics="ggml" every
        quantizer and GEMV is ggml's (lt_ggml.hip); the rest of the chain is unchanged."""
        cfg, m, p = self.cfg, self.model, self.profile
        h = self.dev.handle
        E, F, hd, nh, nkv = cfg.n_embd, cfg.n_ff, cfg.head_dim, cfg.n_head, cfg.n_head_kv
        eps = ctypes.c_float(cfg.norm_eps)
        if not self.host_embed:
            call("lt_embed_q8", h, m.tok_embd.t.vp, self.tok.vp, self.resid_in.vp, E, cfg.vocab, self.err.vp)
        x = self.resid_in
        for il, L in enumerate(m.layers):
            cache = self.caches[il]
            self._rms_quant(x, L["attn_norm"], E, eps)
            self._gemv(L["wqkv"], self.qkv, L["bqkv"])
            call("lt_rope_qk", h, self.qkv.vp, _vp(cache.len_ptr), nh + nkv, hd, m.freqs.vp)
            k = self.qkv.view(cfg.q_dim, (cfg.kv_dim,))
            v = self.qkv.view(cfg.q_dim + cfg.kv_dim, (cfg.kv_dim,))
            cache.append_at_len_incr(k, v)
            call("lt_attn_decode", h, self.qkv.vp, cache.k.vp, cache.v.vp, _vp(cache.len_ptr),
                 self.att.vp, 1, nh, nkv, hd, ctypes.c_float(self.scale), cache.max_seq,
                 p.attn_nsplit, p.kv_dtype, _vp(self.attn_ws),
                 self.attn_ws.nbytes if self.attn_ws is not None else 0)
            self._quant(self.att, cfg.q_dim)
            self._gemv(L["wo"], self.xres, x)
            self._rms_quant(self.xres, L["ffn_norm"], E, eps)
            self._gemv(L["wgu"], self.gu)
            g = self.gu.view(0, (F,))
            u = self.gu.view(F, (F,))
            if p.numerics == "ggml":     # SiLU(g)*u in place over g, then ggml's quantizer
                call("lt_silu_mul", h, g.vp, u.vp, g.vp, F)
                self._quant(g, F)
            else:
                call("lt_silu_mul_quant", h, g.vp, u.vp, self.xq.vp, self.xd.vp, F)
            self._gemv(L["wdown"], self.carry, self.xres)
            x = self.carry
        self._rms_quant(x, m.output_norm, E, eps)
        self._gemv(m.output, self.logits)
        if self.sampling:
            self._enqueue_sample(record=True)
        else:
            call("lt_argmax_record", h, self.logits.vp, cfg.vocab, self.tok.vp, self.hist.vp, self.hist_count.vp,
                 self.hist_cap, self.am_ws.vp, self.am_ws.nbytes)

    # -- sampling beyond greedy ----------------------------------------------------
    def set_sampling(self, temperature: float | None, top_k: int = 40, top_p: float = 1.0, seed: int = 0,
                     counter: int | None = None) -> None:
        """Draw every step's token with lt_sample (temperature, top-k, top-p; Philox stream
        `seed`, starting at draw `counter`) instead of the greedy argmax; temperature=None
        returns to greedy.  counter=None keeps the device's draw count when the plan already
        has sampling parameters (changing the temperature or the cuts mid-generation does not
        replay draws already spent), and starts at 0 otherwise.  The parameters live on the
        device: a captured graph reads them at every replay, so new values apply without
        re-capture; switching between greedy and sampling changes the launch sequence and
        needs a new capture."""
        if temperature is None:
            self.sampling = False
            return
        if not 1 <= int(top_k) <= LT_SAMPLE_MAX_K:
            raise ValueError(f"top_k={top_k}: 1 .. {LT_SAMPLE_MAX_K}")
        if self._sample_params is None:
            n = _lib.raw("lt_sample_workspace_size")(self.cfg.vocab)
            if n == 0:
                raise ValueError(f"lt_sample: vocab {self.cfg.vocab} is outside 1 .. 262144")
            self._sample_params = DevTensor.empty((32,), np.uint8, self.dev)
            self._sample_ws = DevTensor.empty((n,), np.uint8, self.dev)
            if counter is None:
                counter = 0
        elif counter is None:
            counter = self.sample_counter()
        rec = np.zeros(1, np.dtype([("temperature", "<f4"), ("top_k", "<i4"), ("top_p", "<f4"), ("reserved", "<i4"),
                                    ("seed", "<u8"), ("counter", "<u8")]))
        rec["temperature"], rec["top_k"], rec["top_p"] = temperature, int(top_k), top_p
        rec["seed"], rec["counter"] = int(seed) & (2 ** 64 - 1), int(counter)
        self.dev.h2d(self._sample_params.ptr, rec.view(np.uint8))
        self.sampling = True

    def sample_counter(self) -> int:
        """Draws made so far (the device counter)."""
        out = np.zeros(4, np.uint64)
        self.dev.d2h(out, self._sample_params.ptr)
        return int(out[3])

    def _hist_args(self) -> tuple:
        """The argmax launch records the token unless the sampler draws (and records) it."""
        if self.sampling:
            return (None, None, 0)
        return (self.hist.vp, self.hist_count.vp, self.hist_cap)

    def _enqueue_sample(self, record: bool) -> None:
        call("lt_sample", self.dev.handle, self.logits.vp, self.cfg.vocab, self._sample_params.vp, self.tok.vp,
             self.hist.vp if record else None, self.hist_count.vp if record else None,
             self.hist_cap if record else 0, self._sample_ws.vp, self._sample_ws.nbytes)

    def _enqueue_sample_if_on(self) -> None:
        if self.sampling:
            self._enqueue_sample(record=True)

    def sample_current(self) -> int:
        """Draw a token from the logits now on the device (after a prefill) into the device
        token, without recording it in the history; returns it."""
        if not self.sampling:
            raise ValueError("sample_current: set_sampling first")
        self._enqueue_sample(record=False)
        self.dev.sync()
        return self.read_token()

    def _quant(self, x: DevTensor, K: int) -> None:
        """The step's activation quantizer (the engine's, or ggml's under numerics="ggml")."""
        if self.profile.numerics == "ggml":
            call("lt_quant_q8_ggml", self.dev.handle, x.vp, self.xq.vp, self.xd.vp, K)
        else:
            quant_q8_into(x, self.xq, self.xd, K)

    def _gemv(self, W: Q8Weight, out: DevTensor, resid: DevTensor | None = None) -> None:
        """out = W . (xq, xd) (+ resid) in the step's GEMV order."""
        if self.profile.numerics == "ggml":
            call("lt_q8_gemv_ggml", self.dev.handle, W.t.vp, self.xq.vp, self.xd.vp, _vp(resid), out.vp,
                 W.N, W.K, LT_GGML_VEC)
        else:
            q8_gemv_into(W, self.xq, self.xd, out, resid)

    def _rms_quant(self, x: DevTensor, w: DevTensor, E: int, eps) -> None:
        h = self.dev.handle
        if self.profile.numerics == "ggml":
            call("lt_rmsnorm", h, x.vp, w.vp, self.h.vp, 1, E, eps)
            call("lt_quant_q8_ggml", h, self.h.vp, self.xq.vp, self.xd.vp, E)
        elif self.profile.fused_rms_quant:
            call("lt_rmsnorm_quant", h, x.vp, w.vp, self.xq.vp, self.xd.vp, E, eps)
        else:
            call("lt_rmsnorm", h, x.vp, w.vp, self.h.vp, 1, E, eps)
            call("lt_quant_q8", h, self.h.vp, self.xq.vp, self.xd.vp, E)

    def check_room(self, n: int = 1) -> None:
        """Refuse n more positions when the KV caches cannot hold them: past max_ctx the step
        kernels would attend over an empty context and drop the new row."""
        if self.caches[0].length + n > self.max_ctx:
            raise ValueError(f"KV cache full: {self.caches[0].length} + {n} positions exceed "
                             f"max_ctx {self.max_ctx}")

    def step(self, tok: int | None = None, embedding: np.ndarray | None = None) -> None:
        """Eager step (tok=None: use the device token left by the previous argmax).  A
        host_embed plan takes the token's input row as `embedding`."""
        self.check_room(1)
        if self.host_embed:
            if embedding is None:
                raise ValueError("a host_embed plan steps on a host embedding row")
            self.set_embedding(embedding)
        if tok is not None:
            self.set_token(tok)
        self.enqueue_step()
        for c in self.caches:
            c.length += 1

    def free(self) -> None:
        if self._prefill is not None:
            self._prefill.free()
        for c in self.caches:
            c.free()
        for t in (self.tok, self.err, self.hist, self.hist_count, self.lens, self.resid_in, self.carry,
                  self.xres, self.h, self.qkv, self.att, self.gu, self.v, self.logits, self.xq, self.xd,
                  self.am_ws, self.attn_ws, self._sample_params, self._sample_ws, self.step_ws,
                  self.step_layers):
            if t is not None:
                t.free()


class PrefillBuffers:
    """Device buffers of a batched prefill of up to T tokens."""

    def __init__(self, plan: "DecodePlan", T: int):
        cfg, D = plan.cfg, plan.dev
        E, F = cfg.n_embd, cfg.n_ff
        kmax = max(E, F, cfg.q_dim)
        self.T = T
        self.toks = DevTensor.empty((T,), np.int32, D)
        self.x = DevTensor.empty((T, E), np.float32, D)
        self.xres = DevTensor.empty((T, E), np.float32, D)
        self.qkv = DevTensor.empty((T, cfg.n_qkv), np.float32, D)
        self.att = DevTensor.empty((T, cfg.q_dim), np.float32, D)
        self.v = DevTensor.empty((T, F), np.float32, D)
        self.xq = DevTensor.empty((T * kmax,), np.int8, D)
        self.xd = DevTensor.empty((T * kmax // 32,), np.uint16, D)
        aw = _lib.raw("lt_attn_workspace_size")(T, cfg.n_head, cfg.head_dim, plan.profile.attn_nsplit)
        self.ws = DevTensor.empty((aw,), np.uint8, D) if aw else None

    def free(self) -> None:
        for t in (self.toks, self.x, self.xres, self.qkv, self.att, self.v, self.xq, self.xd, self.ws):
            if t is not None:
                t.free()


def forward_prefill(plan: DecodePlan, tokens, embeddings: np.ndarray | None = None) -> None:
    """Batched prefill of a prompt: every linear layer runs once over all T tokens through
    the int8-MFMA Q8_0 GEMM on the coalesced layouts (tile-major weight copies from
    ResidentModel.prefill_tiles, block-major activation quants; lt_q8_gemm_t), with batched
    RMSNorm/RoPE/KV append and causal attention.  It is device-uniform with the single-token
    path the reference uses (bpd/lib/dev_residency.py:1338-1356): the KV cache, the last
    token's logits and the greedy token it leaves on the device are bit-identical to
    forward_tokens's.  A host_embed plan takes the prompt's input rows as `embeddings`
    (fp32 [T, n_embd]).  The ggml numerics profile has no batched form (its decode order is
    ggml's single-token vec_dot): it prefills with forward_tokens."""
    if plan.profile.numerics != "engine":
        raise ValueError("forward_prefill runs the engine's numerics; a ggml-numerics plan prefills "
                         "token by token (forward_tokens)")
    toks = np.asarray([int(t) for t in np.asarray(tokens).reshape(-1)], np.int32)
    T = int(toks.size)
    if T == 0:
        return
    cfg, m, p, D = plan.cfg, plan.model, plan.profile, plan.dev
    if plan.caches[0].length + T > plan.max_ctx:
        raise ValueError(f"prefill of {T} tokens overflows the {plan.max_ctx}-position KV cache")
    if "wgu_il" not in m.layers[0]:
        raise ValueError("forward_prefill needs the fused gate|up layout (ResidentModel layouts 'fused' or 'both')")
    # every layer's length sits in the plan's one array, so all of them advance in one launch
    # after the last layer's attention (each layer's attention reads only its own)
    if not all(c.len_ptr == plan.lens.ptr + 4 * il and c.max_seq == plan.max_ctx
               for il, c in enumerate(plan.caches)):
        raise ValueError("forward_prefill needs the DecodePlan's joint length array")
    m.prefill_tiles()
    B = plan.prefill_buffers(T)
    h = D.handle
    E, F, hd, nh, nkv = cfg.n_embd, cfg.n_ff, cfg.head_dim, cfg.n_head, cfg.n_head_kv
    QD, KD, NQ = cfg.q_dim, cfg.kv_dim, cfg.n_qkv
    eps = ctypes.c_float(cfg.norm_eps)
    if plan.host_embed:
        if embeddings is None:
            raise ValueError("a host_embed plan prefills from host embedding rows")
        X = np.ascontiguousarray(embeddings, np.float32).reshape(-1)
        if X.size != T * E:
            raise ValueError(f"embeddings hold {X.size} values, expected {T} x {E}")
        D.h2d(B.x.ptr, X)
    else:
        D.h2d(B.toks.ptr, toks)
        call("lt_embed_q8_batch", h, m.tok_embd.t.vp, B.toks.vp, B.x.vp, T, E, cfg.vocab, plan.err.vp)
    _prefill_layers(m, p, B, T, [(c.k.vp, c.v.vp, _vp(c.len_ptr)) for c in plan.caches], plan.max_ctx,
                    plan.scale)
    call("lt_len_add_n", h, _vp(plan.lens.ptr), len(m.layers), T, plan.max_ctx)
    for cache in plan.caches:   # the host mirror advances with the device lengths
        cache.length += T
    # the last token's logits and greedy token, as the decode step computes them
    D.d2d(plan.carry.ptr, B.x.ptr + (T - 1) * E * 4, E * 4)
    call("lt_q8_gemv_rms_argmax", h, plan.carry.vp, m.output_norm.vp, eps, m.output.t.vp, plan.logits.vp,
         cfg.vocab, E, plan.tok.vp, None, None, 0, plan.am_ws.vp, plan.am_ws.nbytes)


def _prefill_layers(m: ResidentModel, p: Profile, B: PrefillBuffers, T: int, caches: list, maxt: int,
                    scale: float) -> None:
    """The layers of a batched prefill of the T rows in B.x, one sequence: caches[il] =
    (k, v, len) device pointers of layer il's cache and its length (read, not advanced)."""
    cfg, h = m.cfg, m.dev.handle
    E, F, hd, nh, nkv = cfg.n_embd, cfg.n_ff, cfg.head_dim, cfg.n_head, cfg.n_head_kv
    QD, NQ = cfg.q_dim, cfg.n_qkv
    eps = ctypes.c_float(cfg.norm_eps)
    ws, ws_n = _vp(B.ws), (B.ws.nbytes if B.ws is not None else 0)
    for il, L in enumerate(m.layers):
        kp, vp, lp = caches[il]
        call("lt_rmsnorm_quant_bm", h, B.x.vp, L["attn_norm"].vp, B.xq.vp, B.xd.vp, T, E, eps)
        call("lt_q8_gemm_t", h, L["wqkv_t"].t.vp, B.xq.vp, B.xd.vp, _vp(L["bqkv"]), None, B.qkv.vp, T, NQ, E)
        call("lt_rope_append_batch", h, B.qkv.vp, T, NQ, lp, nh, nkv, hd, m.freqs.vp, kp, vp, maxt, p.kv_dtype)
        call("lt_attn_prefill", h, B.qkv.vp, NQ, kp, vp, lp, B.att.vp, T, nh, nkv, hd, ctypes.c_float(scale), maxt,
             p.attn_nsplit, p.kv_dtype, ws, ws_n)
        call("lt_quant_q8_bm", h, B.att.vp, B.xq.vp, B.xd.vp, T, QD)
        call("lt_q8_gemm_t", h, L["wo_t"].t.vp, B.xq.vp, B.xd.vp, None, B.x.vp, B.xres.vp, T, E, QD)
        call("lt_rmsnorm_quant_bm", h, B.xres.vp, L["ffn_norm"].vp, B.xq.vp, B.xd.vp, T, E, eps)
        call("lt_q8_gemm_silu_t", h, L["wgu_il_t"].t.vp, B.xq.vp, B.xd.vp, B.v.vp, T, F, E)
        call("lt_quant_q8_bm", h, B.v.vp, B.xq.vp, B.xd.vp, T, F)
        call("lt_q8_gemm_t", h, L["wdown_t"].t.vp, B.xq.vp, B.xd.vp, None, B.xres.vp, B.x.vp, T, E, F)


def forward_tokens(plan: DecodePlan, tokens, embeddings: np.ndarray | None = None) -> np.ndarray:
    """Feed tokens one at a time through the single-token device path (the reference's
    device-uniform prefill, dev_residency.py:1338-1356); return the last token's logits.
    A host_embed plan takes the tokens' input rows as `embeddings` [T, n_embd]."""
    toks = [int(t) for t in np.asarray(tokens).reshape(-1)]
    if plan.host_embed:
        if embeddings is None:
            raise ValueError("a host_embed plan steps on host embedding rows")
        X = np.asarray(embeddings, np.float32).reshape(len(toks), -1)
        for t, row in zip(toks, X):
            plan.step(t, row)
    else:
        for t in toks:
            plan.step(t)
    return plan.read_logits()


class StepGraph:
    """Capture one decode step into a HIP graph and replay it per token
    (reference GraphRunner, bpd/lib/dev_residency.py:1626-1818)."""

    def __init__(self, plan: DecodePlan):
        self.plan = plan
        self.dev = plan.dev
        self.graph = ctypes.c_void_p()    # the five-launch step (every length)
        self.graph4 = ctypes.c_void_p()   # the four-launch step (lengths up to plan.four_launch_len)
        self.graphp = ctypes.c_void_p()   # the persistent step (lengths up to plan.persistent_len)
        self.captured = False
        self.captured_sampling = False

    def seed(self, prompt, batched: bool = False, embeddings: np.ndarray | None = None) -> np.ndarray:
        """Eager prefill over the prompt (fixed buffers, all kernels loaded); returns the
        last prompt token's logits.  The device token then holds the first greedy token.
        batched=True runs forward_prefill (the int8-MFMA GEMM path; bit-identical)."""
        if batched:
            forward_prefill(self.plan, prompt, embeddings)
            logits = self.plan.read_logits()
        else:
            logits = forward_tokens(self.plan, prompt, embeddings)
        self.dev.sync()
        return logits

    def _capture_one(self, out: ctypes.c_void_p, four: bool, persistent: bool = False) -> None:
        call("lt_graph_begin", self.dev.handle)
        try:
            self.plan.enqueue_step(four=four, persistent=persistent)
        except Exception:
            g = ctypes.c_void_p()
            _lib.raw("lt_graph_end")(self.dev.handle, ctypes.byref(g))
            if g.value:
                _lib.raw("lt_graph_free")(g)
            raise
        call("lt_graph_end", self.dev.handle, ctypes.byref(out))

    def capture(self) -> None:
        """Record the step: the five-launch graph, and when the plan has one, the four-launch
        graph that replays take while the cache is short enough for it."""
        if self.captured:
            raise RuntimeError("StepGraph.capture: already captured")
        self._capture_one(self.graph, False)
        try:
            if self.plan.four_launch_len > 0 and self.plan.profile.fused_step:
                self._capture_one(self.graph4, True)
            if self.plan.persistent_len > 0:
                self._capture_one(self.graphp, False, persistent=True)
        except Exception:
            for g in (self.graph, self.graph4):
                if g.value:
                    _lib.raw("lt_graph_free")(g)
            self.graph, self.graph4 = ctypes.c_void_p(), ctypes.c_void_p()
            raise
        self.captured = True
        self.captured_sampling = self.plan.sampling

    def _launch(self) -> None:
        if not self.captured:
            raise RuntimeError("call capture() before replay")
        if self.plan.sampling != self.captured_sampling:
            raise RuntimeError("the plan switched between greedy and sampling after capture: capture again")
        self.plan.check_room(1)
        if self.graphp.value and self.plan.persistent:
            g = self.graphp
        elif self.graph4.value and self.plan.four_launch:
            g = self.graph4
        else:
            g = self.graph
        call("lt_graph_launch", self.dev.handle, g)
        for c in self.plan.caches:
            c.length += 1

    def _set_input(self, tok, embedding) -> None:
        if self.plan.host_embed:
            if embedding is None:
                raise ValueError("a host_embed plan replays on a host embedding row")
            self.plan.set_embedding(embedding)
        if tok is not None:
            self.plan.set_token(tok)

    def replay_logits(self, tok: int, embedding: np.ndarray | None = None) -> np.ndarray:
        self._set_input(tok, embedding)
        self._launch()
        return self.plan.read_logits()

    def replay_token(self, tok: int | None = None, embedding: np.ndarray | None = None) -> int:
        """One graph replay; returns the next token, greedy or drawn by the plan's sampler
        (4 bytes cross to the host)."""
        self._set_input(tok, embedding)
        self._launch()
        return self.plan.read_token()

    def replay_tokens(self, n: int) -> list[int]:
        """n back-to-back replays continuing from the device token; the host reads the n
        generated ids once at the end from the device history.  Same tokens as n calls of
        replay_token()."""
        if self.plan.host_embed:
            raise ValueError("replay_tokens feeds each argmax back on the device; a host_embed "
                             "plan takes every input row from the host (replay_token per token)")
        start = self.plan.history_count()
        if start + n > self.plan.hist_cap:
            raise ValueError(f"token history capacity {self.plan.hist_cap} exceeded")
        self.plan.check_room(n)
        for _ in range(n):
            self._launch()
        return self.plan.history()[start:start + n]

    def free(self) -> None:
        if self.captured:
            call("lt_graph_free", self.graph)
            for g in (self.graph4, self.graphp):
                if g.value:
                    call("lt_graph_free", g)
            self.graph = ctypes.c_void_p()
            self.graph4 = ctypes.c_void_p()
            self.graphp = ctypes.c_void_p()
            self.captured = False


# ----------------------------------------------------------------------------------
# Batched decode (bs > 1): B independent sequences, one token of each per step
# ----------------------------------------------------------------------------------
# the batched step's linear layers: the multi-token GEMV up to here, the GEMM above (C2, graph
# replays: GEMV 5922 / 17969 / 25527 / 33741 tok/s at B = 8 / 32 / 64 / 128, GEMM 2590 / 10107
# / 19686 / 38195)
# from MIXED_MIN_BATCH sequences the step's gate|up, down and vocab projections run the tiled
# GEMM (linear "mixed"), past MIXED_MAX_BATCH every projection does ("gemm"); measured C2 step
# tok/s, GEMV / mixed / GEMM: B = 8 8176 / 6974 / 5675, 16 13626 / 13488 / 11194, 32 21951 /
# 25259 / 21165, 64 31268 / 44419 / 39651, 96 35061 / 57007 / 54339, 128 38245 / 70172 / 69351;
# with the vocab GEMM and the fused SiLU quant, GEMV / mixed: 16 14328 / 13942, 20 17031 /
# 17058, 24 19902 / 20197, 28 22229 / 23110; after the leaf-split kernel's compile-time
# schedule and coalesced epilogues, GEMV / mixed: 2 2311 / 2253, 4 4430 / 4390, 8 8530 / 8654,
# 12 11381 / 12523, 16 14651 / 16491, 24 20275 / 23831
MIXED_MIN_BATCH = 8
MIXED_MAX_BATCH = 128
# from this many sequences the vocab projection runs the tiled GEMM in every form; measured
# 151936 x 896 per launch, multi-token GEMV / tiled GEMM (us): T = 1 32.3 / 54.2, 4 39.2 / 51.5,
# 6 63.2 / 51.8, 8 73.9 / 55.5, 16 125.6 / 56.8
HEAD_GEMM_MIN_BATCH = 5
# up to this many sequences the mixed form's gate|up launch also quantizes its SiLU output
# (lt_q8_gemm_silu_quant_t: workgroups of two row tiles, 8 waves); past it the separate quant
# launch; C2 tok/s fused / separate: B = 64 51389 / 50691, 128 90007 / 88532 (the mixed
# form's whole range)
SILU_QUANT_MAX_BATCH = 128
# from this many sequences the mixed and GEMM forms run q|k|v on the tiled GEMM with the RoPE +
# KV-append epilogue (lt_q8_gemm_rope_t, the weights in the rope-pair order) instead of the
# multi-token GEMV with it (mixed) or the GEMM followed by lt_rope_append_seqs (GEMM form);
# C2 mixed-form tok/s, GEMV / GEMM q|k|v: B = 24 21428 / 21050, 32 27692 / 27312, 64 48003 /
# 49424, 128 77421 / 83263
QKV_GEMM_MIN_BATCH = 48
# from this many sequences the mixed form's attention writes block-major quants
# (lt_attn_decode_rows_q8_bm, one split) and O runs the tiled GEMM with the residual epilogue
# (the GEMM form always does, with one split); C2 mixed-form tok/s, O on the GEMV / GEMM: B =
# 48 38518 / 37539, 64 49727 / 48617, 128 83618 / 86406; after the coalesced epilogues: 8 8654
# / 8506, 12 12523 / 12526, 16 16491 / 16536, 32 30830 / 31088, 64 55985 / 57325
O_GEMM_MIN_BATCH = 16


class BatchDecodePlan:
    """B sequences decoded together (the reference's future-work note on batching its
    device-uniform path, bpd/lib/dev_residency.py:1344-1350).  Each step takes the next token
    of every sequence: the linear layers run once over the B rows through the prefill's
    int8-MFMA GEMM (each weight byte read once per step, not once per sequence), RoPE and the
    KV append per sequence at its own length, the batched decode attention over each
    sequence's own cache, and a row-wise argmax.  Row b is bit-identical to sequence b
    decoded alone by DecodePlan (the GEMM is device-uniform with the GEMV).

    Device state: per layer one K and one V cache of [B][max_ctx][n_kv*head_dim]; lens =
    [pos[0..B), attn[0..B)] with pos[b] the length of sequence b (shared by its layers) and
    attn[b] = pos[b] + 1 the rows its next step attends; toks[b]; histories hist[b][cap]."""

    def __init__(self, model: ResidentModel, batch: int, profile: Profile = PRODUCTION_PROFILE,
                 max_ctx: int | None = None, hist_cap: int = 4096, linear: str = "auto"):
        """linear: "gemv" runs the step's linear layers through the multi-token GEMV
        (lt_q8_gemv_multi: GGUF-layout weights, row-major quants, each weight block read once
        per 8 tokens), "gemm" through the prefill GEMM (tile-major weights), "mixed" QKV and O
        through the GEMV and the rest through the GEMM; "auto" picks the GEMV below
        MIXED_MIN_BATCH sequences, "mixed" up to MIXED_MAX_BATCH and "gemm" past that.
        Same bits every way."""
        assert_certified_composition(profile)
        if linear not in ("auto", "gemv", "gemm", "mixed"):
            raise ValueError(f"linear={linear!r}")
        if profile.numerics != "engine":
            raise ValueError("batched decode runs the engine's numerics")
        if "wgu_il" not in model.layers[0]:
            raise ValueError("batched decode needs the fused gate|up layout (layouts 'fused' or 'both')")
        if batch < 1:
            raise ValueError(f"batch={batch}")
        self.model, self.cfg, self.profile, self.dev = model, model.cfg, profile, model.dev
        self.B = int(batch)
        if linear == "auto":
            linear = "gemv" if self.B < MIXED_MIN_BATCH else "mixed" if self.B <= MIXED_MAX_BATCH else "gemm"
        self.linear = linear
        cfg, D = self.cfg, self.dev
        E, F, B = cfg.n_embd, cfg.n_ff, self.B
        self.max_ctx = int(max_ctx or cfg.max_ctx)
        model.prefill_tiles()
        self.head = model.head_tiles()
        self.qkv_gemm = linear in ("mixed", "gemm") and self.B >= QKV_GEMM_MIN_BATCH
        self.o_gemm = profile.attn_nsplit == 1 and (linear == "gemm" or
                                                    (linear == "mixed" and self.B >= O_GEMM_MIN_BATCH))
        if self.qkv_gemm:
            model.qkv_rope_tiles()
        esz = 2 if profile.kv_dtype == LT_KV_F16 else 4
        self.slot_bytes = self.max_ctx * cfg.kv_dim * esz
        self.k = [DevTensor.empty((B * self.slot_bytes,), np.uint8, D) for _ in range(cfg.n_layers)]
        self.v = [DevTensor.empty((B * self.slot_bytes,), np.uint8, D) for _ in range(cfg.n_layers)]
        self.lens = DevTensor.empty((2 * B,), np.int32, D)
        self.toks = DevTensor.empty((B,), np.int32, D)
        self.err = DevTensor.empty((1,), np.int32, D)
        self.hist_cap = int(hist_cap)
        self.hist = DevTensor.empty((B, self.hist_cap), np.int32, D)
        self.hist_count = DevTensor.empty((B,), np.int32, D)
        kmax = max(E, F, cfg.q_dim)
        self.x = DevTensor.empty((B, E), np.float32, D)
        self.xres = DevTensor.empty((B, E), np.float32, D)
        self.qkv = DevTensor.empty((B, cfg.n_qkv), np.float32, D)
        self.att = DevTensor.empty((B, cfg.q_dim), np.float32, D)
        self.vbuf = DevTensor.empty((B, F), np.float32, D)
        self.xq = DevTensor.empty((B * kmax,), np.int8, D)
        self.xd = DevTensor.empty((B * kmax // 32,), np.uint16, D)
        # the mixed form's SiLU output quants (the gate|up launch writes them while its input
        # quants are still being read, so not into xq / xd)
        self.vq = DevTensor.empty((B * F,), np.int8, D)
        self.vd = DevTensor.empty((B * F // 32,), np.uint16, D)
        self.logits = DevTensor.empty((B, cfg.vocab), np.float32, D)
        aw = _lib.raw("lt_attn_workspace_size")(B, cfg.n_head, cfg.head_dim, profile.attn_nsplit)
        self.attn_ws = DevTensor.empty((aw,), np.uint8, D) if aw else None
        self.am_ws = DevTensor.empty((int(_lib.raw("lt_argmax_rows_workspace_size")(B)),), np.uint8, D)
        self.scale = float(cfg.head_dim ** -0.5)
        self._prefill: PrefillBuffers | None = None
        self.length = [0] * B
        self.reset()

    # -- state --------------------------------------------------------------------
    def reset(self, b: int | None = None) -> None:
        """Empty every sequence (or sequence b): length 0, history cleared."""
        seqs = range(self.B) if b is None else [b]
        for i in seqs:
            self.length[i] = 0
        self._push_lengths()
        cnt = np.zeros(self.B, np.int32)
        if b is not None:
            self.dev.d2h(cnt, self.hist_count.ptr)
            cnt[b] = 0
        self.dev.h2d(self.hist_count.ptr, cnt)
        self.dev.h2d(self.err.ptr, np.zeros(1, np.int32))

    def _push_lengths(self) -> None:
        pos = np.asarray(self.length, np.int32)
        self.dev.h2d(self.lens.ptr, np.concatenate([pos, np.minimum(pos + 1, self.max_ctx)]).astype(np.int32))

    def set_tokens(self, toks) -> None:
        t = np.asarray([int(x) for x in toks], np.int32)
        if t.size != self.B:
            raise ValueError(f"{t.size} tokens for a batch of {self.B}")
        self.dev.h2d(self.toks.ptr, t)

    def read_tokens(self) -> list[int]:
        out = np.zeros(self.B, np.int32)
        self.dev.d2h(out, self.toks.ptr)
        return [int(v) for v in out]

    def read_logits(self) -> np.ndarray:
        out = np.zeros((self.B, self.cfg.vocab), np.float32)
        self.dev.d2h(out, self.logits.ptr)
        return out

    def history(self) -> list[list[int]]:
        cnt = np.zeros(self.B, np.int32)
        self.dev.d2h(cnt, self.hist_count.ptr)
        h = np.zeros((self.B, self.hist_cap), np.int32)
        self.dev.d2h(h, self.hist.ptr)
        return [[int(v) for v in h[b, :cnt[b]]] for b in range(self.B)]

    def check_room(self, n: int = 1) -> None:
        full = [b for b in range(self.B) if self.length[b] + n > self.max_ctx]
        if full:
            raise ValueError(f"KV cache full for sequences {full} (max_ctx {self.max_ctx})")

    # -- prefill of one sequence ----------------------------------------------------
    def prefill(self, b: int, tokens) -> None:
        """Batched prefill of sequence b's prompt (continuing at its current length): its KV
        rows, its length, and -- from the last prompt token -- its logits row and greedy token
        (not recorded in the history), bit-identical to forward_prefill of a lone sequence."""
        toks = np.asarray([int(t) for t in np.asarray(tokens).reshape(-1)], np.int32)
        T = int(toks.size)
        if not 0 <= b < self.B:
            raise ValueError(f"sequence {b} of a batch of {self.B}")
        if T == 0:
            return
        if self.length[b] + T > self.max_ctx:
            raise ValueError(f"prefill of {T} tokens overflows sequence {b}'s {self.max_ctx}-position cache")
        cfg, m, D = self.cfg, self.model, self.dev
        h, E = D.handle, cfg.n_embd
        if self._prefill is None or self._prefill.T < T:
            if self._prefill is not None:
                D.sync()
                self._prefill.free()
            self._prefill = PrefillBuffers(self, max(T, 32))
        Bf = self._prefill
        D.h2d(Bf.toks.ptr, toks)
        call("lt_embed_q8_batch", h, m.tok_embd.t.vp, Bf.toks.vp, Bf.x.vp, T, E, cfg.vocab, self.err.vp)
        lp = self.lens.ptr + 4 * b
        off = b * self.slot_bytes
        _prefill_layers(m, self.profile, Bf, T, [(self.k[il].ptr + off, self.v[il].ptr + off, lp)
                                                 for il in range(cfg.n_layers)], self.max_ctx, self.scale)
        call("lt_len_add", h, _vp(lp), T, self.max_ctx)
        call("lt_len_add", h, _vp(self.lens.ptr + 4 * (self.B + b)), T, self.max_ctx)
        self.length[b] += T
        call("lt_rmsnorm_quant_bm", h, Bf.x.ptr + (T - 1) * E * 4, m.output_norm.vp, Bf.xq.vp, Bf.xd.vp, 1, E,
             ctypes.c_float(cfg.norm_eps))
        call("lt_q8_gemm_t", h, self.head.t.vp, Bf.xq.vp, Bf.xd.vp, None, None, self.logits.ptr + b * cfg.vocab * 4,
             1, cfg.vocab, E)
        call("lt_argmax_rows", h, self.logits.ptr + b * cfg.vocab * 4, 1, cfg.vocab, self.toks.ptr + 4 * b, None,
             None, 0)
        D.sync()

    # -- the batched step -----------------------------------------------------------
    def enqueue_step(self) -> None:
        """Launch one token of every sequence: embed -> layers -> vocab GEMM -> row argmax."""
        if self.linear in ("gemv", "mixed"):
            self._enqueue_step_gemv(mixed=self.linear == "mixed")
            return
        cfg, m, p, B = self.cfg, self.model, self.profile, self.B
        h = self.dev.handle
        E, F, hd, nh, nkv = cfg.n_embd, cfg.n_ff, cfg.head_dim, cfg.n_head, cfg.n_head_kv
        QD, NQ, V = cfg.q_dim, cfg.n_qkv, cfg.vocab
        eps = ctypes.c_float(cfg.norm_eps)
        pos, attn = _vp(self.lens.ptr), _vp(self.lens.ptr + 4 * B)
        ws, ws_n = _vp(self.attn_ws), (self.attn_ws.nbytes if self.attn_ws is not None else 0)
        call("lt_embed_q8_batch", h, m.tok_embd.t.vp, self.toks.vp, self.x.vp, B, E, cfg.vocab, self.err.vp)
        for il, L in enumerate(m.layers):
            kp, vp = self.k[il].vp, self.v[il].vp
            call("lt_rmsnorm_quant_bm", h, self.x.vp, L["attn_norm"].vp, self.xq.vp, self.xd.vp, B, E, eps)
            if self.qkv_gemm:
                call("lt_q8_gemm_rope_t", h, L["wqkv_rt"].t.vp, self.xq.vp, self.xd.vp, B, _vp(L["bqkv"]),
                     self.qkv.vp, NQ, E, pos, nh, nkv, hd, m.freqs.vp, kp, vp, self.max_ctx, p.kv_dtype)
            else:
                call("lt_q8_gemm_t", h, L["wqkv_t"].t.vp, self.xq.vp, self.xd.vp, _vp(L["bqkv"]), None,
                     self.qkv.vp, B, NQ, E)
                call("lt_rope_append_seqs", h, self.qkv.vp, B, NQ, pos, nh, nkv, hd, m.freqs.vp, kp, vp,
                     self.max_ctx, p.kv_dtype)
            if self.o_gemm:
                # the attention writes the O projection's block-major quants itself
                call("lt_attn_decode_rows_q8_bm", h, self.qkv.vp, NQ, kp, vp, attn, None, self.xq.vp, self.xd.vp,
                     B, nh, nkv, hd, ctypes.c_float(self.scale), self.max_ctx, p.kv_dtype)
            else:
                call("lt_attn_decode_rows", h, self.qkv.vp, NQ, kp, vp, attn, self.att.vp, B, nh, nkv, hd,
                     ctypes.c_float(self.scale), self.max_ctx, p.attn_nsplit, p.kv_dtype, ws, ws_n)
                call("lt_quant_q8_bm", h, self.att.vp, self.xq.vp, self.xd.vp, B, QD)
            call("lt_q8_gemm_t", h, L["wo_t"].t.vp, self.xq.vp, self.xd.vp, None, self.x.vp, self.xres.vp, B, E, QD)
            call("lt_rmsnorm_quant_bm", h, self.xres.vp, L["ffn_norm"].vp, self.xq.vp, self.xd.vp, B, E, eps)
            call("lt_q8_gemm_silu_t", h, L["wgu_il_t"].t.vp, self.xq.vp, self.xd.vp, self.vbuf.vp, B, F, E)
            call("lt_quant_q8_bm", h, self.vbuf.vp, self.xq.vp, self.xd.vp, B, F)
            call("lt_q8_gemm_t", h, L["wdown_t"].t.vp, self.xq.vp, self.xd.vp, None, self.xres.vp, self.x.vp, B, E, F)
        call("lt_len_add_n", h, _vp(self.lens.ptr), 2 * B, 1, self.max_ctx)
        call("lt_rmsnorm_quant_bm", h, self.x.vp, m.output_norm.vp, self.xq.vp, self.xd.vp, B, E, eps)
        call("lt_q8_gemm_t", h, self.head.t.vp, self.xq.vp, self.xd.vp, None, None, self.logits.vp, B, V, E)
        call("lt_argmax_rows_ws", h, self.logits.vp, B, V, self.toks.vp, self.hist.vp, self.hist_count.vp,
             self.hist_cap, self.am_ws.vp, self.am_ws.nbytes)

    def _enqueue_step_gemv(self, mixed: bool = False) -> None:
        """The step with the multi-token GEMV: 8 launches per layer (the QKV launch also rotates
        q and k and appends k and v; the attention writes the O projection's activation quants
        itself), each weight matrix streamed from its GGUF-layout
        blocks once per group of 2 to 8 sequences.  mixed: gate|up, down and the vocab
        projection run the tiled GEMM instead (tile-major weights, block-major quants; the
        leaf-split kernel at these token counts), whose weight blocks are read once per 32
        sequences; O stays on the GEMV, and QKV too below QKV_GEMM_MIN_BATCH sequences (from
        there the GEMM with the RoPE + KV-append epilogue)."""
        cfg, m, p, B = self.cfg, self.model, self.profile, self.B
        h = self.dev.handle
        E, F, hd, nh, nkv = cfg.n_embd, cfg.n_ff, cfg.head_dim, cfg.n_head, cfg.n_head_kv
        QD, NQ, V = cfg.q_dim, cfg.n_qkv, cfg.vocab
        eps = ctypes.c_float(cfg.norm_eps)
        pos, attn = _vp(self.lens.ptr), _vp(self.lens.ptr + 4 * B)
        ws, ws_n = _vp(self.attn_ws), (self.attn_ws.nbytes if self.attn_ws is not None else 0)
        xq, xd = self.xq.vp, self.xd.vp
        call("lt_embed_q8_batch", h, m.tok_embd.t.vp, self.toks.vp, self.x.vp, B, E, cfg.vocab, self.err.vp)
        for il, L in enumerate(m.layers):
            kp, vp = self.k[il].vp, self.v[il].vp
            # q|k|v + bias, RoPE and the KV append in one launch
            if self.qkv_gemm:
                call("lt_rmsnorm_quant_bm", h, self.x.vp, L["attn_norm"].vp, xq, xd, B, E, eps)
                call("lt_q8_gemm_rope_t", h, L["wqkv_rt"].t.vp, xq, xd, B, _vp(L["bqkv"]), self.qkv.vp, NQ, E, pos,
                     nh, nkv, hd, m.freqs.vp, kp, vp, self.max_ctx, p.kv_dtype)
            else:
                call("lt_rmsnorm_quant_rows", h, self.x.vp, L["attn_norm"].vp, xq, xd, B, E, eps)
                call("lt_q8_gemv_multi_rope", h, L["wqkv"].t.vp, xq, xd, B, _vp(L["bqkv"]), self.qkv.vp, NQ, E,
                     pos, nh, nkv, hd, m.freqs.vp, kp, vp, self.max_ctx, p.kv_dtype)
            if self.o_gemm:
                call("lt_attn_decode_rows_q8_bm", h, self.qkv.vp, NQ, kp, vp, attn, None, xq, xd, B, nh, nkv, hd,
                     ctypes.c_float(self.scale), self.max_ctx, p.kv_dtype)
                call("lt_q8_gemm_t", h, L["wo_t"].t.vp, xq, xd, None, self.x.vp, self.xres.vp, B, E, QD)
            else:
                call("lt_attn_decode_rows_q8", h, self.qkv.vp, NQ, kp, vp, attn, None, xq, xd, B, nh, nkv, hd,
                     ctypes.c_float(self.scale), self.max_ctx, p.attn_nsplit, p.kv_dtype, ws, ws_n)
                call("lt_q8_gemv_multi", h, L["wo"].t.vp, xq, xd, B, self.x.vp, self.xres.vp, E, QD,
                     LT_MULTI_RESID)
            if mixed:
                call("lt_rmsnorm_quant_bm", h, self.xres.vp, L["ffn_norm"].vp, xq, xd, B, E, eps)
                if B <= SILU_QUANT_MAX_BATCH:
                    # gate|up + SiLU with the block-major quant of its output in one launch
                    call("lt_q8_gemm_silu_quant_t", h, L["wgu_il_t"].t.vp, xq, xd, self.vq.vp, self.vd.vp, B, F,
                         E)
                    call("lt_q8_gemm_t", h, L["wdown_t"].t.vp, self.vq.vp, self.vd.vp, None, self.xres.vp,
                         self.x.vp, B, E, F)
                else:
                    call("lt_q8_gemm_silu_t", h, L["wgu_il_t"].t.vp, xq, xd, self.vbuf.vp, B, F, E)
                    call("lt_quant_q8_bm", h, self.vbuf.vp, xq, xd, B, F)
                    call("lt_q8_gemm_t", h, L["wdown_t"].t.vp, xq, xd, None, self.xres.vp, self.x.vp, B, E, F)
            else:
                call("lt_rmsnorm_quant_rows", h, self.xres.vp, L["ffn_norm"].vp, xq, xd, B, E, eps)
                call("lt_q8_gemv_multi", h, L["wgu_il"].t.vp, xq, xd, B, None, self.vbuf.vp, 2 * F, E,
                     LT_MULTI_SILU)
                call("lt_quant_q8", h, self.vbuf.vp, xq, xd, B * F)
                call("lt_q8_gemv_multi", h, L["wdown"].t.vp, xq, xd, B, self.xres.vp, self.x.vp, E, F,
                     LT_MULTI_RESID)
        call("lt_len_add_n", h, _vp(self.lens.ptr), 2 * B, 1, self.max_ctx)
        if mixed or B >= HEAD_GEMM_MIN_BATCH:
            call("lt_rmsnorm_quant_bm", h, self.x.vp, m.output_norm.vp, xq, xd, B, E, eps)
            call("lt_q8_gemm_t", h, self.head.t.vp, xq, xd, None, None, self.logits.vp, B, V, E)
        else:
            call("lt_rmsnorm_quant_rows", h, self.x.vp, m.output_norm.vp, xq, xd, B, E, eps)
            call("lt_q8_gemv_multi", h, m.output.t.vp, xq, xd, B, None, self.logits.vp, V, E, LT_MULTI_STORE)
        call("lt_argmax_rows_ws", h, self.logits.vp, B, V, self.toks.vp, self.hist.vp, self.hist_count.vp,
             self.hist_cap, self.am_ws.vp, self.am_ws.nbytes)

    def step(self, toks=None) -> None:
        """Eager step (toks=None: each sequence continues from its device token)."""
        self.check_room(1)
        if toks is not None:
            self.set_tokens(toks)
        self.enqueue_step()
        self.dev.sync()
        self.length = [n + 1 for n in self.length]

    def free(self) -> None:
        self.dev.sync()
        if self._prefill is not None:
            self._prefill.free()
        for t in [*self.k, *self.v, self.lens, self.toks, self.err, self.hist, self.hist_count, self.x, self.xres,
                  self.qkv, self.att, self.vbuf, self.xq, self.xd, self.vq, self.vd, self.logits, self.attn_ws,
                  self.am_ws]:
            if t is not None:
                t.free()


class BatchStepGraph:
    """The batched step captured once and replayed per token (all sequences advance)."""

    def __init__(self, plan: BatchDecodePlan):
        self.plan, self.dev = plan, plan.dev
        self.graph = ctypes.c_void_p()

    def capture(self) -> None:
        if self.graph.value:
            raise RuntimeError("BatchStepGraph.capture: already captured")
        call("lt_graph_begin", self.dev.handle)
        try:
            self.plan.enqueue_step()
        except Exception:
            g = ctypes.c_void_p()
            _lib.raw("lt_graph_end")(self.dev.handle, ctypes.byref(g))
            if g.value:
                _lib.raw("lt_graph_free")(g)
            raise
        call("lt_graph_end", self.dev.handle, ctypes.byref(self.graph))

    def replay(self) -> None:
        if not self.graph.value:
            raise RuntimeError("call capture() before replay")
        self.plan.check_room(1)
        call("lt_graph_launch", self.dev.handle, self.graph)
        self.plan.length = [n + 1 for n in self.plan.length]

    def replay_tokens(self, n: int) -> list[list[int]]:
        """n back-to-back replays; the generated ids of every sequence, read once at the end."""
        before = [len(h) for h in self.plan.history()]
        if max(before) + n > self.plan.hist_cap:
            raise ValueError(f"token history capacity {self.plan.hist_cap} exceeded")
        self.plan.check_room(n)
        for _ in range(n):
            self.replay()
        return [h[s:s + n] for h, s in zip(self.plan.history(), before)]

    def free(self) -> None:
        if self.graph.value:
            call("lt_graph_free", self.graph)
            self.graph = ctypes.c_void_p()


def batch_generate(model: ResidentModel, prompts, n_tokens: int, profile: Profile = PRODUCTION_PROFILE,
                   max_ctx: int | None = None, linear: str = "auto") -> list[list[int]]:
    """Greedy generation of n_tokens after each of len(prompts) prompts, decoded together:
    each prompt prefilled (batched GEMM), the first token its greedy argmax, then n_tokens - 1
    replays of the captured batched step.  Sequence b's tokens equal generate(model,
    prompts[b], n_tokens)."""
    prompts = [[int(t) for t in np.asarray(pr).reshape(-1)] for pr in prompts]
    if not prompts or any(not pr for pr in prompts):
        raise ValueError("batch_generate: every prompt needs at least one token")
    if n_tokens < 1:
        return [[] for _ in prompts]
    need = max(len(pr) for pr in prompts) + n_tokens - 1
    plan = BatchDecodePlan(model, len(prompts), profile, max_ctx=max(max_ctx or 0, need, 1), hist_cap=n_tokens,
                           linear=linear)
    gr = BatchStepGraph(plan)
    try:
        for b, pr in enumerate(prompts):
            plan.prefill(b, pr)
        out = [[t] for t in plan.read_tokens()]
        if n_tokens > 1:
            gr.capture()
            for o, more in zip(out, gr.replay_tokens(n_tokens - 1)):
                o.extend(more)
        return out
    finally:
        gr.free()
        plan.free()


def generate(model, input_ids, n_tokens: int, profile: Profile = PRODUCTION_PROFILE,
             batched_prefill: bool = True, max_ctx: int | None = None,
             sampling: dict | None = None) -> list[int]:
    """Generation of n_tokens after input_ids, the reference's decode loop
    (decode_fact.py:54-111 semantics; GraphRunner seed -> capture -> replay,
    dev_residency.py:1626-1818): the prompt is prefilled, the first token is its greedy
    argmax, and every further token comes from one replay of the captured step.
    sampling={temperature, top_k, top_p, seed} draws every generated token with the device
    sampler instead (DecodePlan.set_sampling, after the prompt: draw i of the sequence is
    Philox counter i).

    `model` is a ResidentModel or the path of a Q8_0 GGUF file (loaded and freed here)."""
    own = not isinstance(model, ResidentModel)
    m = ResidentModel.from_gguf(model, max_ctx=max_ctx or 1024) if own else model
    plan = gr = None
    try:
        ids = [int(t) for t in np.asarray(input_ids).reshape(-1)]
        if not ids:
            raise ValueError("generate: empty prompt")
        if n_tokens < 1:
            return []
        # the history records one entry per token through the step's argmax: the prompt's
        # (when it is fed token by token) and every generated one
        plan = DecodePlan(m, profile, max_ctx=max_ctx, hist_cap=len(ids) + n_tokens)
        if len(ids) + n_tokens - 1 > plan.max_ctx:
            raise ValueError(f"generate: {len(ids)} prompt + {n_tokens - 1} decode positions exceed "
                             f"the {plan.max_ctx}-position KV cache")
        gr = StepGraph(plan)
        gr.seed(ids, batched=batched_prefill and profile.numerics == "engine" and "wgu_il" in m.layers[0])
        if sampling:
            plan.set_sampling(**sampling)
            out = [plan.sample_current()]
        else:
            out = [plan.read_token()]
        if n_tokens > 1:
            gr.capture()
            out += gr.replay_tokens(n_tokens - 1)
        return out
    finally:
        if gr is not None:
            gr.free()
        if plan is not None:
            plan.free()
        if own:
            m.free()

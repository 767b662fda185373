"""ctypes binding of libllamatov_hip.so (the C ABI declared in include/llamatov_hip.h).

The reference binds the CUDA driver API the same way (ctypes, raw pointers, int return
codes; bpd/lib/fact_dispatch.py:36-72).  There is no fallback: if the HIP library is
missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_size_t, c_uint8, c_void_p
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("LT_HIP_LIB", _PKG / "libllamatov_hip.so"))

LT_KV_F32 = 0
LT_KV_F16 = 1
LT_GGML_VEC = 0
LT_GGML_LLAMAFILE = 1
LT_SAMPLE_MAX_K = 1024
LT_MULTI_STORE, LT_MULTI_RESID, LT_MULTI_SILU = 0, 1, 2

_P = c_void_p
# name -> (restype, argtypes)
_SIGS = {
    "lt_version": (c_int, []),
    "lt_last_error": (c_int, [ctypes.c_char_p, c_size_t]),
    "lt_device_count": (c_int, [POINTER(c_int)]),
    "lt_init": (c_int, [c_int, POINTER(c_void_p)]),
    "lt_free_ctx": (c_int, [_P]),
    "lt_malloc": (c_int, [_P, POINTER(c_void_p), c_size_t]),
    "lt_free": (c_int, [_P, _P]),
    "lt_memcpy_h2d": (c_int, [_P, _P, _P, c_size_t]),
    "lt_memcpy_d2h": (c_int, [_P, _P, _P, c_size_t]),
    "lt_memcpy_d2d": (c_int, [_P, _P, _P, c_size_t]),
    "lt_fill_u8": (c_int, [_P, _P, c_uint8, c_size_t]),
    "lt_sync": (c_int, [_P]),
    "lt_quant_q8": (c_int, [_P, _P, _P, _P, c_int]),
    "lt_silu_mul_quant": (c_int, [_P, _P, _P, _P, _P, c_int]),
    "lt_silu_mul": (c_int, [_P, _P, _P, _P, c_int]),
    "lt_add": (c_int, [_P, _P, _P, _P, c_int]),
    "lt_rope_append_seqs": (c_int, [_P, _P, c_int, c_int, _P, c_int, c_int, c_int, _P, _P, _P, c_int, c_int]),
    "lt_attn_decode_rows": (c_int, [_P, _P, c_int, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_float, c_int,
                                    c_int, c_int, _P, c_size_t]),
    "lt_attn_decode_rows_q8": (c_int, [_P, _P, c_int, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_float,
                                       c_int, c_int, c_int, _P, c_size_t]),
    "lt_attn_decode_rows_q8_bm": (c_int, [_P, _P, c_int, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_float,
                                          c_int, c_int]),
    "lt_argmax_rows": (c_int, [_P, _P, c_int, c_int, _P, _P, _P, c_int]),
    "lt_argmax_rows_workspace_size": (c_size_t, [c_int]),
    "lt_argmax_rows_ws": (c_int, [_P, _P, c_int, c_int, _P, _P, _P, c_int, _P, c_size_t]),
    "lt_rmsnorm_quant_rows": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_float]),
    "lt_q8_gemv_multi": (c_int, [_P, _P, _P, _P, c_int, _P, _P, c_int, c_int, c_int]),
    "lt_q8_gemv_multi_rope": (c_int, [_P, _P, _P, _P, c_int, _P, _P, c_int, c_int, _P, c_int, c_int, c_int, _P, _P,
                                      _P, c_int, c_int]),
    "lt_sample_workspace_size": (c_size_t, [c_int]),
    "lt_sample": (c_int, [_P, _P, c_int, _P, _P, _P, _P, c_int, _P, c_size_t]),
    "lt_quant_q8_ggml": (c_int, [_P, _P, _P, _P, c_int]),
    "lt_quant_q8_0_ggml": (c_int, [_P, _P, _P, c_int]),
    "lt_q8_gemv_ggml": (c_int, [_P, _P, _P, _P, _P, _P, c_int, c_int, c_int]),
    "lt_qmatmul_q8_0_workspace_size": (c_size_t, [c_int, c_int]),
    "lt_qmatmul_q8_0_ggml": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, _P, c_size_t]),
    "lt_qmatmul_q8_0_llamafile": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, _P, c_size_t]),
    "lt_rmsnorm": (c_int, [_P, _P, _P, _P, c_int, c_int, c_float]),
    "lt_rmsnorm_quant": (c_int, [_P, _P, _P, _P, _P, c_int, c_float]),
    "lt_q8_gemv": (c_int, [_P, _P, _P, _P, _P, _P, c_int, c_int]),
    "lt_q8_gemv_isums": (c_int, [_P, _P, _P, _P, c_int, c_int]),
    "lt_rope_qk": (c_int, [_P, _P, _P, c_int, c_int, _P]),
    "lt_rope_freqs": (c_int, [c_int, c_float, _P]),
    "lt_kv_append_incr": (c_int, [_P, _P, _P, _P, _P, _P, c_int, c_int, c_int]),
    "lt_attn_decode": (c_int, [_P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_float,
                               c_int, c_int, c_int, _P, c_size_t]),
    "lt_attn_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int]),
    "lt_attn_decode_noalloc": (c_int, [_P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_float,
                                       c_int, c_int, c_int]),
    "lt_argmax": (c_int, [_P, _P, c_int, _P, _P, c_size_t]),
    "lt_argmax_workspace_size": (c_size_t, []),
    "lt_argmax_record": (c_int, [_P, _P, c_int, _P, _P, _P, c_int, _P, c_size_t]),
    "lt_embed_q8": (c_int, [_P, _P, _P, _P, c_int, c_int, _P]),
    "lt_q8_gemv_rms": (c_int, [_P, _P, _P, c_float, _P, _P, _P, c_int, c_int]),
    "lt_q8_gemv_embed_rms": (c_int, [_P, _P, _P, c_int, _P, _P, _P, c_float, _P, _P, _P, c_int, c_int]),
    "lt_q8_gemv_quant": (c_int, [_P, _P, _P, _P, _P, c_int, c_int]),
    "lt_q8_gemv_attn_out": (c_int, [_P, _P, _P, _P, c_size_t, c_int, c_int, c_int, _P, _P, _P, c_int, c_int,
                                    _P, c_int]),
    "lt_q8_gemv_rms_silu": (c_int, [_P, _P, _P, c_float, _P, _P, _P, c_int, c_int]),
    "lt_q8_gemv_rms_rope_kv": (c_int, [_P, _P, _P, _P, c_int, _P, _P, _P, c_float, _P, _P, _P, c_int, _P, _P, _P,
                                       _P, c_int, c_int, c_int, c_int, c_int]),
    "lt_attn_o_max_len": (c_int, [c_int, c_int, c_int, c_int]),
    "lt_q8_gemv_attn_o": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_float, c_int, c_int, _P, _P, _P,
                                  c_int]),
    "lt_q8_gemv_rms_silu_len": (c_int, [_P, _P, _P, c_float, _P, _P, _P, c_int, c_int, _P, c_int]),
    "lt_q8_gemv_rms_swiglu": (c_int, [_P, _P, _P, c_float, _P, _P, c_int, c_int]),
    "lt_q8_gemv_rms_argmax": (c_int, [_P, _P, _P, c_float, _P, _P, c_int, c_int, _P, _P, _P, c_int,
                                      _P, c_size_t]),
    "lt_q8_gemv_argmax_workspace_size": (c_size_t, [c_int]),
    "lt_q8_to_planar": (c_int, [_P, _P, _P, c_int, c_int]),
    "lt_decode_step_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "lt_decode_step_max_len": (c_int, [_P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "lt_decode_step": (c_int, [_P, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_float, _P, _P, c_int,
                               c_int, _P, _P, c_int, _P, _P, _P, _P, c_size_t]),
    "lt_attn_step": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_float, c_int, c_int,
                             c_int, _P, c_size_t]),
    "lt_q8_gemm": (c_int, [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int]),
    "lt_q8_gemm_silu": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int]),
    "lt_q8_tiles_bytes": (c_size_t, [c_int, c_int]),
    "lt_q8_tiles": (c_int, [_P, _P, _P, c_int, c_int]),
    "lt_quant_q8_bm": (c_int, [_P, _P, _P, _P, c_int, c_int]),
    "lt_rmsnorm_quant_bm": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_float]),
    "lt_q8_gemm_t": (c_int, [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int]),
    "lt_q8_gemm_silu_t": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int]),
    "lt_q8_gemm_silu_quant_t": (c_int, [_P, _P, _P, _P, _P, _P, c_int, c_int, c_int]),
    "lt_q8_tiles_rope": (c_int, [_P, _P, _P, c_int, c_int, c_int, c_int, c_int]),
    "lt_q8_gemm_rope_t": (c_int, [_P, _P, _P, _P, c_int, _P, _P, c_int, c_int, _P, c_int, c_int, c_int, _P, _P, _P,
                                  c_int, c_int]),
    "lt_rope_batch": (c_int, [_P, _P, c_int, c_int, _P, c_int, c_int, _P]),
    "lt_kv_append_batch": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, c_int, _P, c_int, c_int, c_int]),
    "lt_len_add": (c_int, [_P, _P, c_int, c_int]),
    "lt_rope_append_batch": (c_int, [_P, _P, c_int, c_int, _P, c_int, c_int, c_int, _P, _P, _P, c_int, c_int]),
    "lt_len_add_n": (c_int, [_P, _P, c_int, c_int, c_int]),
    "lt_attn_prefill": (c_int, [_P, _P, c_int, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_float, c_int,
                                c_int, c_int, _P, c_size_t]),
    "lt_embed_q8_batch": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, _P]),
    "lt_selftest_numerics": (c_int, [_P, _P]),
    "lt_graph_begin": (c_int, [_P]),
    "lt_graph_end": (c_int, [_P, POINTER(c_void_p)]),
    "lt_graph_launch": (c_int, [_P, _P]),
    "lt_graph_free": (c_int, [_P]),
    "lt_event_create": (c_int, [_P, POINTER(c_void_p)]),
    "lt_event_record": (c_int, [_P, _P]),
    "lt_event_elapsed_ms": (c_int, [_P, _P, POINTER(c_float)]),
    "lt_event_destroy": (c_int, [_P]),
}
# the planar-layout twins take their namesakes' arguments
for _n in ("lt_q8_gemv", "lt_q8_gemv_rms", "lt_q8_gemv_embed_rms", "lt_q8_gemv_attn_out", "lt_q8_gemv_rms_silu",
           "lt_q8_gemv_rms_argmax"):
    _SIGS[_n + "_pl"] = _SIGS[_n]


class LtError(RuntimeError):
    """A non-zero return code from the C ABI, with lt_last_error()'s message."""

    def __init__(self, fn: str, rc: int, msg: str):
        super().__init__(f"{fn} -> {rc}: {msg}")
        self.fn, self.rc, self.msg = fn, rc, msg


_lib = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load the HIP library once; raise loudly if it is absent (no CPU fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise ImportError(
            f"{p} is missing: build it with `python -m llamatov_amd.build` "
            "(hipcc --offload-arch=gfx950). The decode path has no CPU fallback.")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return list(_SIGS)


def last_error() -> str:
    buf = ctypes.create_string_buffer(1024)
    load().lt_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def call(name: str, *args) -> int:
    """Call an int-returning entry point and raise LtError on a non-zero code."""
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise LtError(name, rc, last_error())
    return rc


def raw(name: str):
    return getattr(load(), name)

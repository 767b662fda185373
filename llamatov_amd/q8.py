"""Host-side GGUF Q8_0 codec (numpy).

A Q8_0 block is 34 bytes: an fp16 scale d (little endian) followed by 32 int8 values;
the row-major [N][K/32] block array is the GGUF tensor layout (ne0 = K, ne1 = N).

quantize_rows follows the engine's weight quantizer, fact_dispatch._quantize_weight_q8_0
(bpd/lib/fact_dispatch.py:255-282): per block d = fp16(amax/127) (1.0 if amax == 0),
q = clip(rint(w / float32(d16)), -127, 127).  For blocks produced by this quantizer the
reference's dequant -> requant residency round trip (dequant bpd/llamatov_run.py:184-207,
requant fact_dispatch.py:255-282) returns the same d16 and q, so uploading these blocks
verbatim is value-identical to the reference's split int8 + fp16 residency.
"""
from __future__ import annotations

import numpy as np

QK = 32
BLOCK_BYTES = 34


def row_bytes(K: int) -> int:
    if K % QK:
        raise ValueError(f"K={K} is not a multiple of {QK}")
    return K // QK * BLOCK_BYTES


def quantize_rows(W: np.ndarray, chunk_rows: int = 8192) -> np.ndarray:
    """fp32 [N, K] -> uint8 [N, K/32*34] GGUF Q8_0 blocks."""
    W = np.asarray(W, dtype=np.float32)
    if W.ndim != 2:
        raise ValueError("quantize_rows expects a 2-D matrix")
    N, K = W.shape
    nb = K // QK
    out = np.empty((N, nb * BLOCK_BYTES), dtype=np.uint8)
    for r0 in range(0, N, chunk_rows):
        blk = W[r0:r0 + chunk_rows].reshape(-1, nb, QK)
        amax = np.abs(blk).max(axis=2)
        d = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
        d16 = d.astype(np.float16)
        q = np.rint(blk / d16.astype(np.float32)[..., None])
        q = np.clip(q, -127, 127).astype(np.int8)
        o = out[r0:r0 + chunk_rows].reshape(-1, nb, BLOCK_BYTES)
        o[..., 0:2] = d16.view(np.uint8).reshape(-1, nb, 2)
        o[..., 2:] = q.view(np.uint8)
    return out


def dequantize_rows(B: np.ndarray, K: int) -> np.ndarray:
    """uint8 [N, K/32*34] -> fp32 [N, K] (y = q * d, exact)."""
    B = np.asarray(B, dtype=np.uint8)
    nb = K // QK
    blk = B.reshape(B.shape[0], nb, BLOCK_BYTES)
    d = blk[..., 0:2].copy().view(np.float16).astype(np.float32)
    q = blk[..., 2:].view(np.int8).astype(np.float32)
    return (q * d).reshape(B.shape[0], K)


def split_blocks(B: np.ndarray, K: int) -> tuple[np.ndarray, np.ndarray]:
    """Blocks -> (int8 quants [N, K], fp16 scale bits [N, K/32])."""
    nb = K // QK
    blk = np.asarray(B, dtype=np.uint8).reshape(-1, nb, BLOCK_BYTES)
    d = blk[..., 0:2].copy().view(np.uint16).reshape(-1, nb)
    q = blk[..., 2:].copy().view(np.int8).reshape(-1, K)
    return q, d


def join_blocks(q: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    """(int8 [N, K], uint16 [N, K/32]) -> blocks uint8 [N, K/32*34]."""
    q = np.asarray(q, dtype=np.int8)
    N, K = q.shape
    nb = K // QK
    out = np.empty((N, nb, BLOCK_BYTES), dtype=np.uint8)
    out[..., 0:2] = np.asarray(d_bits, dtype=np.uint16).reshape(N, nb, 1).view(np.uint8)
    out[..., 2:] = q.reshape(N, nb, QK).view(np.uint8)
    return out.reshape(N, nb * BLOCK_BYTES)

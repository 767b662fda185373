"""GGUF v2/v3 files: a memory-mapped reader, a writer, and the model loader of the decode path.

Reader.  `parse_gguf(path) -> (md, ts, data_offset)` returns what the reference's parser
returns (bpd/llamatov_run.py:9-40): the metadata dict, `ts[name] = (dims, ggml_type,
relative_offset)` with dims ne0-first, and the absolute offset of the tensor data, rounded up
to `general.alignment` (default 32).  Differences, all in what the reference does not check:
- metadata values of every GGUF type are decoded; the reference's value reader
  (llamatov_run.py:31-40) returns None for the 8/16-bit integers, int64 and float64;
- a bad magic, an unknown version, a truncated file, an unknown value type, a tensor that
  lies outside the file or whose size is not whole blocks raise GGUFError; the reference
  asserts the magic only.

`lt(path, data_offset, info)` is the reference's tensor loader (llamatov_run.py:497-511) for
F32, F16, Q4_0, Q5_0 and Q8_0, returning float32 numpy in the reference's orientation
(2-D tensors as [ne0, ne1], the transpose of the stored [ne1][ne0] rows).  The other types
the reference dequantizes (K-quants) raise GGUFError here: the decode path reads Q8_0 files.

Loader.  `load_q8_model(path)` builds a ModelConfig from the metadata the way the reference's
decode loader does (bpd/decode_fact.py:39-51, defaults of the Qwen2.5-0.5B model) and
returns the GGUF-named tensors ResidentModel uploads:
- Q8_0 weights as zero-copy views of the mapped file, blocks [N][K/32] x 34 B.  The
  reference dequantizes them (dq8_0, llamatov_run.py:184-207) and quantizes them again into
  its device layout (fact_dispatch._quantize_weight_q8_0, bpd/lib/fact_dispatch.py:255-282).
  For a block with a finite scale d > 0 whose largest |q| is 127 - every block ggml writes,
  since its quantizer maps the block's largest magnitude to 127 - that round trip returns the
  same d and q: q*d is exact in fp32, 127*d / 127 = d exactly, and q*d / d = q.  Other
  blocks are replaced by the round trip's result (canonical_q8_0), so the device holds
  exactly what the reference computes with, for any Q8_0 file;
- F32/F16/Q4_0/Q5_0 weight matrices are dequantized and quantized with the same weight
  quantizer, which is what the reference does with every weight;
- norm weights and biases as float32 vectors.
"""
from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass

import numpy as np

from . import q8
from .model import ModelConfig, weight_specs

GGUF_MAGIC = 0x46554747            # b"GGUF" read as a little-endian uint32
GGUF_VERSIONS = (2, 3)             # v1 used 32-bit counts and lengths
DEFAULT_ALIGNMENT = 32

# Metadata value types (GGUF specification).
GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16, GGUF_UINT32, GGUF_INT32, GGUF_FLOAT32, \
    GGUF_BOOL, GGUF_STRING, GGUF_ARRAY, GGUF_UINT64, GGUF_INT64, GGUF_FLOAT64 = range(13)

_SCALAR = {GGUF_UINT8: "<u1", GGUF_INT8: "<i1", GGUF_UINT16: "<u2", GGUF_INT16: "<i2",
           GGUF_UINT32: "<u4", GGUF_INT32: "<i4", GGUF_FLOAT32: "<f4", GGUF_BOOL: "<u1",
           GGUF_UINT64: "<u8", GGUF_INT64: "<i8", GGUF_FLOAT64: "<f8"}
_STRUCT = {GGUF_UINT8: "<B", GGUF_INT8: "<b", GGUF_UINT16: "<H", GGUF_INT16: "<h",
           GGUF_UINT32: "<I", GGUF_INT32: "<i", GGUF_FLOAT32: "<f", GGUF_BOOL: "<B",
           GGUF_UINT64: "<Q", GGUF_INT64: "<q", GGUF_FLOAT64: "<d"}

# ggml tensor types read here: (block elements, block bytes).
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q5_0, GGML_Q8_0 = 0, 1, 2, 6, 8
GGML_TYPE_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0",
                   9: "Q8_1", 10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K",
                   15: "Q8_K", 30: "BF16"}
_BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q4_0: (32, 18), GGML_Q5_0: (32, 22),
          GGML_Q8_0: (32, 34)}


class GGUFError(ValueError):
    """A file that is not a readable GGUF, or a tensor this loader cannot use."""


def type_name(t: int) -> str:
    return GGML_TYPE_NAMES.get(t, f"type{t}")


def tensor_nbytes(dims, ggml_type: int) -> int:
    """Bytes of a tensor of `dims` (ne0 first) stored as `ggml_type`."""
    if ggml_type not in _BLOCK:
        raise GGUFError(f"tensor type {type_name(ggml_type)} is not supported by this loader")
    be, bb = _BLOCK[ggml_type]
    n = 1
    for d in dims:
        n *= int(d)
    if dims and int(dims[0]) % be:
        raise GGUFError(f"ne0={dims[0]} is not a multiple of the {type_name(ggml_type)} block ({be})")
    return n // be * bb


# ----------------------------------------------------------------------------------
# Reader
# ----------------------------------------------------------------------------------
class _Cursor:
    """Bounds-checked little-endian reads from a byte buffer."""

    def __init__(self, buf, size: int):
        self.buf, self.size, self.pos = buf, size, 0

    def take(self, n: int) -> int:
        p = self.pos
        if n < 0 or p + n > self.size:
            raise GGUFError(f"file is short: needs {p + n} bytes, has {self.size}")
        self.pos = p + n
        return p

    def unpack(self, fmt: str):
        p = self.take(struct.calcsize(fmt))
        return struct.unpack_from(fmt, self.buf, p)[0]

    def string(self) -> str:
        n = self.unpack("<Q")
        p = self.take(n)
        try:
            return bytes(self.buf[p:p + n]).decode("utf-8")
        except UnicodeDecodeError as e:
            raise GGUFError(f"string at byte {p} is not UTF-8: {e}") from None

    def value(self, vt: int):
        if vt == GGUF_STRING:
            return self.string()
        if vt == GGUF_ARRAY:
            at = self.unpack("<I")
            n = self.unpack("<Q")
            if at in _SCALAR:
                dt = np.dtype(_SCALAR[at])
                p = self.take(n * dt.itemsize)
                a = np.frombuffer(self.buf, dtype=dt, count=n, offset=p)
                return [bool(v) for v in a] if at == GGUF_BOOL else a.tolist()
            if at in (GGUF_STRING, GGUF_ARRAY):
                return [self.value(at) for _ in range(n)]
            raise GGUFError(f"unknown array element type {at}")
        if vt in _SCALAR:
            v = self.unpack(_STRUCT[vt])
            return bool(v) if vt == GGUF_BOOL else v
        raise GGUFError(f"unknown metadata value type {vt}")


@dataclass
class TensorInfo:
    name: str
    dims: tuple            # ne0 first, as stored
    ggml_type: int
    offset: int            # relative to the data section
    nbytes: int

    @property
    def shape(self) -> tuple:
        """Row-major shape of the stored data (dims reversed)."""
        return tuple(self.dims[::-1])


class GGUFReader:
    """A GGUF file mapped read-only.  `md` metadata, `tensors` name -> TensorInfo (file
    order), `data_offset` absolute start of the tensor data.  Tensor accessors return views
    of the mapping (no copy); they stay valid while the reader is open."""

    def __init__(self, path):
        self.path = os.fspath(path)
        with open(self.path, "rb") as f:
            size = os.fstat(f.fileno()).st_size
            if size < 24:
                raise GGUFError(f"{self.path}: file is short ({size} bytes) for a GGUF header")
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        self.size = size
        try:
            self._parse()
        except Exception:
            self.close()
            raise
        self.bytes = np.frombuffer(self._mm, dtype=np.uint8)

    def _parse(self) -> None:
        c = _Cursor(self._mm, self.size)
        magic = c.unpack("<I")
        if magic != GGUF_MAGIC:
            raise GGUFError(f"{self.path}: bad magic {magic:#010x} (not a GGUF file)")
        self.version = c.unpack("<I")
        if self.version not in GGUF_VERSIONS:
            raise GGUFError(f"{self.path}: GGUF version {self.version} is not supported "
                            f"(supported: {GGUF_VERSIONS})")
        nt = c.unpack("<Q")
        nkv = c.unpack("<Q")
        md = {}
        for _ in range(nkv):
            k = c.string()
            md[k] = c.value(c.unpack("<I"))
        infos = []
        for _ in range(nt):
            name = c.string()
            nd = c.unpack("<I")
            if nd > 8:
                raise GGUFError(f"tensor {name!r}: {nd} dimensions")
            dims = tuple(c.unpack("<Q") for _ in range(nd))
            tt = c.unpack("<I")
            off = c.unpack("<Q")
            infos.append((name, dims, tt, off))
        al = md.get("general.alignment", DEFAULT_ALIGNMENT)
        if not isinstance(al, int) or al <= 0:
            raise GGUFError(f"general.alignment={al!r}")
        self.alignment = al
        self.data_offset = (c.pos + al - 1) // al * al
        self.md = md
        self.tensors: dict[str, TensorInfo] = {}
        for name, dims, tt, off in infos:
            if name in self.tensors:
                raise GGUFError(f"tensor {name!r} appears twice")
            nbytes = tensor_nbytes(dims, tt) if tt in _BLOCK else None
            if nbytes is not None and self.data_offset + off + nbytes > self.size:
                raise GGUFError(f"tensor {name!r} ({type_name(tt)} {list(dims)}) ends at byte "
                                f"{self.data_offset + off + nbytes}, past the file end {self.size}")
            self.tensors[name] = TensorInfo(name, dims, tt, off, nbytes)

    # -- access --------------------------------------------------------------------
    def info(self, name: str) -> TensorInfo:
        try:
            return self.tensors[name]
        except KeyError:
            raise GGUFError(f"{self.path}: no tensor {name!r}") from None

    def raw(self, name: str) -> np.ndarray:
        """The tensor's stored bytes (uint8 view)."""
        ti = self.info(name)
        if ti.nbytes is None:
            raise GGUFError(f"tensor {name!r}: type {type_name(ti.ggml_type)} is not supported")
        p = self.data_offset + ti.offset
        return self.bytes[p:p + ti.nbytes]

    def q8_blocks(self, name: str) -> np.ndarray:
        """A Q8_0 matrix as uint8 [N][K/32*34] (N = ne1 rows of K = ne0), a view."""
        ti = self.info(name)
        if ti.ggml_type != GGML_Q8_0:
            raise GGUFError(f"tensor {name!r} is {type_name(ti.ggml_type)}, not Q8_0")
        if len(ti.dims) != 2:
            raise GGUFError(f"tensor {name!r}: Q8_0 matrix expected, dims {list(ti.dims)}")
        K, N = ti.dims
        return self.raw(name).reshape(N, q8.row_bytes(K))

    def dequantize(self, name: str) -> np.ndarray:
        """float32 in the stored row-major shape (dims reversed)."""
        ti = self.info(name)
        return dequantize_bytes(self.raw(name), ti.ggml_type).reshape(ti.shape)

    def close(self) -> None:
        self.bytes = None
        if getattr(self, "_mm", None) is not None:
            try:
                self._mm.close()
            except BufferError:
                pass              # views still alive; the mapping ends with them
            self._mm = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def parse_gguf(path):
    """(md, ts, data_offset) as the reference parser returns them (llamatov_run.py:9-40):
    ts[name] = (dims list ne0-first, ggml type, offset relative to data_offset)."""
    r = GGUFReader(path)
    try:
        ts = {n: (list(t.dims), t.ggml_type, t.offset) for n, t in r.tensors.items()}
        return r.md, ts, r.data_offset
    finally:
        r.close()


# ----------------------------------------------------------------------------------
# Dequantization (ggml block formats)
# ----------------------------------------------------------------------------------
def _f16_scales(bl: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(bl[:, 0:2]).view(np.float16).astype(np.float32).reshape(-1)


def dequantize_bytes(raw: np.ndarray, ggml_type: int) -> np.ndarray:
    """Stored bytes -> flat float32, element order as stored.
    Q8_0: y[32b + j] = q_j * d (dq8_0, llamatov_run.py:184-207).
    Q4_0: 18-byte blocks, d then 16 bytes; byte j's low nibble is element j and its high
      nibble element j + 16; y = (nibble - 8) * d (dq4_0).
    Q5_0: 22-byte blocks, d, a little-endian uint32 qh whose bit i is element i's fifth bit,
      then the Q4_0 nibbles; y = ((nibble | bit << 4) - 16) * d (dq5_0, llamatov_run.py:156-183).
    Each product is one fp32 multiply of exact operands."""
    raw = np.asarray(raw, dtype=np.uint8)
    if ggml_type == GGML_F32:
        return raw.view("<f4").astype(np.float32)
    if ggml_type == GGML_F16:
        return raw.view("<f2").astype(np.float32)
    if ggml_type not in _BLOCK:
        raise GGUFError(f"tensor type {type_name(ggml_type)} is not supported by this loader")
    _, bb = _BLOCK[ggml_type]
    bl = raw.reshape(-1, bb)
    d = _f16_scales(bl)
    if ggml_type == GGML_Q8_0:
        q = bl[:, 2:].view(np.int8).astype(np.float32)
    else:
        qs = bl[:, bb - 16:]
        nib = np.concatenate([qs & 0x0F, qs >> 4], axis=1).astype(np.int32)
        if ggml_type == GGML_Q4_0:
            q = (nib - 8).astype(np.float32)
        else:
            qh = np.ascontiguousarray(bl[:, 2:6]).view("<u4").reshape(-1, 1)
            hi = ((qh >> np.arange(32, dtype=np.uint32)) & 1).astype(np.int32)
            q = ((nib | (hi << 4)) - 16).astype(np.float32)
    return (d[:, None] * q).reshape(-1)


def lt(path, data_offset: int, info) -> np.ndarray:
    """The reference's tensor loader (llamatov_run.py:497-511) for F32/F16/Q4_0/Q5_0/Q8_0:
    float32 with 2-D tensors as [ne0, ne1]; 3-D Q4_0/Q5_0 tensors as [ne0, ne1, ne2]
    (_finalize_dequant, llamatov_run.py:46-60); every other case reshaped to dims as listed."""
    dims, tt, ro = info
    dims = [int(d) for d in dims]
    n = tensor_nbytes(dims, tt)
    with open(path, "rb") as f:
        f.seek(data_offset + ro)
        raw = np.frombuffer(f.read(n), dtype=np.uint8)
    if raw.size != n:
        raise GGUFError(f"{path}: tensor at {data_offset + ro} is cut short")
    flat = dequantize_bytes(raw, tt)
    if len(dims) == 2:
        return np.ascontiguousarray(flat.reshape(dims[::-1]).T)
    if len(dims) == 3 and tt in (GGML_Q4_0, GGML_Q5_0):
        return np.ascontiguousarray(flat.reshape(dims[::-1]).transpose(2, 1, 0))
    return flat.reshape(dims).copy()


# ----------------------------------------------------------------------------------
# Q8_0 canonical form
# ----------------------------------------------------------------------------------
def q8_block_is_canonical(blocks: np.ndarray) -> np.ndarray:
    """Per block of uint8 [..., 34]: True where the block has a finite scale d > 0 (fp16 bits
    0x0001..0x7BFF) and max |q| == 127.  Such a block is left unchanged by the reference's
    dequant -> requant round trip (q*d -> d' = fp16(amax/127) -> q' = clip(rint(x/d'), +-127)).
    The test is sufficient, not necessary: with a subnormal d, fp16(126*d/127) can round back
    to d, so some blocks that fail it also come back unchanged."""
    bl = np.asarray(blocks, dtype=np.uint8)
    dbits = bl[..., 0].astype(np.uint16) | (bl[..., 1].astype(np.uint16) << 8)
    q = bl[..., 2:].view(np.int8)
    qmin = q.min(axis=-1)
    qmax = q.max(axis=-1)
    return (dbits > 0) & (dbits < 0x7C00) & (qmin >= -127) & ((qmax == 127) | (qmin == -127))


def canonical_q8_0(blocks: np.ndarray, name: str = "tensor", chunk_rows: int = 4096):
    """Q8_0 rows uint8 [N, K/32*34] -> (rows, n_changed): every block as the reference's
    residency holds it, i.e. after dequantizing (y = q*d) and quantizing with the weight
    quantizer.  Blocks that pass q8_block_is_canonical are kept without computing the round
    trip; the rest are recomputed.  When no block changes the input is returned as given
    (a view of a mapped file stays a view).  A block with a non-finite scale, or one whose
    re-quantized scale overflows fp16 (q = -128 with d near the fp16 maximum), raises
    GGUFError: the reference would compute with inf/NaN there."""
    N, rb = blocks.shape
    nb = rb // q8.BLOCK_BYTES
    out = blocks
    changed = 0
    for r0 in range(0, N, chunk_rows):
        part = blocks[r0:r0 + chunk_rows].reshape(-1, nb, q8.BLOCK_BYTES)
        ok = q8_block_is_canonical(part)
        if ok.all():
            continue
        bad_rows, bad_blocks = np.nonzero(~ok)
        sel = part[bad_rows, bad_blocks]
        dbits = sel[:, 0].astype(np.uint16) | (sel[:, 1].astype(np.uint16) << 8)
        nonfinite = (dbits & 0x7C00) == 0x7C00
        if nonfinite.any():
            i = int(np.argmax(nonfinite))
            raise GGUFError(f"{name}: row {r0 + int(bad_rows[i])} block {int(bad_blocks[i])} "
                            f"has a non-finite scale (fp16 bits {int(dbits[i]):#06x})")
        x = dequantize_bytes(sel.reshape(-1), GGML_Q8_0).reshape(-1, q8.QK)
        with np.errstate(over="ignore"):
            fixed = q8.quantize_rows(x).reshape(-1, q8.BLOCK_BYTES)
        fbits = fixed[:, 0].astype(np.uint16) | (fixed[:, 1].astype(np.uint16) << 8)
        over = (fbits & 0x7C00) == 0x7C00
        if over.any():
            i = int(np.argmax(over))
            raise GGUFError(f"{name}: row {r0 + int(bad_rows[i])} block {int(bad_blocks[i])}: "
                            f"amax/127 of its values exceeds the fp16 range")
        diff = (fixed != sel).any(axis=1)
        if not diff.any():
            continue
        if out is blocks:
            out = np.array(blocks, copy=True)
        dst = out[r0:r0 + chunk_rows].reshape(-1, nb, q8.BLOCK_BYTES)
        dst[bad_rows[diff], bad_blocks[diff]] = fixed[diff]
        changed += int(diff.sum())
    return out, changed


# ----------------------------------------------------------------------------------
# Writer
# ----------------------------------------------------------------------------------
def _infer_type(v) -> int:
    if isinstance(v, bool):
        return GGUF_BOOL
    if isinstance(v, int):
        if 0 <= v < 2 ** 32:
            return GGUF_UINT32
        if -2 ** 31 <= v < 0:
            return GGUF_INT32
        return GGUF_UINT64 if v >= 0 else GGUF_INT64
    if isinstance(v, float):
        return GGUF_FLOAT32
    if isinstance(v, str):
        return GGUF_STRING
    if isinstance(v, (list, tuple)):
        return GGUF_ARRAY
    raise GGUFError(f"cannot infer a GGUF type for {type(v).__name__}")


def _pack_value(vt: int, v, out: list, elem_type: int | None = None) -> None:
    if vt == GGUF_STRING:
        b = v.encode("utf-8")
        out.append(struct.pack("<Q", len(b)) + b)
    elif vt == GGUF_ARRAY:
        items = list(v)
        at = elem_type if elem_type is not None else (_infer_type(items[0]) if items else GGUF_UINT32)
        if at == GGUF_ARRAY:
            raise GGUFError("nested arrays need explicit element types")
        out.append(struct.pack("<IQ", at, len(items)))
        if at in _SCALAR:
            out.append(np.asarray(items, dtype=_SCALAR[at]).tobytes())
        else:
            for it in items:
                _pack_value(at, it, out)
    elif vt in _SCALAR:
        out.append(np.asarray([v], dtype=_SCALAR[vt]).tobytes())
    else:
        raise GGUFError(f"unknown metadata value type {vt}")


def write_gguf(path, metadata: dict, tensors: list, alignment: int = DEFAULT_ALIGNMENT,
               version: int = 3) -> None:
    """Write a GGUF file.
    metadata: key -> value, or key -> (value_type, value), or for arrays
      key -> (GGUF_ARRAY, element_type, values); untyped ints are written as uint32 (int32 if
      negative), floats as float32.  general.alignment is added when not the default.
    tensors: (name, dims ne0-first, ggml_type, data) with data the stored bytes (any array
      whose bytes are the tensor), in file order."""
    md = dict(metadata)
    if alignment != DEFAULT_ALIGNMENT:
        md["general.alignment"] = (GGUF_UINT32, alignment)
    parts = [struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(md))]
    for k, v in md.items():
        kb = k.encode("utf-8")
        parts.append(struct.pack("<Q", len(kb)) + kb)
        if isinstance(v, tuple) and len(v) == 3 and v[0] == GGUF_ARRAY:
            parts.append(struct.pack("<I", GGUF_ARRAY))
            _pack_value(GGUF_ARRAY, v[2], parts, elem_type=v[1])
        elif isinstance(v, tuple) and len(v) == 2 and isinstance(v[0], int) and not isinstance(v[0], bool):
            parts.append(struct.pack("<I", v[0]))
            _pack_value(v[0], v[1], parts)
        else:
            vt = _infer_type(v)
            parts.append(struct.pack("<I", vt))
            _pack_value(vt, v, parts)
    off = 0
    blobs = []
    for name, dims, tt, data in tensors:
        b = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        want = tensor_nbytes(dims, tt)
        if b.size != want:
            raise GGUFError(f"tensor {name!r}: {b.size} bytes given, {type_name(tt)} "
                            f"{list(dims)} needs {want}")
        nb = name.encode("utf-8")
        parts.append(struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims)))
        parts.append(struct.pack(f"<{len(dims)}Q", *[int(d) for d in dims]) if dims else b"")
        parts.append(struct.pack("<IQ", tt, off))
        blobs.append((off, b))
        off = (off + b.size + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        head = b"".join(parts)
        f.write(head)
        f.write(b"\0" * ((-len(head)) % alignment))
        pos = 0
        for o, b in blobs:
            f.write(b"\0" * (o - pos))
            f.write(b.tobytes())
            pos = o + b.size


# ----------------------------------------------------------------------------------
# Model loader (GGUF -> ModelConfig + GGUF-named tensors for ResidentModel)
# ----------------------------------------------------------------------------------
def config_from_gguf(md: dict, tensors: dict, name: str | None = None, max_ctx: int = 1024) -> ModelConfig:
    """ModelConfig from GGUF metadata, with the reference decode loader's defaults
    (decode_fact.load_model, bpd/decode_fact.py:39-51: 24 layers, 14 heads, n_embd 896,
    theta 1e6, eps 1e-6, n_head_kv = n_head).  n_ff and the vocabulary come from the tensor
    shapes; the lm_head is tied when output.weight is absent (dev_residency.py:1057); q/k/v
    biases are used when present.  The engine takes head_dim = n_embd / n_head
    (dev_residency.py:1337): a file declaring another key_length is refused."""
    arch = md.get("general.architecture", "llama")
    g = lambda k, d: md.get(f"{arch}.{k}", d)
    n_head = int(g("attention.head_count", 14))
    E = int(g("embedding_length", 896))
    if "token_embd.weight" not in tensors:
        raise GGUFError("no token_embd.weight tensor")
    te = tensors["token_embd.weight"]
    dims = te.dims if isinstance(te, TensorInfo) else tuple(te[0])
    if len(dims) != 2 or int(dims[0]) != E:
        raise GGUFError(f"token_embd.weight dims {list(dims)} do not match n_embd={E}")
    vocab = int(dims[1])
    gate = tensors.get("blk.0.ffn_gate.weight")
    if gate is None:
        raise GGUFError("no blk.0.ffn_gate.weight tensor (a gated-FFN model is required)")
    n_ff = int((gate.dims if isinstance(gate, TensorInfo) else gate[0])[1])
    if E % n_head:
        raise GGUFError(f"n_embd={E} is not a multiple of n_head={n_head}")
    kl = md.get(f"{arch}.attention.key_length")
    if kl is not None and int(kl) != E // n_head:
        raise GGUFError(f"{arch}.attention.key_length={kl} differs from n_embd/n_head="
                        f"{E // n_head}; the decode engine takes head_dim = n_embd/n_head")
    return ModelConfig(
        name=name or str(md.get("general.name", arch)),
        n_layers=int(g("block_count", 24)), n_embd=E, n_ff=n_ff, n_head=n_head,
        n_head_kv=int(g("attention.head_count_kv", n_head)), vocab=vocab,
        rope_theta=float(g("rope.freq_base", 1000000.0)),
        norm_eps=float(g("attention.layer_norm_rms_epsilon", 1e-6)),
        tied="output.weight" not in tensors,
        qkv_bias="blk.0.attn_q.bias" in tensors,
        max_ctx=max_ctx)


def _expected_shapes(cfg: ModelConfig) -> dict:
    return {name: (kind, shape) for name, kind, shape in weight_specs(cfg)}


@dataclass
class LoadReport:
    verbatim: int = 0           # Q8_0 tensors used as stored
    canonicalized: int = 0      # Q8_0 tensors with at least one block replaced
    blocks_replaced: int = 0
    requantized: int = 0        # F32/F16/Q4_0/Q5_0 matrices quantized to Q8_0


def load_q8_model(path, max_ctx: int = 1024, name: str | None = None):
    """(cfg, weights, reader, report): the tensors ResidentModel uploads, read from a GGUF.
    Q8_0 matrices are views of the reader's mapping (keep `reader` open until the upload is
    done, then close it); everything else is a fresh array."""
    r = GGUFReader(path)
    try:
        cfg = config_from_gguf(r.md, r.tensors, name=name, max_ctx=max_ctx)
        want = _expected_shapes(cfg)
        rep = LoadReport()
        w: dict = {}
        for tname, (kind, shape) in want.items():
            ti = r.tensors.get(tname)
            if ti is None:
                raise GGUFError(f"{path}: missing tensor {tname!r}")
            if ti.shape != tuple(shape):
                raise GGUFError(f"{tname}: stored shape {list(ti.shape)} (dims {list(ti.dims)}), "
                                f"the {cfg.name} configuration needs {list(shape)}")
            if kind == "q8":
                if ti.ggml_type == GGML_Q8_0:
                    blocks, n = canonical_q8_0(r.q8_blocks(tname), name=tname)
                    if n:
                        rep.canonicalized += 1
                        rep.blocks_replaced += n
                    else:
                        rep.verbatim += 1
                    w[tname] = blocks
                elif ti.ggml_type in _BLOCK:
                    w[tname] = q8.quantize_rows(r.dequantize(tname))
                    rep.requantized += 1
                else:
                    raise GGUFError(f"{tname}: type {type_name(ti.ggml_type)} is not supported")
            else:
                w[tname] = np.ascontiguousarray(r.dequantize(tname), dtype=np.float32)
        return cfg, w, r, rep
    except Exception:
        r.close()
        raise


def gguf_arch(cfg: ModelConfig) -> str:
    return "qwen2" if cfg.qkv_bias else "llama"


def save_q8_model(path, cfg: ModelConfig, weights: dict, alignment: int = DEFAULT_ALIGNMENT,
                  metadata: dict | None = None) -> None:
    """Write a ModelConfig and its GGUF-named tensors (Q8_0 blocks, float32 vectors) as a GGUF
    file that load_q8_model reads back to the same configuration and bytes.  `metadata` adds
    keys (write_gguf's value forms), e.g. tokenizer.ggml.tokens."""
    arch = gguf_arch(cfg)
    md = {
        "general.architecture": arch,
        "general.name": cfg.name,
        "general.file_type": (GGUF_UINT32, 7),            # mostly Q8_0
        f"{arch}.block_count": cfg.n_layers,
        f"{arch}.context_length": cfg.max_ctx,
        f"{arch}.embedding_length": cfg.n_embd,
        f"{arch}.feed_forward_length": cfg.n_ff,
        f"{arch}.attention.head_count": cfg.n_head,
        f"{arch}.attention.head_count_kv": cfg.n_head_kv,
        f"{arch}.rope.freq_base": (GGUF_FLOAT32, cfg.rope_theta),
        f"{arch}.attention.layer_norm_rms_epsilon": (GGUF_FLOAT32, cfg.norm_eps),
    }
    md.update(metadata or {})
    tensors = []
    for tname, kind, shape in weight_specs(cfg):
        a = weights[tname]
        if kind == "q8":
            N, K = shape
            tensors.append((tname, (K, N), GGML_Q8_0, np.asarray(a, dtype=np.uint8)))
        else:
            tensors.append((tname, (shape[0],), GGML_F32, np.asarray(a, dtype=np.float32)))
    write_gguf(path, md, tensors, alignment=alignment)

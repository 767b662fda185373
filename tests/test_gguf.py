"""GGUF reader/writer and the Q8_0 model loader (host side, no GPU).

Pins:
- the parser against a file assembled byte by byte in this test from the GGUF layout
  (header, typed key/values, tensor infos, aligned data), independent of the writer;
- the reference's rejection cases (bad magic, truncation; bpd-substrate/file-formats/gguf/
  test_stage0.py) and tensors that lie outside the file;
- Q8_0 dequantization against exact fp16 values computed from the bit fields, on the
  subnormal/normal scale list of the reference's bpd/tests/test_dequant_subnormal.py:34-44;
- Q4_0/Q5_0 nibble and high-bit placement against hand-placed values;
- the reference loader's [ne0, ne1] orientation (llamatov_run.py:497-511);
- the canonical-block test against the dequant -> requant round trip it stands for, on every
  positive finite fp16 scale and on random blocks;
- write -> read of a full synthetic model (configuration and every byte).
"""
import struct
from fractions import Fraction

import numpy as np
import pytest

from llamatov_amd import gguf as G
from llamatov_amd import model as M
from llamatov_amd import q8


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, vt: int, payload: bytes) -> bytes:
    return _s(key) + struct.pack("<I", vt) + payload


def f16_exact(bits: int) -> Fraction:
    """The value of fp16 bit pattern `bits` from its fields (no floating point)."""
    s = -1 if bits & 0x8000 else 1
    e = (bits >> 10) & 0x1F
    m = bits & 0x3FF
    if e == 0:
        return s * Fraction(m, 2 ** 24)
    return s * (1 + Fraction(m, 1024)) * Fraction(2) ** (e - 15)


def test_parse_handbuilt_file(tmp_path):
    al = 64
    kvs = [
        _kv("general.architecture", 8, _s("qwen2")),
        _kv("general.alignment", 4, struct.pack("<I", al)),
        _kv("u8", 0, struct.pack("<B", 250)), _kv("i8", 1, struct.pack("<b", -5)),
        _kv("u16", 2, struct.pack("<H", 65000)), _kv("i16", 3, struct.pack("<h", -300)),
        _kv("i32", 5, struct.pack("<i", -70000)), _kv("f32", 6, struct.pack("<f", 0.5)),
        _kv("b", 7, b"\x01"), _kv("u64", 10, struct.pack("<Q", 2 ** 40)),
        _kv("i64", 11, struct.pack("<q", -2 ** 40)), _kv("f64", 12, struct.pack("<d", 0.1)),
        _kv("tokens", 9, struct.pack("<IQ", 8, 3) + _s("a") + _s("") + _s("é")),
        _kv("ints", 9, struct.pack("<IQ", 5, 4) + struct.pack("<4i", 1, -2, 3, -4)),
        _kv("nested", 9, struct.pack("<IQ", 9, 2) + struct.pack("<IQ", 4, 1) + struct.pack("<I", 7)
            + struct.pack("<IQ", 8, 1) + _s("z")),
    ]
    # tensor a: F32 dims [3, 2] at offset 0; tensor b: Q8_0 dims [32, 1] at offset 64
    a = np.arange(6, dtype=np.float32) + 0.25
    blk = bytes([0x00, 0x3C]) + bytes(range(32))          # d = 1.0, q = 0..31
    infos = (_s("a") + struct.pack("<I", 2) + struct.pack("<2Q", 3, 2) + struct.pack("<IQ", 0, 0)
             + _s("b") + struct.pack("<I", 2) + struct.pack("<2Q", 32, 1) + struct.pack("<IQ", 8, 64))
    head = struct.pack("<4sIQQ", b"GGUF", 3, 2, len(kvs)) + b"".join(kvs) + infos
    pad = (-len(head)) % al
    data = a.tobytes() + b"\0" * (64 - 24) + blk
    p = tmp_path / "hand.gguf"
    p.write_bytes(head + b"\0" * pad + data)

    md, ts, do = G.parse_gguf(p)
    assert do == len(head) + pad and do % al == 0
    assert md["general.architecture"] == "qwen2" and md["general.alignment"] == al
    assert (md["u8"], md["i8"], md["u16"], md["i16"], md["i32"]) == (250, -5, 65000, -300, -70000)
    assert md["f32"] == 0.5 and md["b"] is True and md["u64"] == 2 ** 40 and md["i64"] == -2 ** 40
    assert md["f64"] == 0.1
    assert md["tokens"] == ["a", "", "é"] and md["ints"] == [1, -2, 3, -4]
    assert md["nested"] == [[7], ["z"]]
    assert ts == {"a": ([3, 2], 0, 0), "b": ([32, 1], 8, 64)}

    with G.GGUFReader(p) as r:
        assert r.version == 3
        assert np.array_equal(r.dequantize("a"), a.reshape(2, 3))
        assert np.array_equal(r.q8_blocks("b"), np.frombuffer(blk, np.uint8).reshape(1, 34))
        assert np.array_equal(r.dequantize("b"), np.arange(32, dtype=np.float32).reshape(1, 32))
    # the reference loader's orientation: 2-D tensors come back as [ne0, ne1]
    la = G.lt(p, do, ts["a"])
    assert la.shape == (3, 2) and np.array_equal(la, a.reshape(2, 3).T)
    lb = G.lt(p, do, ts["b"])
    assert lb.shape == (32, 1) and np.array_equal(lb[:, 0], np.arange(32, dtype=np.float32))


def test_rejections(tmp_path):
    p = tmp_path / "x.gguf"
    p.write_bytes(b"NOPE" + b"\x03\x00\x00\x00" + b"\x00" * 16)
    with pytest.raises(G.GGUFError, match="magic"):
        G.parse_gguf(p)
    p.write_bytes(b"GGUF" + b"\x03\x00\x00\x00")
    with pytest.raises(G.GGUFError, match="short"):
        G.parse_gguf(p)
    p.write_bytes(struct.pack("<4sIQQ", b"GGUF", 1, 0, 0))
    with pytest.raises(G.GGUFError, match="version 1"):
        G.parse_gguf(p)
    # one kv promised, none present
    p.write_bytes(struct.pack("<4sIQQ", b"GGUF", 3, 0, 1))
    with pytest.raises(G.GGUFError, match="short"):
        G.parse_gguf(p)
    # unknown value type
    p.write_bytes(struct.pack("<4sIQQ", b"GGUF", 3, 0, 1) + _kv("k", 13, b"\0" * 8))
    with pytest.raises(G.GGUFError, match="value type 13"):
        G.parse_gguf(p)
    # a Q8_0 tensor whose data runs past the end of the file
    head = (struct.pack("<4sIQQ", b"GGUF", 3, 1, 0) + _s("w") + struct.pack("<I", 2)
            + struct.pack("<2Q", 64, 4) + struct.pack("<IQ", 8, 0))
    p.write_bytes(head + b"\0" * ((-len(head)) % 32) + b"\0" * 100)
    with pytest.raises(G.GGUFError, match="past the file end"):
        G.parse_gguf(p)
    # ne0 not a whole number of blocks
    head = (struct.pack("<4sIQQ", b"GGUF", 3, 1, 0) + _s("w") + struct.pack("<I", 2)
            + struct.pack("<2Q", 40, 1) + struct.pack("<IQ", 8, 0))
    p.write_bytes(head + b"\0" * 200)
    with pytest.raises(G.GGUFError, match="multiple"):
        G.parse_gguf(p)
    with pytest.raises(FileNotFoundError):
        G.parse_gguf(tmp_path / "absent.gguf")


# bpd/tests/test_dequant_subnormal.py:34-44
SCALE_CASES = [0x0001, 0x0002, 0x00C2, 0x03FF, 0x0400, 0x3C00, 0x7BFF]


@pytest.mark.parametrize("bits", SCALE_CASES)
def test_q8_0_dequant_scales(bits):
    qs = np.array([1, -1, 127, -127, 0, 5, -128, 64] * 4, dtype=np.int8)
    blk = struct.pack("<H", bits) + qs.tobytes()
    y = G.dequantize_bytes(np.frombuffer(blk, np.uint8), G.GGML_Q8_0)
    d = f16_exact(bits)
    for j in range(32):
        exp = d * int(qs[j])                       # exact in fp32 (<= 18 significant bits)
        assert Fraction(float(y[j])) == exp, (hex(bits), j)


def test_q4_0_q5_0_layout():
    d_bits = 0x3800                                # 0.5
    qs = bytes((j * 7 + 3) & 0xFF for j in range(16))
    y4 = G.dequantize_bytes(np.frombuffer(struct.pack("<H", d_bits) + qs, np.uint8), G.GGML_Q4_0)
    for j in range(16):
        assert y4[j] == 0.5 * ((qs[j] & 15) - 8)
        assert y4[j + 16] == 0.5 * ((qs[j] >> 4) - 8)
    qh = 0xA5C3_0F01
    y5 = G.dequantize_bytes(np.frombuffer(struct.pack("<HI", d_bits, qh) + qs, np.uint8), G.GGML_Q5_0)
    for i in range(32):
        nib = (qs[i] & 15) if i < 16 else (qs[i - 16] >> 4)
        assert y5[i] == 0.5 * ((nib | (((qh >> i) & 1) << 4)) - 16), i


def _roundtrip_changes(blocks: np.ndarray) -> np.ndarray:
    """Per block: does the reference's dequant -> weight-quantizer round trip change it?"""
    x = G.dequantize_bytes(blocks.reshape(-1), G.GGML_Q8_0).reshape(-1, 32)
    back = q8.quantize_rows(x).reshape(-1, 34)
    return (back != blocks.reshape(-1, 34)).any(axis=1)


def _roundtrip(blocks: np.ndarray) -> np.ndarray:
    x = G.dequantize_bytes(blocks.reshape(-1), G.GGML_Q8_0).reshape(-1, 32)
    return q8.quantize_rows(x).reshape(blocks.shape)


def test_canonical_flag_and_form_every_scale():
    """Every positive finite fp16 scale, with q holding +127 or -127 (flagged canonical and
    unchanged by the round trip), then with max |q| = 126 (not flagged; canonical_q8_0 must
    still equal the round trip, which changes the block except where fp16(126 d / 127)
    rounds back to a subnormal d)."""
    rng = np.random.default_rng(5)
    bits = np.arange(1, 0x7C00, dtype=np.uint16)
    n = bits.size
    q = rng.integers(-127, 128, size=(n, 32)).astype(np.int8)
    q[:, 0] = np.where(rng.random(n) < 0.5, 127, -127)
    blocks = np.empty((n, 34), np.uint8)
    blocks[:, 0:2] = bits.view(np.uint8).reshape(n, 2)
    blocks[:, 2:] = q.view(np.uint8)
    ok = G.q8_block_is_canonical(blocks)
    assert ok.all()
    assert not _roundtrip_changes(blocks).any()
    got, n = G.canonical_q8_0(blocks)
    assert n == 0 and got is blocks
    q2 = np.clip(q, -126, 126)
    blocks[:, 2:] = q2.view(np.uint8)
    assert not G.q8_block_is_canonical(blocks).any()
    ch = _roundtrip_changes(blocks)
    assert ch[bits >= 0x0400].all()                # every normal scale changes
    got, n = G.canonical_q8_0(blocks)
    assert n == ch.sum() and np.array_equal(got, _roundtrip(blocks))


def test_canonical_form_random():
    rng = np.random.default_rng(11)
    n = 200_000
    blocks = rng.integers(0, 256, size=(n, 34), dtype=np.uint8)
    # bias toward the interesting cases: scales 0 / negative / tiny, q extremes
    blocks[: n // 4, 1] &= 0x03                    # zero and subnormal scales
    blocks[n // 4: n // 2, 2] = 127
    blocks[n // 2: 3 * n // 4, 3] = 0x81           # -127
    blocks[3 * n // 4:, 4] = 0x80                  # -128
    dbits = blocks[:, 0].astype(np.uint16) | (blocks[:, 1].astype(np.uint16) << 8)
    finite = (dbits & 0x7C00) < 0x7800             # |d| < 32768: no fp16 overflow on requant
    b = blocks[finite]
    ok = G.q8_block_is_canonical(b)
    ch = _roundtrip_changes(b)
    assert not (ok & ch).any()                     # flagged blocks are fixed points
    assert ok.sum() > 1000 and ch.sum() > 1000
    m = b.shape[0] // 4 * 4                        # rows of 4 blocks (K = 128)
    got, n = G.canonical_q8_0(b[:m].reshape(-1, 34 * 4).copy())
    assert np.array_equal(got.reshape(-1, 34), _roundtrip(b[:m].copy())) and n == ch[:m].sum()


def test_canonical_q8_0_replaces_only_failing_blocks():
    rng = np.random.default_rng(2)
    w = rng.standard_normal((8, 128), dtype=np.float32)
    w[3, 32:64] = 0.0                              # an all-zero block (d = 1 after quantize_rows)
    rows = q8.quantize_rows(w)
    same, n = G.canonical_q8_0(rows)
    assert n == 0 and same is rows
    bad = rows.copy()
    blk = bad[5].reshape(4, 34)
    blk[2, 2:] = (blk[2, 2:].view(np.int8) // 2).view(np.uint8)   # max |q| now 63
    blk[1, 0:2] = 0                                               # scale 0
    fixed, n = G.canonical_q8_0(bad)
    assert n == 2 and fixed is not bad
    expect = q8.quantize_rows(q8.dequantize_rows(bad, 128))
    assert np.array_equal(fixed, expect)
    # the round trip changes the values of the halved block: that is what the reference uses
    assert not np.array_equal(q8.dequantize_rows(fixed, 128)[5, 64:96],
                              q8.dequantize_rows(bad, 128)[5, 64:96])
    inf = rows.copy()
    inf[0, 0:2] = np.frombuffer(struct.pack("<H", 0x7C00), np.uint8)
    inf[0, 2] = 0
    with pytest.raises(G.GGUFError, match="non-finite"):
        G.canonical_q8_0(inf)
    big = rows.copy()
    big[0, 0:2] = np.frombuffer(struct.pack("<H", 0x7BFF), np.uint8)   # 65504
    big[0, 2] = 0x80                                                    # q = -128
    with pytest.raises(G.GGUFError, match="fp16 range"):
        G.canonical_q8_0(big)


def test_ggml_quantizer_blocks_are_canonical():
    """Blocks quantized the way ggml does it (d = amax/127, q = round-half-away(x * (1/d)))
    load verbatim; only all-zero blocks (d = 0) differ from the reference's residency."""
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((4000, 32)) * rng.uniform(1e-6, 10, (4000, 1))).astype(np.float32)
    x[17] = 0.0
    amax = np.abs(x).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    idv = np.where(d > 0, np.float32(1) / np.where(d > 0, d, 1), 0).astype(np.float32)
    v = x * idv[:, None]
    q = (np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))).astype(np.int8)
    blocks = np.empty((4000, 34), np.uint8)
    blocks[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = q.view(np.uint8)
    ok = G.q8_block_is_canonical(blocks)
    assert not ok[17] and ok[np.arange(4000) != 17].all()


def test_config_from_metadata_defaults():
    ts = {"token_embd.weight": ([896, 1000], 8, 0), "blk.0.ffn_gate.weight": ([896, 4864], 8, 0),
          "blk.0.attn_q.bias": ([896], 0, 0)}
    cfg = G.config_from_gguf({}, ts)
    # decode_fact.load_model's defaults (bpd/decode_fact.py:39-51)
    assert (cfg.n_layers, cfg.n_head, cfg.n_head_kv, cfg.n_embd) == (24, 14, 14, 896)
    assert cfg.rope_theta == 1e6 and cfg.norm_eps == 1e-6
    assert cfg.vocab == 1000 and cfg.n_ff == 4864 and cfg.tied and cfg.qkv_bias
    md = {"general.architecture": "llama", "llama.attention.head_count": 32,
          "llama.attention.head_count_kv": 8, "llama.embedding_length": 4096,
          "llama.block_count": 32, "llama.rope.freq_base": 500000.0,
          "llama.attention.layer_norm_rms_epsilon": 1e-5}
    ts = {"token_embd.weight": ([4096, 128256], 8, 0), "output.weight": ([4096, 128256], 8, 0),
          "blk.0.ffn_gate.weight": ([4096, 14336], 8, 0)}
    cfg = G.config_from_gguf(md, ts)
    ref = M.LLAMA3_8B
    for f in ("n_layers", "n_embd", "n_ff", "n_head", "n_head_kv", "vocab", "rope_theta",
              "norm_eps", "tied", "qkv_bias"):
        assert getattr(cfg, f) == getattr(ref, f), f
    with pytest.raises(G.GGUFError, match="key_length"):
        G.config_from_gguf(dict(md, **{"llama.attention.key_length": 256}), ts)


@pytest.mark.parametrize("cfg", [M.TINY, M.TINY.replace(tied=False, qkv_bias=False)],
                         ids=["qwen2-tied-bias", "llama-untied"])
def test_model_write_read_roundtrip(tmp_path, cfg):
    w = M.synth_weights(cfg, seed=77)
    p = tmp_path / "m.gguf"
    G.save_q8_model(p, cfg, w)
    got_cfg, got_w, reader, rep = G.load_q8_model(p, max_ctx=cfg.max_ctx, name=cfg.name)
    try:
        f32 = lambda v: float(np.float32(v))
        assert got_cfg == cfg.replace(norm_eps=f32(cfg.norm_eps), rope_theta=f32(cfg.rope_theta),
                                      norm_init="ones")   # a generator setting, not stored
        assert set(got_w) == set(w)
        for k in w:
            assert got_w[k].dtype == w[k].dtype and np.array_equal(got_w[k], w[k]), k
        n_q8 = sum(1 for _, kind, _ in M.weight_specs(cfg) if kind == "q8")
        assert (rep.verbatim, rep.canonicalized, rep.requantized) == (n_q8, 0, 0)
        # Q8_0 tensors are views of the mapping, not copies
        assert not got_w["token_embd.weight"].flags.owndata
    finally:
        del got_w
        reader.close()


def test_model_file_carries_extra_metadata(tmp_path):
    """save_q8_model's extra keys (a tokenizer's token strings and BOS id) read back through
    parse_gguf, where llamatov_gpu_resident's command line looks them up."""
    cfg = M.TINY
    toks = [f"t{i}" for i in range(cfg.vocab)]
    toks[17] = "Hello"
    p = tmp_path / "m.gguf"
    G.save_q8_model(p, cfg, M.synth_weights(cfg, seed=5), metadata={
        "tokenizer.ggml.tokens": (G.GGUF_ARRAY, G.GGUF_STRING, toks),
        "tokenizer.ggml.bos_token_id": (G.GGUF_UINT32, 3)})
    md, ts, _ = G.parse_gguf(p)
    assert md["tokenizer.ggml.tokens"] == toks and md["tokenizer.ggml.bos_token_id"] == 3
    assert len(ts) == len(M.weight_specs(cfg))


def test_gpu_resident_run_signature():
    """The reference's run(path, input_ids, n_tokens=10) signature (llamatov_gpu_resident.py:20);
    without arguments its command line prints its usage instead of loading anything."""
    import inspect
    from llamatov_amd import llamatov_gpu_resident as R
    sig = inspect.signature(R.run)
    assert list(sig.parameters) == ["path", "input_ids", "n_tokens"]
    assert sig.parameters["n_tokens"].default == 10
    assert R.main([]) == 2


def test_loader_requantizes_other_types(tmp_path):
    cfg = M.TINY
    w = M.synth_weights(cfg, seed=3)
    p = tmp_path / "m.gguf"
    G.save_q8_model(p, cfg, w)
    md, ts, do = G.parse_gguf(p)
    # rewrite one weight as F16 and one Q8_0 tensor with a non-canonical block
    with G.GGUFReader(p) as r:
        tensors = []
        for name, ti in r.tensors.items():
            data = np.array(r.raw(name))
            tt = ti.ggml_type
            if name == "blk.1.ffn_up.weight":
                data = r.dequantize(name).astype(np.float16)
                tt = G.GGML_F16
            if name == "blk.0.attn_k.weight":
                blk = data.reshape(-1, 34)
                blk[5, 2:] = (blk[5, 2:].view(np.int8) // 3).view(np.uint8)
            tensors.append((name, ti.dims, tt, data))
        md2 = dict(r.md)
    typed = {k: v for k, v in md2.items()}
    typed[f"qwen2.rope.freq_base"] = (G.GGUF_FLOAT32, md2["qwen2.rope.freq_base"])
    typed[f"qwen2.attention.layer_norm_rms_epsilon"] = (G.GGUF_FLOAT32,
                                                        md2["qwen2.attention.layer_norm_rms_epsilon"])
    p2 = tmp_path / "m2.gguf"
    G.write_gguf(p2, typed, tensors)
    _, got, reader, rep = G.load_q8_model(p2)
    try:
        assert rep.requantized == 1 and rep.canonicalized == 1 and rep.blocks_replaced == 1
        up = w["blk.1.ffn_up.weight"]
        assert np.array_equal(got["blk.1.ffn_up.weight"],
                              q8.quantize_rows(q8.dequantize_rows(up, cfg.n_embd).astype(np.float16)
                                               .astype(np.float32)))
        k = got["blk.0.attn_k.weight"]
        orig = w["blk.0.attn_k.weight"]
        assert np.array_equal(k.reshape(-1, 34)[np.arange(k.size // 34) != 5],
                              orig.reshape(-1, 34)[np.arange(k.size // 34) != 5])
    finally:
        del got
        reader.close()


def test_loader_shape_errors(tmp_path):
    cfg = M.TINY
    w = M.synth_weights(cfg, seed=3)
    w2 = dict(w)
    del w2["blk.1.ffn_down.weight"]
    p = tmp_path / "m.gguf"
    with pytest.raises(KeyError):
        G.save_q8_model(p, cfg, w2)
    G.save_q8_model(p, cfg.replace(n_ff=cfg.n_ff), w)
    # declare a wrong head count: attn_q rows no longer match
    with G.GGUFReader(p) as r:
        md = dict(r.md)
        tensors = [(n, ti.dims, ti.ggml_type, np.array(r.raw(n))) for n, ti in r.tensors.items()]
    md["qwen2.attention.head_count_kv"] = 1
    md["qwen2.rope.freq_base"] = (G.GGUF_FLOAT32, md["qwen2.rope.freq_base"])
    md["qwen2.attention.layer_norm_rms_epsilon"] = (G.GGUF_FLOAT32,
                                                    md["qwen2.attention.layer_norm_rms_epsilon"])
    p2 = tmp_path / "bad.gguf"
    G.write_gguf(p2, md, tensors)
    with pytest.raises(G.GGUFError, match="attn_k.weight"):
        G.load_q8_model(p2)

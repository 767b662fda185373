"""Host-side logic of the reference surface (llamatov_amd.dev_residency, llamatov_run) that
runs without a GPU: the fp32 -> Q8_0 weight conversion of a reference weight dict, the
config mapping, the embedding round-trip test that selects host rows, the flag gate."""
import numpy as np
import pytest

from llamatov_amd import dev_residency as dr
from llamatov_amd import model as M
from llamatov_amd import q8 as hq8


def reference_w(cfg, qw):
    w = {}
    for name, kind, shape in M.weight_specs(cfg):
        a = qw[name]
        if kind == "q8":
            a = hq8.dequantize_rows(a, shape[1]).T
        w[name] = np.ascontiguousarray(a, np.float32)
    return w


@pytest.mark.parametrize("cfg", [M.TINY, M.TINY.replace(name="t-untied", tied=False, qkv_bias=False)],
                         ids=lambda c: c.name)
def test_reference_weights_convert_to_the_same_blocks(cfg):
    qw = M.synth_weights(cfg, seed=3)
    w = reference_w(cfg, qw)
    mc = dr._engine_cfg(cfg.as_cfg(), w)
    assert (mc.n_layers, mc.n_embd, mc.n_ff, mc.n_head, mc.n_head_kv, mc.vocab, mc.tied, mc.qkv_bias) == \
        (cfg.n_layers, cfg.n_embd, cfg.n_ff, cfg.n_head, cfg.n_head_kv, cfg.vocab, cfg.tied, cfg.qkv_bias)
    ew = dr._engine_weights(w, mc)
    for name, kind, _ in M.weight_specs(cfg):
        assert np.array_equal(ew[name], qw[name]), name
    rows = dr._embedding_rows(w, cfg.n_embd)
    assert np.array_equal(hq8.dequantize_rows(ew["token_embd.weight"], cfg.n_embd), rows)


def test_engine_cfg_refuses_a_decoupled_head_dim():
    cfg = M.TINY
    w = reference_w(cfg, M.synth_weights(cfg, seed=3))
    c = dict(cfg.as_cfg(), head_dim=cfg.head_dim * 2)
    with pytest.raises(ValueError):
        dr._engine_cfg(c, w)


def test_composition_gate_on_the_host():
    try:
        dr.apply_production_profile()
        dr.assert_certified_composition()
        dr._QFUSED = True
        with pytest.raises(RuntimeError):
            dr.assert_certified_composition()
        dr.apply_production_profile()
        dr._DEVICE_ATTN = False
        with pytest.raises(RuntimeError):
            dr.assert_certified_composition()
        dr.apply_production_profile()
        dr._KV_ELEM_BYTES = 3
        with pytest.raises(RuntimeError):
            dr.assert_certified_composition()
    finally:
        dr.apply_production_profile()
        dr._KV_ELEM_BYTES = 4
    live = dr.attest_profile()
    assert all(live[k] == v for k, v in dr.PRODUCTION_PROFILE.items())
    # the attestation names the flags that select nothing here, and what the engine runs
    assert set(live["_INERT_FLAGS"]) <= set(dr.PRODUCTION_PROFILE) | {"_RMS_QUANT_FUSED"}
    assert "_KV_ELEM_BYTES" not in live["_INERT_FLAGS"] and "_ATTN_SPLIT_K" not in live["_INERT_FLAGS"]
    assert live["_ENGINE"]["fused_step"] and live["_ENGINE"]["numerics"] == "engine"
    assert live["_ENGINE"]["kv_dtype"] == ("f16" if dr._KV_ELEM_BYTES == 2 else "f32")


def test_engine_profile_refusals():
    """The engine's Profile gate (the reference's composition gate, dev_residency.py:1268-1281)
    refuses uncertified splits, cache types and numerics, and a ggml-numerics profile that
    asks for the fused step."""
    from llamatov_amd import engine as E
    E.assert_certified_composition(E.PRODUCTION_PROFILE)
    E.assert_certified_composition(E.GGML_PROFILE)
    for bad in (E.Profile(attn_nsplit=3), E.Profile(kv_dtype=2), E.Profile(numerics="fast"),
                E.Profile(numerics="ggml"), E.Profile(numerics="ggml", fused_step=False, fused_rms_quant=True)):
        with pytest.raises(RuntimeError):
            E.assert_certified_composition(bad)


def test_attn_nsplit_rule():
    from llamatov_amd import engine as E
    certified = {1, 2, 4, 8, 16, 32, 64, 128}
    for B in (1, 2, 8, 32):
        for L in (1, 30, 64, 100, 1000, 4096, 6400, 16384, 32768, 131072):
            n = E.attn_nsplit_for(B, L, 8)
            assert n in certified
            assert n == 1 or L // n >= 64                      # at least 64 rows per split
    assert [E.attn_nsplit_for(1, L, 8) for L in (4096, 16384, 32768)] == [64, 64, 64]
    assert [E.attn_nsplit_for(8, L, 8) for L in (4096, 16384, 32768)] == [32, 32, 64]


def test_load_model_orientation(tmp_path):
    from llamatov_amd import gguf
    from llamatov_amd import llamatov_run as R
    cfg = M.TINY
    qw = M.synth_weights(cfg, seed=4)
    p = tmp_path / "t.gguf"
    gguf.save_q8_model(p, cfg, qw)
    c, w = R.load_model(str(p))
    assert (c["n_layers"], c["n_head"], c["n_head_kv"], c["n_embd"]) == (cfg.n_layers, cfg.n_head,
                                                                          cfg.n_head_kv, cfg.n_embd)
    wq = np.asarray(w["blk.0.attn_q.weight"])
    assert wq.shape == (cfg.n_embd, cfg.q_dim)      # [ne0, ne1] = inputs x outputs
    assert np.array_equal(wq.T, hq8.dequantize_rows(qw["blk.0.attn_q.weight"], cfg.n_embd))
    emb = np.asarray(w["token_embd.weight"])
    assert emb.shape == (cfg.n_embd, cfg.vocab)
    ew = dr._engine_weights(w, dr._engine_cfg(c, w))
    assert np.array_equal(ew["token_embd.weight"], qw["token_embd.weight"])


def test_resident_cache_keys_on_the_dict_and_its_content(monkeypatch):
    """Two weight dicts that share token_embd but differ in one layer weight get separate
    device models; the same unchanged dict hits; a dict whose tensor was replaced is uploaded
    again (the stale model freed); release_resident frees and forgets.  (No GPU: the upload is
    replaced by a recorder.)"""
    built = []

    class Recorder:
        def __init__(self, mc, ew, dev, layouts):
            self.freed = False
            built.append(self)

        def free(self):
            self.freed = True

    monkeypatch.setattr(dr.engine, "ResidentModel", Recorder)
    monkeypatch.setattr(dr, "_dev", lambda: None)
    monkeypatch.setattr(dr, "_MODELS", {})
    cfg = M.TINY
    w1 = reference_w(cfg, M.synth_weights(cfg, seed=3))
    w2 = dict(w1)   # the same arrays, token_embd included
    w2["blk.1.ffn_down.weight"] = (w1["blk.1.ffn_down.weight"] * np.float32(1.5)).astype(np.float32)
    m1 = dr._resident(w1, cfg.as_cfg())[0]
    m2 = dr._resident(w2, cfg.as_cfg())[0]
    assert m1 is not m2 and len(built) == 2
    assert dr._resident(w1, cfg.as_cfg())[0] is m1 and len(built) == 2
    w1["blk.0.attn_q.weight"] = (w1["blk.0.attn_q.weight"] + np.float32(0.01)).astype(np.float32)
    m1b = dr._resident(w1, cfg.as_cfg())[0]
    assert m1b is not m1 and m1.freed and not m1b.freed
    dr.release_resident(w1)
    dr.release_resident(w2)
    assert m1b.freed and m2.freed and not dr._MODELS

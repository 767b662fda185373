"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py):
the oracle must still reproduce them bit for bit (CPU), and the gfx950 kernels must match
them through the C ABI (gpu)."""
import ctypes
from pathlib import Path

import numpy as np
import pytest

from llamatov_amd import model as M

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(GOLD / name, allow_pickle=False)


def same_bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), np.asarray(b, np.float32).view(np.uint32)
    return a.shape == b.shape and np.array_equal(a, b)


# ---- CPU: the oracle still reproduces the fixtures ---------------------------------
def test_oracle_gemv_fixture(oracle):
    g = load("gemv_canonical_64x256.npz")
    assert same_bits(oracle.q8_gemv(g["W"], g["xq"], g["xd"], 256), g["y"])
    assert same_bits(oracle.q8_gemv(g["W"], g["xq"], g["xd"], 256, g["resid"]), g["y_resid"])
    assert np.array_equal(oracle.block_dots(g["W"], g["xq"], 256), g["isum"])


def test_oracle_quant_rms_rope_fixtures(oracle):
    g = load("quant_q8_896.npz")
    xq, xd = oracle.quant_q8(g["x"])
    assert np.array_equal(xq, g["xq"]) and np.array_equal(xd, g["xd"])
    sq, sd = oracle.silu_mul_quant(g["x"], g["u"])
    assert np.array_equal(sq, g["silu_xq"]) and np.array_equal(sd, g["silu_xd"])
    r = load("rmsnorm_896.npz")
    assert same_bits(oracle.rmsnorm(r["x"], r["w"], float(r["eps"])), r["y"])
    p = load("rope_hd64.npz")
    assert same_bits(oracle.rope_freqs(64, float(p["theta"])), p["freqs"])
    for i, pos in enumerate(p["pos"]):
        assert same_bits(oracle.rope(p["x"], int(pos), 16, 64, float(p["theta"])), p["y"][i])


def test_oracle_attention_fixture(oracle):
    a = load("attn_small.npz")
    L, sc = int(a["L"]), float(a["scale"])
    for f16, (kc, vc) in ((False, (a["kc"], a["vc"])), (True, (a["kc16"], a["vc16"]))):
        for s in (1, 3):
            out = oracle.attn_decode(a["q"], kc, vc, L, 4, 2, 32, sc, f16, s)
            assert same_bits(out, a[f"out_{'f16' if f16 else 'f32'}_s{s}"])


def test_oracle_decode_fixture(oracle):
    import hashlib
    g = load("decode_tiny.npz")
    w = M.synth_weights(M.TINY, seed=99)
    h = hashlib.sha256()
    for k in sorted(w):
        h.update(k.encode())
        h.update(np.ascontiguousarray(w[k]).tobytes())
    assert h.hexdigest() == str(g["weights_sha256"]), "synthetic weight generator changed"
    om = oracle.OracleModel(M.TINY, w)
    toks, _ = om.generate(g["prompt"].tolist(), 16)
    assert toks == g["tokens"].tolist()
    assert same_bits(om.step(toks[-1]), g["final_logits"])


# ---- GPU: the kernels match the fixtures --------------------------------------------
@pytest.mark.gpu
def test_gpu_matches_op_fixtures(gpu):
    from llamatov_amd import engine as dr
    from llamatov_amd._lib import LT_KV_F16, LT_KV_F32, call, raw
    up = lambda a: dr.DevTensor.from_host(np.ascontiguousarray(a))
    print("[gpu-case] golden op fixtures", flush=True)
    g = load("gemv_canonical_64x256.npz")
    W = dr.Q8Weight(g["W"], 256)
    y = dr.DevTensor.empty((64,), np.float32)
    dr.q8_gemv_into(W, up(g["xq"]), up(g["xd"]), y)
    assert same_bits(y.to_host(), g["y"])
    dr.q8_gemv_into(W, up(g["xq"]), up(g["xd"]), y, up(g["resid"]))
    assert same_bits(y.to_host(), g["y_resid"])

    q = load("quant_q8_896.npz")
    dq, dd = dr.DevTensor.empty((896,), np.int8), dr.DevTensor.empty((28,), np.uint16)
    dr.quant_q8_into(up(q["x"]), dq, dd, 896)
    assert np.array_equal(dq.to_host(), q["xq"]) and np.array_equal(dd.to_host(), q["xd"])

    r = load("rmsnorm_896.npz")
    ry = dr.DevTensor.empty((896,), np.float32)
    dr.rms_norm_into(up(r["x"]), up(r["w"]), float(r["eps"]), ry)
    assert same_bits(ry.to_host(), r["y"])

    p = load("rope_hd64.npz")
    for i, pos in enumerate(p["pos"]):
        dx = up(p["x"])
        call("lt_rope_qk", gpu.handle, dx.vp, up(np.array([pos], np.int32)).vp, 16, 64, up(p["freqs"]).vp)
        assert same_bits(dx.to_host(), p["y"][i])

    a = load("attn_small.npz")
    L = int(a["L"])
    for kvd, (kc, vc), tag in ((LT_KV_F32, (a["kc"], a["vc"]), "f32"), (LT_KV_F16, (a["kc16"], a["vc16"]), "f16")):
        for s in (1, 3):
            ws_n = raw("lt_attn_workspace_size")(1, 4, 32, s)
            ws = dr.DevTensor.empty((max(ws_n, 1),), np.uint8)
            out = dr.DevTensor.empty((128,), np.float32)
            call("lt_attn_decode", gpu.handle, up(a["q"]).vp, up(kc).vp, up(vc).vp,
                 up(np.array([L], np.int32)).vp, out.vp, 1, 4, 2, 32, ctypes.c_float(float(a["scale"])),
                 24, s, kvd, ws.vp, ws.nbytes)
            assert same_bits(out.to_host(), a[f"out_{tag}_s{s}"]), (tag, s)


@pytest.mark.gpu
@pytest.mark.parametrize("kv", ["f32", "f16_split4"])
def test_gpu_matches_decode_fixture(gpu, kv):
    from llamatov_amd import engine as dr
    from llamatov_amd._lib import LT_KV_F16, LT_KV_F32
    print(f"[gpu-case] golden decode fixture {kv}", flush=True)
    g = load("decode_tiny.npz")
    w = M.synth_weights(M.TINY, seed=99)
    prof = dr.Profile() if kv == "f32" else dr.Profile(kv_dtype=LT_KV_F16, attn_nsplit=4)
    plan = dr.DecodePlan(dr.ResidentModel(M.TINY, w), prof)
    gr = dr.StepGraph(plan)
    gr.seed(g["prompt"].tolist())
    first = plan.read_token()
    gr.capture()
    toks = [first] + gr.replay_tokens(15)
    exp = g["tokens"] if kv == "f32" else g["tokens_f16_split4"]
    assert toks == exp.tolist()
    if kv == "f32":
        assert same_bits(gr.replay_logits(toks[-1]), g["final_logits"])
    gr.free()
    plan.free()

"""lt_attn_decode_noalloc: the split-K decode attention with its partials in the library's
device scratch array instead of a workspace, against lt_attn_decode with a workspace, bit for
bit, on two calls in a row (the second with a smaller input), plus the size refusal.  Calls
go through the C ABI."""
import ctypes

import numpy as np
import pytest

from llamatov_amd import _lib
from llamatov_amd import engine as dr
from llamatov_amd._lib import LT_KV_F16, LT_KV_F32, call

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[gpu-case] {msg}", flush=True)


def up(a):
    return dr.DevTensor.from_host(np.ascontiguousarray(a))


def run_pair(gpu, rng, B, L, nh, nkv, hd, nsplit, kv_dtype):
    f16 = kv_dtype == LT_KV_F16
    k = rng.standard_normal((B, L, nkv * hd), dtype=np.float32)
    v = rng.standard_normal((B, L, nkv * hd), dtype=np.float32)
    if f16:
        k, v = k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
    q = rng.standard_normal((B, nh * hd), dtype=np.float32)
    lens = np.array([L - 3 * b for b in range(B)], np.int32)
    dq, dk, dv, dl = up(q), up(k), up(v), up(lens)
    scale = ctypes.c_float(hd ** -0.5)
    wsn = _lib.raw("lt_attn_workspace_size")(B, nh, hd, nsplit)
    ws = dr.DevTensor.empty((max(wsn, 16),), np.uint8)
    ref = dr.DevTensor.empty((B, nh * hd), np.float32)
    got = dr.DevTensor.empty((B, nh * hd), np.float32)
    gpu.fill(got.ptr, 0xFF, got.nbytes)
    call("lt_attn_decode", gpu.handle, dq.vp, dk.vp, dv.vp, dl.vp, ref.vp, B, nh, nkv, hd, scale, L, nsplit,
         kv_dtype, ws.vp, ws.nbytes)
    call("lt_attn_decode_noalloc", gpu.handle, dq.vp, dk.vp, dv.vp, dl.vp, got.vp, B, nh, nkv, hd, scale, L,
         nsplit, kv_dtype)
    r, g = ref.to_host(), got.to_host()
    for t in (dq, dk, dv, dl, ws, ref, got):
        t.free()
    return r, g, q, k, v, lens


@pytest.mark.parametrize("first,second", [
    ((8, 4096, 32, 8, 128, 32, LT_KV_F16), (2, 1000, 32, 8, 128, 8, LT_KV_F16)),
    ((4, 700, 14, 2, 64, 16, LT_KV_F32), (1, 65, 14, 2, 64, 4, LT_KV_F32)),
    ((1, 300, 16, 8, 128, 1, LT_KV_F16), (1, 100, 16, 8, 128, 3, LT_KV_F16)),
])
def test_noalloc_equals_workspace_entry(gpu, oracle, first, second):
    rng = np.random.default_rng(31)
    for shape in (first, second):
        B, L, nh, nkv, hd, nsplit, kvd = shape
        case(f"noalloc B={B} L={L} nh={nh} nkv={nkv} hd={hd} nsplit={nsplit} kv={kvd}")
        r, g, q, k, v, lens = run_pair(gpu, rng, B, L, nh, nkv, hd, nsplit, kvd)
        assert np.array_equal(r.view(np.uint32), g.view(np.uint32)), shape
        exp = oracle.attn_decode(q[-1], k[-1], v[-1], int(lens[-1]), nh, nkv, hd, float(hd ** -0.5),
                                 kvd == LT_KV_F16, nsplit)
        assert np.array_equal(g[-1].view(np.uint32), exp.view(np.uint32)), shape


def test_noalloc_refuses_more_than_its_scratch(gpu):
    case("noalloc size refusal")
    B, L, nh, nkv, hd, nsplit = 8, 256, 32, 8, 128, 128
    need = _lib.raw("lt_attn_workspace_size")(B, nh, hd, nsplit)
    assert need > 16 << 20
    z = dr.DevTensor.empty((B * L * nkv * hd,), np.uint16)
    q = dr.DevTensor.empty((B * nh * hd,), np.float32)
    lens = up(np.full(B, L, np.int32))
    out = dr.DevTensor.empty((B * nh * hd,), np.float32)
    gpu.fill(out.ptr, 0x7F, out.nbytes)
    gpu.fill(z.ptr, 0, z.nbytes)
    gpu.fill(q.ptr, 0, q.nbytes)
    rc = _lib.raw("lt_attn_decode_noalloc")(gpu.handle, q.vp, z.vp, z.vp, lens.vp, out.vp, B, nh, nkv, hd,
                                            ctypes.c_float(1.0), L, nsplit, LT_KV_F16)
    assert rc == -1 and "scratch" in _lib.last_error()
    assert np.all(out.to_host().view(np.uint32) == 0x7F7F7F7F)   # nothing launched


def test_noalloc_refuses_a_second_context(gpu):
    """The scratch is one array per GPU: once a context has used it, a call from another
    context on that GPU is refused (LT_ESTATE, nothing launched), a call that needs no
    scratch (nsplit 1) still runs there, and the owner keeps working."""
    rng = np.random.default_rng(7)
    shape = (2, 300, 14, 2, 64, 4, LT_KV_F16)
    case("noalloc owner claims the scratch")
    r, g, *_ = run_pair(gpu, rng, *shape)
    assert np.array_equal(r.view(np.uint32), g.view(np.uint32))
    other = ctypes.c_void_p()
    call("lt_init", gpu.index, ctypes.byref(other))
    try:
        case("noalloc second context refused")
        B, L, nh, nkv, hd, nsplit, kvd = shape
        k = up(np.zeros((B, L, nkv * hd), np.uint16))
        q = up(rng.standard_normal((B, nh * hd), dtype=np.float32))
        lens = up(np.full(B, L, np.int32))
        out = dr.DevTensor.empty((B, nh * hd), np.float32)
        gpu.fill(out.ptr, 0x7F, out.nbytes)
        fn = _lib.raw("lt_attn_decode_noalloc")
        rc = fn(other, q.vp, k.vp, k.vp, lens.vp, out.vp, B, nh, nkv, hd, ctypes.c_float(0.125), L, nsplit, kvd)
        assert rc == -2 and "another context" in _lib.last_error()
        gpu.sync()
        assert np.all(out.to_host().view(np.uint32) == 0x7F7F7F7F)
        case("noalloc second context, nsplit 1")
        rc = fn(other, q.vp, k.vp, k.vp, lens.vp, out.vp, B, nh, nkv, hd, ctypes.c_float(0.125), L, 1, kvd)
        assert rc == 0
        call("lt_sync", other)
        assert np.all(out.to_host() == 0.0)    # zero K and V rows give zero outputs
        for t in (k, q, lens, out):
            t.free()
    finally:
        call("lt_free_ctx", other)
    case("noalloc owner after the refusal")
    r, g, *_ = run_pair(gpu, rng, 1, 100, 14, 2, 64, 3, LT_KV_F32)
    assert np.array_equal(r.view(np.uint32), g.view(np.uint32))

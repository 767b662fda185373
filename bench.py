#!/usr/bin/env python3
"""Benchmark of the Q8_0 bs=1 decode hot path on one MI355X.

Workload ("C2"): greedy decode of a random-init
Qwen2.5-0.5B-architecture Q8_0 model (24 layers, hidden 896, FFN 4864, 14 Q / 2 KV heads,
head_dim 64, vocab 151936, tied lm_head), fp16 KV cache with max context 1024, a 32-token
uniform-random prompt, 128 decoded tokens at batch 1.  A step is one decode token: one
replay of the captured HIP graph (embedding gather -> 24 layers -> logits -> argmax), with
every weight and the KV cache resident in HBM before the timed region starts.

Printed (one JSON line on stdout): decode tok/s; `step_kernels`, every launch of the step
timed live with HIP events on the library's stream (a captured graph of back-to-back
launches over rotated weight copies >= 600 MB, so the 256 MB Infinity Cache cannot serve
them), with its algorithmic bytes, HBM rate and share of the step's kernel time;
`roofline`, the largest-share kernel of that table; the CPU baseline: the oracle (C
restatement of the reference arithmetic, OpenMP over GEMV rows) decoding a bounded sample of
the same workload and timing the C1 GEMV on the host cores, all cores and one core; and the
other BASELINE configs as legs of the same line (`gemv_sweep`: C1 and C3; `c4_attention`: C4;
`c5`: the 8B prefill and decode), selected by --legs (default all three) or by naming legs
one by one (--gemv-sweep, --c4, --c5: then only those).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "bs=1 decode tok/s (Q8_0 0.5B/8B-arch) + Q8_0 GEMV HBM GB/s % of peak"
HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Events:
    def __init__(self, dev):
        from llamatov_amd import _lib
        self._lib = _lib
        self.dev = dev
        self.a, self.b = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.call("lt_event_create", dev.handle, ctypes.byref(self.a))
        _lib.call("lt_event_create", dev.handle, ctypes.byref(self.b))

    def start(self):
        self._lib.call("lt_event_record", self.dev.handle, self.a)

    def stop_ms(self) -> float:
        self._lib.call("lt_event_record", self.dev.handle, self.b)
        ms = ctypes.c_float()
        self._lib.call("lt_event_elapsed_ms", self.a, self.b, ctypes.byref(ms))
        return float(ms.value)

    def free(self):
        self._lib.call("lt_event_destroy", self.a)
        self._lib.call("lt_event_destroy", self.b)


def graph_us_per_launch(dev, launches, reps: int = 3) -> float:
    """Average duration of one launch: the launches captured back to back into one graph,
    replayed `reps` times between two HIP events on the library's stream."""
    from llamatov_amd import _lib
    for f in launches:   # warm: code objects loaded, pages mapped
        f()
    dev.sync()
    _lib.call("lt_graph_begin", dev.handle)
    for f in launches:
        f()
    g = ctypes.c_void_p()
    _lib.call("lt_graph_end", dev.handle, ctypes.byref(g))
    _lib.call("lt_graph_launch", dev.handle, g)
    dev.sync()
    ev = Events(dev)
    ev.start()
    for _ in range(reps):
        _lib.call("lt_graph_launch", dev.handle, g)
    ms = ev.stop_ms()
    ev.free()
    _lib.raw("lt_graph_free")(g)
    return ms * 1e3 / (reps * len(launches))


def rotation(dev, mats, min_bytes: float = 600e6):
    """The given device matrices plus device copies of them, cycled, until the set holds at
    least min_bytes (so a back-to-back loop streams from HBM, not the Infinity Cache).
    Returns (set, extra copies to free)."""
    from llamatov_amd import engine as dr
    out, extra, i = list(mats), [], 0
    while sum(m.nbytes for m in out) < min_bytes:
        src = mats[i % len(mats)]
        t = dr.DevTensor.empty(src.shape, src.dtype, dev)
        dev.d2d(t.ptr, src.ptr, src.nbytes)
        out.append(t)
        extra.append(t)
        i += 1
    return out, extra


def persistent_entry(dev, plan, L: int) -> dict:
    """The persistent step (lt_decode_step: every layer in one launch) timed on its own: a
    graph of back-to-back launches alternating between the plan's weights and a device copy of
    every layer matrix (~760 MB together, more than the 256 MB Infinity Cache holds), the caches
    at length L (each launch appends a row; the lengths are restored after).  Algorithmic bytes
    per launch: every layer's Q8_0 weights, the K/V rows attended (at the mean length of the
    launches) and appended, the norm and bias vectors, the embedding row and the output row."""
    from llamatov_amd import engine as dr
    cfg, m = plan.cfg, plan.model
    copies, extra = {}, []
    for il, Ly in enumerate(m.layers):
        for name in ("wqkv", "wo", "wgu_il", "wdown"):
            src = Ly[name].t
            t = dr.DevTensor.empty(src.shape, src.dtype, dev)
            dev.d2d(t.ptr, src.ptr, src.nbytes)
            copies[(il, name)] = t
            extra.append(t)
    alt = plan.step_layer_descs(copies)
    launches = [lambda: plan.enqueue_layers(), lambda: plan.enqueue_layers(alt)] * 4
    saved = plan.lengths().copy()
    dev.h2d(plan.lens.ptr, np.full(cfg.n_layers, L, np.int32))
    us = graph_us_per_launch(dev, launches)   # 5 x 8 launches: lengths L .. L + 39
    dev.h2d(plan.lens.ptr, saved)
    if plan.error():
        raise RuntimeError(f"persistent step reported device error {plan.error()} while timed")
    for t in extra:
        t.free()
    alt.free()
    rb = lambda N, K: N * (K // 32) * 34
    E, F, QD, NQ = cfg.n_embd, cfg.n_ff, cfg.q_dim, cfg.n_qkv
    esz = 2 if plan.profile.kv_dtype else 4
    per_layer = (rb(NQ, E) + rb(E, QD) + rb(2 * F, E) + rb(E, F) + 2 * (L + 20) * cfg.kv_dim * esz
                 + 2 * cfg.kv_dim * esz + 8 * E + (4 * NQ if cfg.qkv_bias else 0))
    nbytes = cfg.n_layers * per_layer + (E // 32) * 34 + 4 * E
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"step kernel step (persistent): {us:.2f} us, {gbs:.0f} GB/s")
    return {"name": "step", "kernel": "k_decode_step<f16> (lt_decode_step: every layer in one launch)",
            "shape": [cfg.n_layers, E, F, cfg.n_head, cfg.n_head_kv, cfg.head_dim, L + 20], "launches_per_step": 1,
            "avg_launch_us": round(us, 3), "bytes_per_launch": int(nbytes), "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def step_kernels(dev, plan, only: str | None = None, attn_len: int | None = None,
                 five: bool = False) -> list[dict]:
    """Every launch of the fused C2 decode step, timed on its own (graph of back-to-back
    launches over rotated weights), with its algorithmic bytes per launch:
      qkv     rmsnorm -> quant -> QKV GEMV + bias         N(K/32)34 + 8K + 8N
      attn    RoPE -> KV append -> attention -> quant      2 (L+1) kv_dim 2 (fp16 rows) + 4 n_qkv + QD + QD/16
      o       O GEMV + residual                            N(K/32)34 + K + K/16 + 8N
      gateup  rmsnorm -> quant -> gate|up GEMV -> SiLU*up -> quant   2F(K/32)34 + 8K + F + F/16
      down    down GEMV + residual                         N(K/32)34 + K + K/16 + 8N
      vocab   final rmsnorm -> quant -> vocab GEMV -> argmax        V(K/32)34 + 8K + 4V
    The attention runs at cache length attn_len (default: the plan's current length; the
    decode bench passes the mean length of its timed tokens), over rows the decode wrote; its
    launches leave the lengths unchanged.  When the plan runs the persistent step at that
    length (and five is False) the table is that launch (persistent_entry) and the vocab
    launch."""
    from llamatov_amd import engine as dr
    from llamatov_amd._lib import call
    cfg, m, p = plan.cfg, plan.model, plan.profile
    if not p.fused_step or p.swiglu_fp32 or p.attn_nsplit != 1:
        raise ValueError("step_kernels times the default fused step (nsplit 1, quantizing gate|up epilogue)")
    Lq = attn_len if attn_len is not None else plan.caches[0].length
    persistent = not five and plan.persistent_len >= Lq + 1
    four = not persistent and plan.four_launch_len >= Lq + 1
    h = dev.handle
    E, F, hd, nh, nkv = cfg.n_embd, cfg.n_ff, cfg.head_dim, cfg.n_head, cfg.n_head_kv
    QD, NQ, V = cfg.q_dim, cfg.n_qkv, cfg.vocab
    eps = ctypes.c_float(cfg.norm_eps)
    rb = lambda N, K: N * (K // 32) * 34
    L = plan.caches[0].length if attn_len is None else int(attn_len)
    # the four-launch step's kernels read (QKV, attention) or bump (gate|up) a length: here a
    # scratch int holding L, so the plan's own lengths stay as they are
    lenL = dr.DevTensor.from_host(np.array([L], np.int32), dev)
    lenB = dr.DevTensor.from_host(np.array([L], np.int32), dev)
    maxt = plan.caches[0].max_seq
    kinds4 = {
        "qkv": dict(kernel="k_gemv_fused<4, PRO_RMS, EPI_ROPE_KV> (lt_q8_gemv_rms_rope_kv)", shape=[NQ, E],
                    mats=[Ly["wqkv"].t for Ly in m.layers], count=cfg.n_layers,
                    bytes=rb(NQ, E) + 8 * E + 8 * NQ + 2 * cfg.kv_dim * (2 if p.kv_dtype else 4),
                    fn=lambda w, il: call("lt_q8_gemv_rms_rope_kv", h, plan.carry.vp, None, None, V, None,
                                          plan.err.vp, m.layers[il]["attn_norm"].vp, eps, w.vp,
                                          dr._vp(m.layers[il]["bqkv"]), plan.qkv.vp, E, m.freqs.vp,
                                          plan.caches[il].k.vp, plan.caches[il].v.vp, lenL.vp, nh, nkv, hd, maxt,
                                          p.kv_dtype)),
        "attn_o": dict(kernel="k_attn_o<f16> (lt_q8_gemv_attn_o: attention + quant + O GEMV + residual)",
                       shape=[E, QD, nh, nkv, hd, L + 1], mats=[Ly["wo"].t for Ly in m.layers], count=cfg.n_layers,
                       bytes=rb(E, QD) + 2 * (L + 1) * cfg.kv_dim * (2 if p.kv_dtype else 4) + 4 * QD + 8 * E,
                       fn=lambda w, il: call("lt_q8_gemv_attn_o", h, plan.qkv.vp, plan.caches[il].k.vp,
                                             plan.caches[il].v.vp, lenL.vp, nh, nkv, hd, ctypes.c_float(plan.scale),
                                             maxt, p.kv_dtype, w.vp, plan.carry.vp, plan.xres.vp, E)),
        "gateup": dict(kernel="k_gemv_fused<4, PRO_RMS, EPI_SILU, staged> (lt_q8_gemv_rms_silu_len)",
                       shape=[2 * F, E], mats=[Ly["wgu_il"].t for Ly in m.layers], count=cfg.n_layers,
                       bytes=rb(2 * F, E) + 8 * E + F + F // 16,
                       fn=lambda w, il: call("lt_q8_gemv_rms_silu_len", h, plan.xres.vp, m.layers[il]["ffn_norm"].vp,
                                             eps, w.vp, plan.xq.vp, plan.xd.vp, F, E, lenB.vp, maxt)),
    }
    kinds = {
        "qkv": dict(kernel="k_gemv_fused<4, PRO_RMS, EPI_RESID> (lt_q8_gemv_rms)", shape=[NQ, E],
                    mats=[Ly["wqkv"].t for Ly in m.layers], count=cfg.n_layers,
                    bytes=rb(NQ, E) + 8 * E + 8 * NQ,
                    fn=lambda w, il: call("lt_q8_gemv_rms", h, plan.carry.vp, m.layers[il]["attn_norm"].vp, eps,
                                          w.vp, dr._vp(m.layers[il]["bqkv"]), plan.qkv.vp, NQ, E)),
        "attn": dict(kernel="k_attn_w1<f16, STEP> (lt_attn_step)", shape=[nh, nkv, hd, L + 1],
                     mats=None, count=cfg.n_layers,
                     bytes=2 * (L + 1) * cfg.kv_dim * 2 + 4 * NQ + QD + QD // 16,
                     fn=lambda w, il: call("lt_attn_step", h, plan.qkv.vp, m.freqs.vp, plan.caches[il].k.vp,
                                           plan.caches[il].v.vp, dr._vp(plan.caches[il].len_ptr), None,
                                           plan.xq.vp, plan.xd.vp, nh, nkv, hd, ctypes.c_float(plan.scale),
                                           plan.caches[il].max_seq, 1, p.kv_dtype, None, 0)),
        "o": dict(kernel="k_gemv_fused<1, PRO_MERGE, EPI_RESID> (lt_q8_gemv_attn_out)", shape=[E, QD],
                  mats=[Ly["wo"].t for Ly in m.layers], count=cfg.n_layers,
                  bytes=rb(E, QD) + QD + QD // 16 + 8 * E,
                  fn=lambda w, il: call("lt_q8_gemv_attn_out", h, plan.xq.vp, plan.xd.vp, None, 0, 1, nh, hd, w.vp,
                                        plan.carry.vp, plan.xres.vp, E, QD, None, 0)),
        "gateup": dict(kernel="k_gemv_fused<4, PRO_RMS, EPI_SILU, staged> (lt_q8_gemv_rms_silu)", shape=[2 * F, E],
                       mats=[Ly["wgu_il"].t for Ly in m.layers], count=cfg.n_layers,
                       bytes=rb(2 * F, E) + 8 * E + F + F // 16,
                       fn=lambda w, il: call("lt_q8_gemv_rms_silu", h, plan.xres.vp, m.layers[il]["ffn_norm"].vp, eps,
                                             w.vp, plan.xq.vp, plan.xd.vp, F, E)),
        "down": dict(kernel="k_gemv_fused<1, PRO_STAGE, EPI_RESID> (lt_q8_gemv)", shape=[E, F],
                     mats=[Ly["wdown"].t for Ly in m.layers], count=cfg.n_layers,
                     bytes=rb(E, F) + F + F // 16 + 8 * E,
                     fn=lambda w, il: call("lt_q8_gemv", h, w.vp, plan.xq.vp, plan.xd.vp, plan.xres.vp, plan.carry.vp,
                                           E, F)),
        "vocab": dict(kernel=("k_gemv_fused<16, PRO_RMS, EPI_ARGMAX, planar> + k_argmax_finalize "
                              "(lt_q8_gemv_rms_argmax_pl)" if plan.head_pl else
                              "k_gemv_fused<4, PRO_RMS, EPI_ARGMAX> + k_argmax_finalize (lt_q8_gemv_rms_argmax)"),
                      shape=[V, E], mats=[(plan.head_pl or m.output).t], count=1, bytes=rb(V, E) + 8 * E + 4 * V,
                      fn=lambda w, il: call("lt_q8_gemv_rms_argmax" + ("_pl" if plan.head_pl else ""), h,
                                            plan.carry.vp, m.output_norm.vp, eps, w.vp, plan.logits.vp, V, E,
                                            plan.tok.vp, None, None, 0, plan.am_ws.vp, plan.am_ws.nbytes)),
    }
    if four:
        kinds = {"qkv": kinds4["qkv"], "attn_o": kinds4["attn_o"], "gateup": kinds4["gateup"],
                 "down": kinds["down"], "vocab": kinds["vocab"]}
    out = []
    if persistent:
        kinds = {"vocab": kinds["vocab"]}
        if not only or only == "step":
            out.append(persistent_entry(dev, plan, L))
    for name, k in kinds.items():
        if only and name != only:
            continue
        extra = []
        if k["mats"] is None:   # attention: one launch per layer cache, twice over, at length L
            saved = plan.lengths().copy()
            dev.h2d(plan.lens.ptr, np.full(cfg.n_layers, L, np.int32))
            launches = [lambda il=il: k["fn"](None, il) for il in range(cfg.n_layers)] * 2
        else:
            mats, extra = rotation(dev, k["mats"])
            launches = [lambda w=w, i=i: k["fn"](w, i % cfg.n_layers) for i, w in enumerate(mats)]
        us = graph_us_per_launch(dev, launches)
        if k["mats"] is None:
            dev.h2d(plan.lens.ptr, saved)
        for t in extra:
            t.free()
        gbs = k["bytes"] / (us * 1e-6) / 1e9
        out.append({"name": name, "kernel": k["kernel"], "shape": k["shape"], "launches_per_step": k["count"],
                    "avg_launch_us": round(us, 3), "bytes_per_launch": int(k["bytes"]), "GB/s": round(gbs, 1),
                    "frac": round(gbs / HBM_PEAK_GBS, 4)})
        log(f"step kernel {name}: {us:.2f} us, {gbs:.0f} GB/s")
    lenL.free()
    lenB.free()
    tot = sum(e["avg_launch_us"] * e["launches_per_step"] for e in out)
    for e in out:
        e["share"] = round(e["avg_launch_us"] * e["launches_per_step"] / tot, 4) if tot else None
    return out


def roofline_of(entry: dict) -> dict:
    """The bench line's roofline object for one step-kernel entry; traffic (HBM bytes per
    launch) comes from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE runs of the same
    kernel when profiles/ holds them (bench.py --roofline-only is the counter command)."""
    traffic, src = None, None
    tf = ROOT / "profiles" / f"traffic_{entry['name']}_c2.txt"
    if tf.exists():
        import re
        mt = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", tf.read_text(), flags=re.M)
        if mt:
            traffic, src = int(mt.group(1)), f"profiles/{tf.name} (committed counter run, not this run)"
    return {"kernel": entry["kernel"], "step_kernel": entry["name"], "shape": entry["shape"], "bound": "hbm",
            "achieved": entry["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": entry["frac"],
            "traffic": traffic, "traffic_source": src, "bytes_per_launch": entry["bytes_per_launch"],
            "avg_launch_us": entry["avg_launch_us"], "launches_per_step": entry["launches_per_step"],
            "share_of_step_kernel_time": entry["share"],
            "timing": "HIP events on the library stream around a graph of back-to-back launches over >= 600 MB "
                      "of rotated weight copies"}


GEMV_SWEEP = [("C1 ffn_up 0.5B", 4864, 896), ("C3 q/o 8B", 4096, 4096), ("C3 gate/up 8B", 14336, 4096),
              ("C3 down 8B", 4096, 14336), ("C3 lm_head 8B", 128256, 4096), ("C2 lm_head 0.5B", 151936, 896)]


def gemv_sweep(dev, launches: int = 60, reps: int = 5) -> list[dict]:
    """Q8_0 GEMV bandwidth (BASELINE configs 1 and 3, plus the 0.5B vocab projection):
    lt_q8_gemv on random blocks, rotating >= 600 MB of weight copies so the MALL cannot
    serve them, timed with HIP events on the library's stream: one untimed pass over the
    copies, then the median of `reps` timed runs of `launches` back-to-back launches."""
    from llamatov_amd import engine as dr
    from llamatov_amd._lib import call
    out = []
    rng = np.random.default_rng(5)
    for name, N, K in GEMV_SWEEP:
        nb = K // 32
        blk = np.empty((N, nb, 34), np.uint8)
        blk[..., 2:] = rng.integers(-127, 128, size=(N, nb, 32), dtype=np.int8).view(np.uint8)
        blk[..., :2] = (rng.standard_normal((N, nb)) * 0.01).astype(np.float16).view(np.uint8).reshape(N, nb, 2)
        wbytes = blk.nbytes
        copies = max(2, int(np.ceil(600e6 / wbytes)))
        ws = [dr.DevTensor.from_host(blk.reshape(N, nb * 34), dev) for _ in range(copies)]
        del blk
        xq = dr.DevTensor.from_host(rng.integers(-127, 128, K, dtype=np.int64).astype(np.int8), dev)
        xd = dr.DevTensor.from_host((rng.standard_normal(nb) * 0.05).astype(np.float16).view(np.uint16), dev)
        y = dr.DevTensor.empty((N,), np.float32, dev)

        def timed(fn, mats):
            for i in range(copies):
                call(fn, dev.handle, mats[i].vp, xq.vp, xd.vp, None, y.vp, N, K)
            dev.sync()
            runs = []
            for _ in range(reps):
                ev = Events(dev)
                ev.start()
                for i in range(launches):
                    call(fn, dev.handle, mats[i % copies].vp, xq.vp, xd.vp, None, y.vp, N, K)
                runs.append(ev.stop_ms() / 1e3 / launches)
                ev.free()
            return float(np.median(runs))
        alg = N * nb * 34 + K + 2 * nb + 4 * N
        avg_b = timed("lt_q8_gemv", ws)
        row = {"shape": f"{name} {N}x{K}"}
        if K % 1024 == 0:
            # the decode path streams planar copies of such matrices (lt_q8_to_planar): the
            # figure is lt_q8_gemv_pl's, the GGUF-block kernel's beside it
            pls = []
            for t in ws:
                p = dr.DevTensor.empty((t.nbytes,), np.uint8, dev)
                call("lt_q8_to_planar", dev.handle, t.vp, p.vp, N, K)
                pls.append(p)
            avg = timed("lt_q8_gemv_pl", pls)
            for t in pls:
                t.free()
            row["layout"] = "planar"
            row["blocks_us"] = round(avg_b * 1e6, 2)
        else:
            avg = avg_b
            row["layout"] = "blocks"
        for t in ws + [xq, xd, y]:
            t.free()
        row.update({"us": round(avg * 1e6, 2), "GB/s": round(alg / avg / 1e9, 1),
                    "frac": round(alg / avg / 1e9 / HBM_PEAK_GBS, 4)})
        out.append(row)
        log(f"gemv {name} {N}x{K} ({row['layout']}): {avg * 1e6:.2f} us, {alg / avg / 1e9:.0f} GB/s"
            + (f" (blocks {avg_b * 1e6:.2f} us)" if K % 1024 == 0 else ""))
    return out


INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA, TOP/s (2 ops per MAC)
C5_ATTN_NSPLIT = 16       # C5 decode attention: ceil(776/16) = 49 positions per split


def attention_sweep(dev, reps: int = 20) -> list[dict]:
    """GQA decode attention, 32 Q / 8 KV heads, head_dim 128, fp16 KV
    N(0,1), one query token per sequence, L in {4k, 16k, 32k}, batch 1 and 8 (split-K over
    context with the ascending-split merge).  Algorithmic bytes: the K and V rows read plus
    q and out.  Per shape: 3 untimed calls, then the median of 5 timed runs of `reps` calls
    (HIP events on the library's stream)."""
    from llamatov_amd import engine as dr
    from llamatov_amd._lib import LT_KV_F16, call, raw
    out = []
    nh, nkv, hd = 32, 8, 128
    rng = np.random.default_rng(9)
    for L in (4096, 16384, 32768):
        for B in (1, 8):
            kv = (rng.standard_normal((B * L * nkv * hd,), dtype=np.float32)).astype(np.float16).view(np.uint16)
            kc = dr.DevTensor.from_host(kv, dev)
            vc = dr.DevTensor.from_host(kv[::-1].copy(), dev)
            del kv
            q = dr.DevTensor.from_host(rng.standard_normal(B * nh * hd).astype(np.float32), dev)
            lens = dr.DevTensor.from_host(np.full(B, L, np.int32), dev)
            o = dr.DevTensor.empty((B * nh * hd,), np.float32, dev)
            nsplit = dr.attn_nsplit_for(B, L, nkv)   # CU-filling, 64 .. 512 rows per split
            wsn = raw("lt_attn_workspace_size")(B, nh, hd, nsplit)
            ws = dr.DevTensor.empty((max(wsn, 16),), np.uint8, dev)
            args = (dev.handle, q.vp, kc.vp, vc.vp, lens.vp, o.vp, B, nh, nkv, hd, ctypes.c_float(hd ** -0.5), L,
                    nsplit, LT_KV_F16, ws.vp, ws.nbytes)
            for _ in range(3):
                call("lt_attn_decode", *args)
            dev.sync()
            runs = []
            for _ in range(5):   # the median of 5 timed runs of `reps` calls
                ev = Events(dev)
                ev.start()
                for _ in range(reps):
                    call("lt_attn_decode", *args)
                runs.append(ev.stop_ms() / reps)
                ev.free()
            ms = sorted(runs)[2]
            alg = B * 2 * L * nkv * hd * 2 + 2 * B * nh * hd * 4
            out.append({"L": L, "batch": B, "nsplit": nsplit, "us": round(ms * 1e3, 2),
                        "GB/s": round(alg / (ms * 1e-3) / 1e9, 1), "frac": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
            log(f"attention L={L} B={B} nsplit={nsplit}: {ms * 1e3:.1f} us, {alg / (ms * 1e-3) / 1e9:.0f} GB/s")
            for t in (kc, vc, q, lens, o, ws):
                t.free()
    return out


def c5_cpu_decode(cfg, w, n_prompt: int = 4, n_decode: int = 3) -> dict:
    """The oracle decoding the C5 model on the host (all cores): n_prompt tokens stepped
    untimed, then n_decode greedy tokens timed."""
    from oracle import oracle as orc
    from llamatov_amd import model as M
    cores = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))
    orc.set_threads(cores)
    m = orc.OracleModel(cfg, w, kv_f16=True, attn_nsplit=C5_ATTN_NSPLIT, max_ctx=n_prompt + n_decode + 4)
    logits = None
    for t in M.random_prompt(cfg, n_prompt, seed=17):
        logits = m.step(t)
    t0 = time.perf_counter()
    for _ in range(n_decode):
        logits = m.step(orc.argmax(logits))
    dt = time.perf_counter() - t0
    return {"value": round(n_decode / dt, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"C5 model, {n_prompt}-token prompt stepped untimed, then {n_decode} greedy decode steps "
                      f"timed on {cores} threads (oracle/lt_oracle.c)"}


def c5_leg(dev, n_prefill: int = 512, n_decode: int = 256, eager: bool = False, cpu: bool = False) -> dict:
    """random-init Llama-3-8B-architecture Q8_0 model (N(0,0.02) weights
    quantized with the engine quantizer), a 512-token prefill of random ids through the
    tiled int8-MFMA GEMM, then 256 greedy decode tokens (graph replay) with an fp16 KV cache."""
    from llamatov_amd import engine as dr
    from llamatov_amd import model as M
    from llamatov_amd._lib import LT_KV_F16
    cfg = M.LLAMA3_8B
    t0 = time.perf_counter()
    w = M.synth_weights(cfg, seed=4321)
    log(f"C5 weights generated in {time.perf_counter() - t0:.1f}s")
    cpu_res = None
    if cpu:
        log("C5 CPU baseline: oracle decode")
        cpu_res = c5_cpu_decode(cfg, w)
    model = dr.ResidentModel(cfg, w, dev, layouts="fused")
    del w
    # split-K over the context (the declared split order, merged in the attention launch)
    plan = dr.DecodePlan(model, dr.Profile(kv_dtype=LT_KV_F16, attn_nsplit=C5_ATTN_NSPLIT),
                         max_ctx=n_prefill + n_decode + 8, hist_cap=4096)
    prompt = M.random_prompt(cfg, n_prefill, seed=17)
    # warm the prefill kernels on a short prompt, then rewind
    dr.forward_prefill(plan, prompt[:8])
    plan.prefill_buffers(n_prefill)      # activation buffers are set-up, not prefill work
    dev.sync()
    plan.reset()
    ev = Events(dev)
    ev.start()
    dr.forward_prefill(plan, prompt)
    pre_ms = ev.stop_ms()
    macs = n_prefill * cfg.n_layers * (cfg.n_qkv * cfg.n_embd + cfg.n_embd * cfg.q_dim + 2 * cfg.n_ff * cfg.n_embd
                                      + cfg.n_embd * cfg.n_ff)
    res = {"model": cfg.name, "cpu_baseline": cpu_res, "prefill_tokens": n_prefill, "prefill_ms": round(pre_ms, 3),
           "prefill_tok_s": round(n_prefill / (pre_ms / 1e3), 1),
           "prefill_mfma_util": round(2 * macs / (pre_ms / 1e3) / (INT8_PEAK_TOPS * 1e12), 4),
           "prefill_gemm_macs": int(macs)}
    if n_decode <= 4:   # prefill only (counter runs)
        log(f"C5: prefill {pre_ms:.1f} ms ({res['prefill_mfma_util'] * 100:.1f}% of int8 MFMA peak)")
        ev.free()
        plan.free()
        model.free()
        return res
    runner = dr.StepGraph(plan)
    one = plan.step if eager else runner._launch
    if not eager:
        runner.capture()
    for _ in range(4):   # warm replay (these tokens are part of the decode)
        one()
    dev.sync()
    ev.start()
    for _ in range(n_decode - 4):
        one()
    dec_ms = ev.stop_ms()
    tok_s = (n_decode - 4) / (dec_ms / 1e3)
    kv_bytes = sum(cfg.n_layers * 2 * (n_prefill + i + 1) * cfg.kv_dim * 2 for i in range(n_decode)) / n_decode
    step_bytes = cfg.weight_bytes() + kv_bytes
    res.update({"decode_tokens": n_decode, "decode_tok_s": round(tok_s, 2),
                "decode_ms_per_token": round(dec_ms / (n_decode - 4), 4), "decode_step_bytes": int(step_bytes),
                "decode_roofline_frac": round(step_bytes * tok_s / (HBM_PEAK_GBS * 1e9), 4)})
    log(f"C5: prefill {pre_ms:.1f} ms ({res['prefill_mfma_util'] * 100:.1f}% of int8 MFMA peak), "
        f"decode {tok_s:.1f} tok/s")
    ev.free()
    runner.free()
    plan.free()
    model.free()
    return res


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, weights, prompt, n_decode: int, kv_f16: bool, n_decode_1core: int = 12,
                 gemv_iters: int = 200) -> tuple[dict, list[int]]:
    """The oracle on the host: C2 greedy decode tok/s over n_decode tokens after the prompt
    (all cores), the same on one core over the first n_decode_1core of those tokens, and the
    C1 GEMV (4864 x 896 on rotated weight copies > 512 MB) median over gemv_iters calls."""
    from oracle import oracle as orc
    cores = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))

    def decode(n, threads):
        orc.set_threads(threads)
        m = orc.OracleModel(cfg, weights, kv_f16=kv_f16)
        logits = None
        for t in prompt:
            logits = m.step(t)
        toks = []
        t0 = time.perf_counter()
        for _ in range(n):
            tok = orc.argmax(logits)
            toks.append(tok)
            logits = m.step(tok)
        return n / (time.perf_counter() - t0), toks

    tps, toks = decode(n_decode, cores)
    tps1, toks1 = decode(n_decode_1core, 1)
    # C1: 4864 x 896 GEMV on N(0, 0.02) weights and an N(0,1) activation, both quantized
    rng = np.random.default_rng(11)
    from llamatov_amd import q8
    W = q8.quantize_rows((rng.standard_normal((4864, 896), dtype=np.float32) * np.float32(0.02)))
    copies = [W] + [W.copy() for _ in range(int(np.ceil(512e6 / W.nbytes)))]
    xq, xd = orc.quant_q8(rng.standard_normal(896, dtype=np.float32))
    gemv = {}
    for threads in (cores, 1):
        orc.set_threads(threads)
        ts = []
        for i in range(gemv_iters):
            t0 = time.perf_counter()
            orc.q8_gemv(copies[i % len(copies)], xq, xd, 896)
            ts.append(time.perf_counter() - t0)
        gemv[threads] = float(np.median(ts)) * 1e6
    orc.set_threads(cores)
    c1_bytes = 4864 * 28 * 34 + 896 + 28 * 2 + 4 * 4864
    return ({"value": round(tps, 3), "unit": "tok/s", "cores": cores, "kind": "port",
             "value_1core": round(tps1, 3), "cpu_model": _cpu_model(),
             "c1_gemv_median_us": round(gemv[cores], 2), "c1_gemv_median_us_1core": round(gemv[1], 2),
             "c1_gemv_GBs": round(c1_bytes / (gemv[cores] * 1e-6) / 1e9, 2),
             "sample": f"C2 model, {len(prompt)}-token prompt prefilled untimed, then {n_decode} greedy decode "
                       f"steps timed on {cores} threads and the first {n_decode_1core} on 1 thread "
                       f"(oracle/lt_oracle.c, OpenMP over GEMV rows); C1 4864x896 GEMV median of {gemv_iters} "
                       f"calls over {len(copies)} rotated weight copies",
             "tokens_1core_match": toks1 == toks[:n_decode_1core]}, toks)


def batched_leg(dev, model, cfg, kv_dtype, batches, prompt_len: int, steps: int, warmup: int,
                eager: bool = False) -> list:
    """Batched decode (BatchDecodePlan): B sequences with prompt_len-token random prompts,
    prefilled, then `steps` replays of the captured batched step timed with HIP events;
    aggregate decode tok/s = B * steps / time.  Not the headline (BASELINE's metric is bs=1).
    eager: eager steps (a host synchronization each) instead of graph replays, for traced runs."""
    from llamatov_amd import engine as dr
    from llamatov_amd import model as M
    out = []
    for B in batches:
        plan = dr.BatchDecodePlan(model, B, dr.Profile(kv_dtype=kv_dtype), max_ctx=cfg.max_ctx,
                                  hist_cap=steps + warmup + 1)
        gr = dr.BatchStepGraph(plan)
        try:
            for b in range(B):
                plan.prefill(b, M.random_prompt(cfg, prompt_len, seed=100 + b))
            step = plan.step if eager else gr.replay
            if not eager:
                gr.capture()
            for _ in range(warmup):
                step()
            dev.sync()
            ev = Events(dev)
            ev.start()
            for _ in range(steps):
                step()
            ms = ev.stop_ms()
            dev.sync()
            ev.free()
            out.append({"batch": B, "tok_s": round(B * steps / (ms / 1e3), 1),
                        "ms_per_step": round(ms / steps, 4), "steps": steps, "linear": plan.linear,
                        "launch": "eager" if eager else "graph",
                        "context": f"{prompt_len + warmup} .. {prompt_len + warmup + steps}"})
            log(f"batched decode B={B}: {out[-1]['tok_s']} tok/s, {out[-1]['ms_per_step']} ms/step")
        finally:
            gr.free()
            plan.free()
    return out


def sampled_leg(dev, plan, prompt, steps: int) -> dict:
    """The C2 decode with the device sampler drawing every token (temperature 0.8, top-k 40,
    top-p 0.95): one graph replay per token, timed with HIP events, plus the sampler's own
    launch pair (lt_sample on the 151936 logits) timed back to back."""
    from llamatov_amd import engine as dr
    from llamatov_amd import _lib
    cfg = plan.cfg
    dev.h2d(plan.lens.ptr, np.full(cfg.n_layers, len(prompt), np.int32))
    for c in plan.caches:
        c.length = len(prompt)
    plan.set_sampling(0.8, top_k=40, top_p=0.95, seed=1)
    gr = dr.StepGraph(plan)
    try:
        gr.capture()
        for _ in range(4):
            gr._launch()
        dev.sync()
        dev.h2d(plan.lens.ptr, np.full(cfg.n_layers, len(prompt), np.int32))
        for c in plan.caches:
            c.length = len(prompt)
        ev = Events(dev)
        ev.start()
        for _ in range(steps):
            gr._launch()
        ms = ev.stop_ms()
        dev.sync()
        ev.free()
        us = graph_us_per_launch(dev, [lambda: plan._enqueue_sample(record=False)], reps=20)
    finally:
        gr.free()
        plan.set_sampling(None)
    return {"tok_s": round(steps / (ms / 1e3), 1), "ms_per_step": round(ms / steps, 4),
            "settings": "temperature 0.8, top_k 40, top_p 0.95", "sampler_us": round(us, 2)}


def ggml_leg(dev, model, prompt, steps: int) -> dict:
    """The ggml-compatible numerics profile: its per-op decode step at C2 (graph replays, HIP
    events) and its GEMV (vec_dot order) on the C1 and vocab shapes over rotated weights."""
    from llamatov_amd import engine as dr
    from llamatov_amd._lib import LT_GGML_VEC, LT_KV_F16, call
    cfg = model.cfg
    plan = dr.DecodePlan(model, dr.Profile(kv_dtype=LT_KV_F16, fused_step=False, numerics="ggml"))
    gr = dr.StepGraph(plan)
    out = {}
    try:
        gr.seed(prompt)
        gr.capture()
        for _ in range(4):
            gr._launch()
        dev.sync()
        ev = Events(dev)
        ev.start()
        for _ in range(steps):
            gr._launch()
        ms = ev.stop_ms()
        dev.sync()
        ev.free()
        out["decode_tok_s"] = round(steps / (ms / 1e3), 1)
        h = dev.handle
        for name, W in (("c1_4864x896", model.layers[0]["wgu"]), ("vocab_151936x896", model.output)):
            N, K = W.N, W.K
            if name.startswith("c1"):
                N = 4864
            mats, extra = rotation(dev, [W.t])
            fns = [lambda t=t, N=N, K=K: call("lt_q8_gemv_ggml", h, t.vp, plan.xq.vp, plan.xd.vp, None,
                                               plan.logits.vp, N, K, LT_GGML_VEC) for t in mats]
            us = graph_us_per_launch(dev, fns)
            nbytes = N * (K // 32) * 34 + K + K // 16 + 4 * N
            out[name] = {"us": round(us, 2), "GB/s": round(nbytes / us / 1e3, 1)}
            for t in extra:
                t.free()
    finally:
        gr.free()
        plan.free()
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="timed decode tokens")
    ap.add_argument("--warmup", type=int, default=16, help="untimed decode tokens before timing")
    ap.add_argument("--repeats", type=int, default=5,
                    help="timed runs of --steps tokens each, from the same post-prompt state; value is their "
                         "median (the reference's protocol takes the median of 6 runs, rms_quant_prod_ab.py:38-47)")
    ap.add_argument("--kv", choices=["f16", "f32"], default="f16")
    ap.add_argument("--prompt", type=int, default=32)
    ap.add_argument("--cpu-tokens", type=int, default=128, help="decode tokens in the CPU baseline sample")
    ap.add_argument("--cpu-tokens-1core", type=int, default=12, help="decode tokens of the 1-core CPU figure")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-roofline", action="store_true")
    ap.add_argument("--legs", default="gemv,c4,c5",
                    help="the other BASELINE configs to run after C2, from gemv (C1/C3 GEMV sweep), c4 (attention "
                         "sweep), c5 (8B prefill + decode); empty for none.  Naming a leg by its own flag "
                         "(--gemv-sweep, --c4, --c5) runs only the legs so named")
    ap.add_argument("--c4", action="store_true", help="time BASELINE config 4 attention (adds c4_attention)")
    ap.add_argument("--c5", action="store_true",
                    help="run BASELINE config 5 (Llama-3-8B arch: 512-token MFMA prefill + 256 decode; adds c5)")
    ap.add_argument("--c5-decode", type=int, default=256,
                    help="C5 decode tokens (at most 4: prefill only, for counter runs)")
    ap.add_argument("--gemv-sweep", action="store_true",
                    help="time the Q8_0 GEMV on the BASELINE config 1/3 shapes (adds gemv_sweep)")
    ap.add_argument("--per-op", action="store_true",
                    help="thirteen per-op launches per layer (the reference's kernel-per-op chain) "
                         "instead of the five fused launches")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only one step kernel's timing loop (--roofline-kernel), plus a device copy of a weight "
                         "matrix (the known-size kernel that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE); "
                         "for counter runs")
    ap.add_argument("--roofline-kernel", default="step",
                    choices=["step", "qkv", "attn", "o", "attn_o", "gateup", "down", "vocab"])
    ap.add_argument("--batched", default="8,64",
                    help="batch sizes of the batched-decode leg (adds batched_decode; empty to skip)")
    ap.add_argument("--no-sampled", action="store_true", help="skip the sampled-decode leg")
    ap.add_argument("--ggml", action="store_true",
                    help="also run the ggml-compatible numerics profile (adds ggml_numerics)")
    ap.add_argument("--eager", action="store_true",
                    help="launch the step's kernels directly instead of replaying the captured graph "
                         "(same kernels; for profilers that cannot trace graph launches)")
    args = ap.parse_args()
    named = {k for k, on in (("gemv", args.gemv_sweep), ("c4", args.c4), ("c5", args.c5)) if on}
    legs = named or {x.strip() for x in args.legs.split(",") if x.strip()}
    bad = legs - {"gemv", "c4", "c5"}
    if bad:
        print(f"bench.py: unknown legs {sorted(bad)} (gemv, c4, c5)", file=sys.stderr)
        return 2

    if args.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU; --gpus {args.gpus} is not supported "
              "(the hot path is single-GPU; see DESIGN.md for how it would shard)", file=sys.stderr)
        return 2

    from llamatov_amd import engine as dr
    from llamatov_amd import model as M
    from llamatov_amd._lib import LT_KV_F16, LT_KV_F32

    cfg = M.QWEN25_05B
    if args.roofline_only:
        w = M.synth_weights(cfg, seed=1234)
        dev = dr.get_device()
        model = dr.ResidentModel(cfg, w, dev, layouts="fused")
        plan = dr.DecodePlan(model, dr.Profile(kv_dtype=LT_KV_F16))
        # the cache as the timed decode sees it on average (prompt + half the steps), so the
        # attention runs at the length of the main bench line's step table
        dr.forward_prefill(plan, M.random_prompt(cfg, args.prompt + args.steps // 2, seed=7))
        entry = step_kernels(dev, plan, only=args.roofline_kernel,
                             five=args.roofline_kernel not in ("step", "vocab"))[0]
        src = model.layers[0]["wgu_il"].t
        dst = dr.DevTensor.empty(src.shape, src.dtype, dev)
        dev.d2d(dst.ptr, src.ptr, src.nbytes)   # calibration: a plain copy of known size
        dev.sync()
        print(json.dumps({"roofline": roofline_of(dict(entry, share=None)),
                          "calibration_copy_bytes": int(src.nbytes)}), flush=True)
        return 0
    if args.prompt + args.steps > cfg.max_ctx or args.prompt + args.warmup > cfg.max_ctx:
        print("bench.py: prompt + steps exceeds the 1024-position KV cache", file=sys.stderr)
        return 2
    kv_dtype = LT_KV_F16 if args.kv == "f16" else LT_KV_F32
    log("generating synthetic weights")
    t0 = time.perf_counter()
    w = M.synth_weights(cfg, seed=1234)
    log(f"weights ready in {time.perf_counter() - t0:.1f}s; uploading")
    dev = dr.get_device()
    model = dr.ResidentModel(cfg, w, dev, layouts="per_op" if args.per_op else ("both" if args.ggml else "fused"))
    plan = dr.DecodePlan(model, dr.Profile(kv_dtype=kv_dtype, fused_step=not args.per_op), hist_cap=4096)
    runner = dr.StepGraph(plan)
    prompt = M.random_prompt(cfg, args.prompt, seed=7)

    log("prefill (eager) + capture")
    runner.seed(prompt)
    first = plan.read_token()
    if not args.eager:
        runner.capture()

    def one_step():
        if args.eager:
            plan.step()
        else:
            runner._launch()

    def rewind():
        dev.h2d(plan.lens.ptr, np.full(cfg.n_layers, len(prompt), np.int32))
        for c in plan.caches:
            c.length = len(prompt)
        plan.set_token(first)
        dev.sync()

    # warmup: untimed replays from the post-prompt state
    log(f"warmup {args.warmup}")
    for _ in range(args.warmup):
        one_step()
    dev.sync()

    # timed: K back-to-back replays from the post-prompt state (the C2 decode), repeated; each
    # run is bracketed by device synchronizations and times exactly K steps
    runs = []
    tokens = None
    for r in range(max(1, args.repeats)):
        rewind()
        hist0 = plan.history_count()
        ev = Events(dev)
        t0 = time.perf_counter()
        ev.start()
        for _ in range(args.steps):
            one_step()
        gpu_ms = ev.stop_ms()
        dev.sync()
        wall_r = time.perf_counter() - t0
        ev.free()
        run_tokens = [first] + plan.history()[hist0:hist0 + args.steps]
        if tokens is None:
            tokens = run_tokens
        elif run_tokens != tokens:
            raise RuntimeError(f"bench: timed run {r} decoded other tokens than run 0")
        runs.append((wall_r, gpu_ms))
        log(f"timed run {r}: {args.steps} steps, wall {wall_r * 1e3:.2f} ms, events {gpu_ms:.2f} ms")
    order = sorted(range(len(runs)), key=lambda i: runs[i][0])
    wall, gpu_ms = runs[order[len(runs) // 2]]

    # the same decode with a host round trip per token (reference replay_token protocol), run
    # on to the CPU baseline's token count (untimed past --steps)
    n_cpu = 0 if args.no_cpu_baseline else min(args.cpu_tokens, cfg.max_ctx - len(prompt))
    rewind()
    t1 = time.perf_counter()
    sync_tokens = [first]
    for i in range(max(args.steps, n_cpu)):
        if i == args.steps:
            wall_sync = time.perf_counter() - t1
        one_step()
        sync_tokens.append(plan.read_token())
    if args.steps >= n_cpu:
        wall_sync = time.perf_counter() - t1
    long_tokens = sync_tokens
    sync_tokens = sync_tokens[:args.steps + 1]

    tok_s = args.steps / wall
    step_bytes = cfg.weight_bytes() + sum(
        cfg.n_layers * 2 * (len(prompt) + i + 1) * cfg.kv_dim * (2 if kv_dtype == LT_KV_F16 else 4)
        for i in range(args.steps)) / args.steps
    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": f"C2: {cfg.name} Q8_0 greedy decode, prompt {len(prompt)}, {args.steps} tokens, "
                        f"bs=1, {args.kv} KV cache max ctx {cfg.max_ctx}, one HIP-graph replay per token",
            "model": cfg.name, "global_batch": 1, "seq_len": len(prompt) + args.steps,
            "parallelism": "none (1 GPU)",
        },
        "host_sync_tok_s": round(args.steps / wall_sync, 2),
        "gpu_event_ms_per_step": round(gpu_ms / args.steps, 4),
        "decode_step_bytes": int(step_bytes),
        "decode_roofline_frac": round(step_bytes * tok_s / (HBM_PEAK_GBS * 1e9), 4),
        "tokens_consistent": tokens == sync_tokens,
        "repeats": len(runs),
        "runs_tok_s": [round(args.steps / w_, 2) for w_, _ in runs],
        "timing": f"median of {len(runs)} timed runs of {args.steps} graph replays each (wall clock between "
                  f"device synchronizations), all from the same post-prompt state",
        "launch_mode": "eager" if args.eager else "graph",
        "step_kernels": "per_op" if args.per_op else "fused",
    }

    if not args.no_roofline and not args.per_op:
        log("step kernels")
        table = step_kernels(dev, plan, attn_len=len(prompt) + args.steps // 2)
        result["step_kernels"] = table
        result["roofline"] = roofline_of(max(table, key=lambda e: e["share"]))
        if plan.persistent_len > 0:
            # the five-launch step the plan takes past the persistent step's length
            log("five-launch step kernels")
            result["five_launch_step_kernels"] = step_kernels(dev, plan, attn_len=len(prompt) + args.steps // 2,
                                                              five=True)

    if "gemv" in legs:
        log("GEMV sweep")
        result["gemv_sweep"] = gemv_sweep(dev)
    if "c4" in legs:
        log("C4 attention sweep")
        result["c4_attention"] = attention_sweep(dev)

    if not args.no_cpu_baseline:
        log(f"CPU baseline: oracle over {n_cpu} decode tokens")
        cb, cpu_tokens = cpu_baseline(cfg, w, prompt, n_cpu, kv_dtype == LT_KV_F16,
                                      n_decode_1core=min(args.cpu_tokens_1core, n_cpu))
        result["cpu_baseline"] = cb
        result["tokens_match_cpu"] = cpu_tokens == long_tokens[:n_cpu]

    runner.free()
    if not args.no_sampled and not args.eager:
        log("sampled decode leg")
        result["sampled_decode"] = sampled_leg(dev, plan, prompt, 64)
    plan.free()
    if args.ggml:
        log("ggml numerics leg")
        result["ggml_numerics"] = ggml_leg(dev, model, prompt, 64)
    batches = [int(b) for b in args.batched.split(",") if b.strip()]
    if batches and not args.per_op:
        log("batched decode leg")
        result["batched_decode"] = batched_leg(dev, model, cfg, kv_dtype, batches, len(prompt), 64, 8,
                                               eager=args.eager)
    if "c5" in legs:
        model.free()
        log("C5 leg")
        result["c5"] = c5_leg(dev, n_decode=args.c5_decode, eager=args.eager, cpu=not args.no_cpu_baseline)
        if result["c5"].get("cpu_baseline") and "cpu_baseline" in result:
            result["cpu_baseline"]["c5_decode_tok_s"] = result["c5"]["cpu_baseline"]["value"]
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

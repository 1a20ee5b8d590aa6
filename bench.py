"""Benchmark of the causal multi-head attention forward path on one MI355X.

Headline (``value``): full causal MHA forward at BASELINE config c3
(batch 4, seq 4096, d_model 1024, 16 heads x 64), one "step" being one pass
of the hot path over the whole batch, every kernel through the C ABI:

    cdml_project_qkv_rope  (fused Q/K/V fp32-MFMA GEMM; bias and the
                            interleaved RoPE of Q and K in its epilogue,
                            per-sequence positions)
    cdml_sdpa_fwd      (flash-style fp32-MFMA causal attention)
    cdml_linear        (output projection, bias epilogue)

``value`` = algorithmic matmul FLOPs of that step (274.91 GFLOP) / step time,
in TFLOP/s.  Beside it the line carries the flash kernel alone (``roofline``,
bound "mfma", timed with HIP events on the library stream around every
launch in the timed region), the c4 decode step (B 64 queries against a
K/V cache of 8192 x 2048, ``decode``, bound "hbm") and the multi-threaded
CPU restatement of the reference's AccelerationMutliThreadCPU timed on this
host (``cpu_baseline``).

Inputs are resident in HBM before the timed region starts.  The process never
imports torch: torch ships its own HIP runtime, and the C ABI is driven
through ctypes exactly as a P/Invoke host would.

``other_configs`` adds end-to-end figures for the other BASELINE configs: a
c2 MHA layer, the c3 12-layer decoder stack (MHA + FFN + LayerNorms), the c5
time-series model, the c1 text model's forward and greedy generation, and one
c3 sequence through the drop-in manager with host arrays (PCIe included).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-extras]
"""
from __future__ import annotations

import argparse
import ctypes as C
import hashlib
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "callaghandev.ml_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

METRIC = "attn fwd TFLOP/s (% fp32 MFMA peak) @seq4096; decode HBM GB/s @KV8192"
FP32_MFMA_PEAK_TFLOPS = 157.3   # MI355X dense fp32 matrix, AMD published
HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, AMD published

# HBM bytes per launch come from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes that
# profile_bench.py records in this profile, together with a digest of the kernel
# sources they were measured on; a record measured on other sources is not used.
TRAFFIC_PROFILE = os.path.join("profiles", "mha_c3_decode_c4_hbm_traffic.md")
TRAFFIC_SOURCES = {
    "flash_c3": ("callaghandev.ml_amd/csrc/flash_attn.hip", "callaghandev.ml_amd/csrc/common.h"),
    "decode_c4": ("callaghandev.ml_amd/csrc/decode_attn.hip", "callaghandev.ml_amd/csrc/common.h"),
}


def source_digest(paths):
    """sha256 (first 16 hex digits) of the named files' bytes, in order."""
    h = hashlib.sha256()
    for p in paths:
        with open(os.path.join(ROOT, p), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(name):
    """(HBM bytes per launch or None, provenance) for kernel `name` from the
    traffic profile; None when the profile was measured on other sources."""
    prov = {"profile": TRAFFIC_PROFILE, "current_sources": source_digest(TRAFFIC_SOURCES[name])}
    try:
        with open(os.path.join(ROOT, TRAFFIC_PROFILE)) as f:
            m = re.search(r"<!-- traffic-record (\{.*?\}) -->", f.read(), re.S)
        rec = json.loads(m.group(1)) if m else None
    except OSError:
        rec = None
    if not rec or name not in rec.get("bytes", {}):
        prov["status"] = "no record"
        return None, prov
    prov["measured_on_sources"] = rec["sources"][name]
    prov["measured"] = rec.get("date")
    if rec["sources"][name] != prov["current_sources"]:
        prov["status"] = "stale: the kernel sources changed since the profile (rerun profile_bench.py)"
        return None, prov
    prov["status"] = "current"
    return int(rec["bytes"][name]), prov

# c3: one MHA layer of the long-context stack
C3 = dict(batch=4, seq=4096, dim=1024, heads=16)
# c4: decode step
C4 = dict(batch=64, t=8192, dim=2048, heads=16)


def mha_flops(batch, seq, dim, heads):
    hd = dim // heads
    pairs = seq * (seq + 1) // 2
    core = 4 * batch * heads * hd * pairs          # Q.K^T and P.V over causal pairs
    qkv = 6 * batch * seq * dim * dim
    out = 2 * batch * seq * dim * dim
    return core, qkv, out


def decode_bytes(batch, t, dim):
    return 2 * batch * t * dim * 4 + 2 * batch * dim * 4   # K, V read once; q read, o written


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Timer:
    """Pairs of HIP events on the library stream around each launch of one kernel."""

    def __init__(self, N, n):
        self.N = N
        self.pairs = [(N.Event(), N.Event()) for _ in range(n)]
        self.i = 0

    def start(self, st):
        self.pairs[self.i][0].record(st)

    def stop(self, st):
        self.pairs[self.i][1].record(st)
        self.i += 1

    def ms(self):
        return [a.elapsed_ms(b) for a, b in self.pairs[: self.i]]


def bench_mha(N, st, steps, warmup, cfg=None):
    lib = N.lib()
    cfg = cfg or C3
    B, L, D, H = cfg["batch"], cfg["seq"], cfg["dim"], cfg["heads"]
    hd = D // H
    rows = B * L
    from cdml import synth

    rng = np.random.default_rng(3)
    x = rng.standard_normal((rows, D), dtype=np.float32)          # N(0,1) embeddings
    ws = [synth.xavier_uniform(30 + i, D, D) for i in range(4)]   # Wq Wk Wv Wo, Xavier-uniform
    bz = np.zeros(D, np.float32)                                   # biases 0 (reference init)
    dx = N.DeviceBuffer.from_array(x, st)
    dw = [N.DeviceBuffer.from_array(w, st) for w in ws]
    db = N.DeviceBuffer.from_array(bz, st)
    dq, dk, dv, da, dy = (N.DeviceBuffer(rows * D * 4) for _ in range(5))
    s = st.handle
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    # RoPE (cos, sin) table of the L positions: a per-model constant like the
    # weights, built once outside the timed region
    dcs = N.DeviceBuffer(L * hd * 4)
    N.check(lib.cdml_rope_table(dcs.ptr, L, hd, 10000.0, s))

    def step(t_flash=None, t_qkv=None, t_out=None):
        if t_qkv:
            t_qkv.start(st)
        N.check(lib.cdml_project_qkv_rope(dx.ptr, dw[0].ptr, db.ptr, dw[1].ptr, db.ptr, dw[2].ptr,
                                          db.ptr, dq.ptr, dk.ptr, dv.ptr, rows, D, D, hd, dcs.ptr, L,
                                          0, L, s))
        if t_qkv:
            t_qkv.stop(st)
        if t_flash:
            t_flash.start(st)
        N.check(lib.cdml_sdpa_fwd(dq.ptr, D, dk.ptr, D, dv.ptr, D, da.ptr, D, B, L, L, D, H, scale, 1,
                                  None, s))
        if t_flash:
            t_flash.stop(st)
        if t_out:
            t_out.start(st)
        N.check(lib.cdml_linear(da.ptr, D, dw[3].ptr, db.ptr, dy.ptr, D, rows, D, D, 0, s))
        if t_out:
            t_out.stop(st)

    log(f"[bench] c3 MHA warmup {warmup}")
    for _ in range(warmup):
        step()
    st.synchronize()
    # Timed region 1: whole steps, host clock (the step time) ...
    log(f"[bench] c3 MHA timed {steps} steps")
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    st.synchronize()
    wall = time.perf_counter() - t0
    # ... timed region 2: the same steps with HIP events around each kernel.
    tf, tq, to = Timer(N, steps), Timer(N, steps), Timer(N, steps)
    e0, e1 = N.Event(), N.Event()
    e0.record(st)
    for _ in range(steps):
        step(tf, tq, to)
    e1.record(st)
    st.synchronize()
    dev_ms = e0.elapsed_ms(e1) / steps
    flash_ms, qkv_ms, out_ms = (float(np.mean(t.ms())) for t in (tf, tq, to))
    y = dy.download((rows, D), stream=st)
    assert np.all(np.isfinite(y)), "non-finite MHA output"
    err = float64_prefix_check(x[:64], ws, y[:64], H)
    return dict(wall_s=wall, dev_ms=dev_ms, flash_ms=flash_ms, qkv_ms=qkv_ms, out_ms=out_ms,
                selfcheck_max_abs_err=err)


def float64_prefix_check(x, ws, y, heads, atol=1e-4, rtol=1e-3):
    """The first rows of sequence 0 depend only on its first rows (causal), so
    they are recomputed here in float64 numpy from the same inputs (Q/K/V
    projections, interleaved RoPE with base 10000, causal softmax attention,
    output projection; zero biases) and the timed kernels' output must meet
    the parity bar against them.  Returns the largest absolute difference."""
    n, D = x.shape
    hd = D // heads
    xd = x.astype(np.float64)
    q, k, v = (xd @ w.astype(np.float64).T for w in ws[:3])
    pos = np.arange(n, dtype=np.float64)[:, None]
    theta = pos / (10000.0 ** (2.0 * np.arange(hd // 2) / hd))[None, :]   # [n, hd/2]
    c, s_ = np.tile(np.cos(theta), heads), np.tile(np.sin(theta), heads)   # [n, D/2]
    for t in (q, k):
        a, b = t[:, 0::2].copy(), t[:, 1::2].copy()
        t[:, 0::2], t[:, 1::2] = a * c - b * s_, a * s_ + b * c
    att = np.empty_like(q)
    scale = 1.0 / np.sqrt(hd)
    mask = np.triu(np.ones((n, n), bool), 1)
    for h in range(heads):
        cols = slice(h * hd, (h + 1) * hd)
        sc = q[:, cols] @ k[:, cols].T * scale
        sc[mask] = -np.inf
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        att[:, cols] = (p / p.sum(axis=1, keepdims=True)) @ v[:, cols]
    want = att @ ws[3].astype(np.float64).T
    diff = np.abs(y.astype(np.float64) - want)
    if not np.all(diff <= atol + rtol * np.abs(want)):
        raise AssertionError(f"bench self-check: MHA output rows differ from float64 by up to {diff.max():.3g}")
    return float(diff.max())


def bench_decode(N, st, steps, warmup):
    lib = N.lib()
    B, T, D, H = C4["batch"], C4["t"], C4["dim"], C4["heads"]
    rng = np.random.default_rng(4)
    per_seq = T * D * 4
    dk, dv = N.DeviceBuffer(B * per_seq), N.DeviceBuffer(B * per_seq)
    # N(0,1) cache rows: 16 distinct [T, D] blocks per tensor, tiled over the batch.
    blocks = 16
    for buf in (dk, dv):
        for j in range(blocks):
            blk = rng.standard_normal((T, D), dtype=np.float32)
            hb = N.DeviceBuffer.from_array(blk, st)
            for b in range(j, B, blocks):
                N.check(lib.cdml_memcpy_d2d_async(buf.ptr + b * per_seq, hb.ptr, per_seq, st.handle))
            st.synchronize()
            hb.free()
    dq = N.DeviceBuffer.from_array(rng.standard_normal((B, D), dtype=np.float32), st)
    dl = N.DeviceBuffer.from_array(np.full(B, T, np.int32), st)
    do = N.DeviceBuffer(B * D * 4)
    wsz = C.c_size_t(0)
    N.check(lib.cdml_decode_attn_workspace_size(B, T, D, H, C.byref(wsz)))
    dws = N.DeviceBuffer(max(4, wsz.value))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D // H)))

    def step():
        N.check(lib.cdml_decode_attn(dq.ptr, dk.ptr, dv.ptr, dl.ptr, do.ptr, B, T, D, H, scale, dws.ptr,
                                     wsz.value, st.handle))

    for _ in range(warmup):
        step()
    st.synchronize()
    tm = Timer(N, steps)
    for _ in range(steps):
        tm.start(st)
        step()
        tm.stop(st)
    st.synchronize()
    ms = tm.ms()
    o = do.download((B, D), stream=st)
    assert np.all(np.isfinite(o)), "non-finite decode output"
    return dict(ms=float(np.mean(ms)), ms_min=float(np.min(ms)))


def bench_mha_backward(N, st, steps, warmup, cfg=None):
    """The c3 MHA layer backward as TransformerTrainer.BackpropAttention runs it
    (TransformerTrainer.cs:933-987): BackpropLinearProjection of the output
    projection, MultiHeadAttentionBackward with the decoder mask, the inverse
    RoPE of dQ and dK, BackpropQKV.  Events around the attention-core kernels
    and around the whole chain.

    Two forms of the attention core (with the inverse RoPE of dQ and dK) are
    timed:
      * from the forward's saved output and row statistics, the rotation
        applied as the kernels store dQ and dK (cdml_sdpa_bwd_saved_rope; the
        forward with statistics, cdml_sdpa_fwd_lse, runs once before timing,
        as in the training step).  The device trainer always takes it, and
        the drop-in manager takes cdml_sdpa_bwd_saved whenever it still holds
        the statistics of the forward call on the same arrays;
      * recomputing the row statistics (cdml_sdpa_bwd), then one
        cdml_rope_qk_table launch: the drop-in manager's form when no forward
        on those arrays preceded the call."""
    lib = N.lib()
    cfg = cfg or C3
    B, L, D, H = cfg["batch"], cfg["seq"], cfg["dim"], cfg["heads"]
    hd = D // H
    rows = B * L
    from cdml import synth

    rng = np.random.default_rng(8)
    bufs = {n: N.DeviceBuffer.from_array(rng.standard_normal((rows, D), dtype=np.float32), st)
            for n in ("x", "q", "k", "v", "att", "dy")}
    dw = [N.DeviceBuffer.from_array(synth.xavier_uniform(50 + i, D, D), st) for i in range(4)]
    gw = [N.DeviceBuffer.from_array(np.zeros((D, D), np.float32), st) for _ in range(4)]
    gb = [N.DeviceBuffer.from_array(np.zeros(D, np.float32), st) for _ in range(4)]
    dcat, dq, dk, dv, dxin = (N.DeviceBuffer(rows * D * 4) for _ in range(5))
    wsz, wss, wsl, wsq = C.c_size_t(0), C.c_size_t(0), C.c_size_t(0), C.c_size_t(0)
    N.check(lib.cdml_sdpa_bwd_stored_ds_workspace_size(B, L, L, D, H, 1, C.byref(wsz)))
    N.check(lib.cdml_sdpa_bwd_saved_workspace_size(B, L, L, D, H, 1, C.byref(wss)))
    N.check(lib.cdml_linear_backward_workspace_size(rows, D, D, C.byref(wsl)))
    N.check(lib.cdml_backprop_qkv_workspace_size(rows, D, D, C.byref(wsq)))
    dws = N.DeviceBuffer(max(16, wsz.value))
    dwss = N.DeviceBuffer(max(16, wss.value))
    dwsg = N.DeviceBuffer(max(16, wsl.value, wsq.value))
    s = st.handle
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    b = bufs
    # the forward's saved output and row statistics (untimed, as in the training step)
    osv, lse = N.DeviceBuffer(rows * D * 4), N.DeviceBuffer(B * H * L * 4)
    N.check(lib.cdml_sdpa_fwd_lse(b["q"].ptr, D, b["k"].ptr, D, b["v"].ptr, D, osv.ptr, D, lse.ptr,
                                  B, L, L, D, H, scale, 1, None, s))

    rcs = N.DeviceBuffer(L * hd * 4)
    N.check(lib.cdml_rope_table(rcs.ptr, L, hd, 10000.0, s))

    def core(saved):
        # with the inverse rotation of dQ and dK, as the trainer applies it: fused into the saved form's
        # stores, a separate table-driven launch after the recomputing form
        if saved:
            N.check(lib.cdml_sdpa_bwd_saved_rope(b["q"].ptr, D, b["k"].ptr, D, b["v"].ptr, D, osv.ptr, D, lse.ptr,
                                                 dcat.ptr, D, dq.ptr, D, dk.ptr, D, dv.ptr, D, B, L, L, D, H, scale,
                                                 1, None, rcs.ptr, L, dwss.ptr, wss.value, s))
        else:
            N.check(lib.cdml_sdpa_bwd(b["q"].ptr, D, b["k"].ptr, D, b["v"].ptr, D, dcat.ptr, D, dq.ptr, D,
                                      dk.ptr, D, dv.ptr, D, B, L, L, D, H, scale, 1, None, dws.ptr, wsz.value, s))
            N.check(lib.cdml_rope_qk_table(dq.ptr, dk.ptr, rows, D, hd, H, rcs.ptr, L, 0, L, 1, s))

    def step(saved, t_core=None):
        N.check(lib.cdml_linear_backward(b["att"].ptr, D, b["dy"].ptr, D, dw[3].ptr, dcat.ptr, D, gw[3].ptr,
                                         gb[3].ptr, rows, D, D, 0, dwsg.ptr, wsl.value, s))
        if t_core:
            t_core.start(st)
        core(saved)
        if t_core:
            t_core.stop(st)
        N.check(lib.cdml_backprop_qkv(b["x"].ptr, dq.ptr, dk.ptr, dv.ptr, dw[0].ptr, dw[1].ptr, dw[2].ptr,
                                      gw[0].ptr, gb[0].ptr, gw[1].ptr, gb[1].ptr, gw[2].ptr, gb[2].ptr,
                                      dxin.ptr, rows, D, D, dwsg.ptr, wsq.value, s))

    def timed(saved):
        for _ in range(warmup):
            step(saved)
        st.synchronize()
        tc = Timer(N, steps)
        e0, e1 = N.Event(), N.Event()
        e0.record(st)
        for _ in range(steps):
            step(saved, tc)
        e1.record(st)
        st.synchronize()
        g = dxin.download((rows, D), stream=st)
        assert np.all(np.isfinite(g)), "non-finite MHA backward output"
        return e0.elapsed_ms(e1) / steps, float(np.mean(tc.ms()))

    step_ms, core_ms = timed(True)
    step_rc, core_rc = timed(False)
    pairs = L * (L + 1) // 2
    core_fl = 8 * B * H * hd * pairs          # dV = P^T dO, dP = dO V^T, dQ = dS K, dK = dS^T Q
    proj_fl = 16 * rows * D * D               # out-proj dX + dW, and Q/K/V dX + dW

    def tf(fl, ms):
        return fl / (ms * 1e-3) / 1e12

    return {"ms": round(step_ms, 4), "tflops": round(tf(core_fl + proj_fl, step_ms), 2),
            "attention_core_ms": round(core_ms, 4),
            "attention_core_tflops": round(tf(core_fl, core_ms), 2),
            "attention_core_frac_of_fp32_mfma_peak": round(tf(core_fl, core_ms) / FP32_MFMA_PEAK_TFLOPS, 4),
            "attention_core_form": "cdml_sdpa_bwd_saved_rope: from the forward's saved output and row "
                                   "statistics, the inverse RoPE of dQ and dK applied as they are stored",
            "recomputing_statistics": {
                "ms": round(step_rc, 4), "tflops": round(tf(core_fl + proj_fl, step_rc), 2),
                "attention_core_ms": round(core_rc, 4),
                "attention_core_tflops": round(tf(core_fl, core_rc), 2),
                "attention_core_frac_of_fp32_mfma_peak": round(tf(core_fl, core_rc) / FP32_MFMA_PEAK_TFLOPS, 4),
                "form": "cdml_sdpa_bwd (the row statistics are recomputed by a forward pass inside the call), "
                        "then cdml_rope_qk_table"},
            "flop_count": "matmul FLOPs of the gradients only: 8 x head_dim per causal (query, key) pair "
                          "for the core (no recompute counted), 4 x rows x D^2 per projection"}


def bench_train(H, cfg, batch, seq_inputs, steps, warmup, lr=0.01):
    """Whole TrainBatchDiscrete steps of the DeviceTrainer on one fixed bucket
    of `batch` synthetic token sequences (seq_inputs + 1 tokens each):
    forward with cache, cross-entropy, backward, global-norm clipping and the
    SGD update.  Matmul FLOPs counted as 3x the forward's (forward, then dX
    and dW of every product; the attention core's backward at 8 x head_dim
    per causal pair, recomputation not counted)."""
    from cdml import host, synth

    lm, _ = host.language_model(cfg, synth.lm_weights(cfg, 17))
    tc = H.TrainingConfig()
    t = H.DeviceTrainer(lm, tc, batch, seq_inputs)
    toks = synth.token_ids(23, batch * (seq_inputs + 1), cfg["vocab"]).reshape(batch, seq_inputs + 1)
    ms = t.time_step(toks, lr, steps, warmup)
    D, Hh, L, FF, V = cfg["dim"], cfg["heads"], cfg["layers"], cfg["ff"], cfg["vocab"]
    rows = batch * seq_inputs
    core, qkv, out = mha_flops(batch, seq_inputs, D, Hh)
    fwd = L * (core + qkv + out + 4 * rows * D * FF) + 2 * rows * D * V
    return {"ms": round(ms, 3), "tokens_per_s": round(rows / (ms * 1e-3), 1),
            "tflops": round(3 * fwd / (ms * 1e-3) / 1e12, 2), "gflop_per_step": round(3 * fwd / 1e9, 1)}


EXTRA_LEGS = ("c2_mha_layer", "c3_mha_layer_backward", "c1_text_model_train_step", "c3_shape_train_step",
              "c5_time_series_train_step", "c3_decoder_stack_12_layers", "c3_mha_one_sequence_dropin_host_arrays",
              "c5_time_series_model", "c1_text_model")


def extras(N, st, only=None):
    """End-to-end figures for the other BASELINE configs (device-resident,
    events on the engine's stream) and the PCIe-inclusive drop-in path.
    `only` (a set of EXTRA_LEGS names) restricts the run to those legs."""
    from cdml import host, synth

    H = host.module()
    out = {}
    want = (lambda name: True) if not only else (lambda name: name in only)
    mgr = None
    if want("c2_mha_layer"):
        # c2: one causal MHA layer, B 16 x L 1024, D 512, 8 heads
        c2 = dict(batch=16, seq=1024, dim=512, heads=8)
        # 100 warm-up steps (about 45 ms): after any idle moment the core clock
        # takes some 30 ms of matrix-core load to reach its steady value
        r = bench_mha(N, st, 50, 100, c2)
        core, qkv, o = mha_flops(**c2)
        tf2 = (core + qkv + o) / (r["wall_s"] / 50) / 1e12
        out["c2_mha_layer"] = {"ms": round(r["wall_s"] / 50 * 1e3, 4),
                               "tflops": round(tf2, 2),
                               "frac_of_fp32_mfma_peak": round(tf2 / FP32_MFMA_PEAK_TFLOPS, 4),
                               "tokens_per_s": round(16 * 1024 / (r["wall_s"] / 50), 1),
                               "flash_ms": round(r["flash_ms"], 4)}
    if want("c3_mha_layer_backward"):
        log("[bench] extras: c3 MHA layer backward")
        out["c3_mha_layer_backward"] = bench_mha_backward(N, st, 5, 3)
    if want("c1_text_model_train_step"):
        log("[bench] extras: c1 train step")
        out["c1_text_model_train_step"] = dict(
            bench_train(H, {"vocab": 200, "dim": 64, "heads": 4, "layers": 2, "ff": 128, "max_seq": 64},
                        4, 63, 20, 5),
            workload="TrainBatchDiscrete on 4 sequences of 64 tokens (63 inputs), config-1 text model")
    if want("c3_shape_train_step"):
        log("[bench] extras: c3-shape train step")
        out["c3_shape_train_step"] = dict(
            bench_train(H, {"vocab": 1000, "dim": 1024, "heads": 16, "layers": 12, "ff": 4096, "max_seq": 4096},
                        4, 4095, 3, 1),
            workload="TrainBatchDiscrete on 4 sequences of 4096 tokens, 12 decoder layers D 1024 / 16 heads / "
                     "FF 4096 (config-3 shape) with a 1000-token vocabulary")
    if want("c5_time_series_train_step"):
        log("[bench] extras: c5 train step")
        cfg5t = {"dim": 256, "heads": 8, "layers": 6, "ff": 1024, "max_seq": 512, "discrete": False,
                 "input_dim": 5, "output_dim": 1}
        lm5t, _ = host.language_model(cfg5t, synth.continuous_lm_weights(cfg5t, 19))
        t5 = H.DeviceTrainer(lm5t, H.TrainingConfig(), 256, 511)
        win = synth.random_walk_windows(33, 256, 512, 5)
        tgt = np.ascontiguousarray(win[:, :, :1])  # next-step regression of the first feature
        ms5t = t5.time_step_continuous(win, tgt, 1e-3, 3, 1)
        core, qkv, o = mha_flops(256, 511, 256, 8)
        fwd5 = 6 * (core + qkv + o + 4 * 256 * 511 * 256 * 1024) + 2 * 256 * 511 * 256 * (5 + 1)
        out["c5_time_series_train_step"] = {
            "ms": round(ms5t, 3), "windows_per_s": round(256 / (ms5t * 1e-3), 1),
            "tflops": round(3 * fwd5 / (ms5t * 1e-3) / 1e12, 2),
            "workload": "TrainBatchContinuous (MSE) on 256 windows of 512 steps, config-5 model"}
        del t5, lm5t
    if want("c3_decoder_stack_12_layers"):
        log("[bench] extras: c3 12-layer decoder stack")
        # c3: 12 post-LN decoder layers (MHA + FFN 4096 + 2 LayerNorms) on N(0,1) embeddings
        cfg3 = {"dim": 1024, "heads": 16, "layers": 12, "ff": 4096, "max_seq": 4096, "discrete": False,
                "input_dim": 1024, "output_dim": 1}
        lm3, mgr = host.language_model(cfg3, synth.continuous_lm_weights(cfg3, 41, biased=False))
        dev3 = H.DeviceLanguageModel(lm3, 4)
        x3 = np.random.default_rng(6).standard_normal((4 * 4096, 1024), dtype=np.float32)
        ms3 = dev3.time_layers(x3, 4, 4096, steps=3, warmup=1)
        core, qkv, o = mha_flops(**C3)
        ffn = 4 * 4 * 4096 * 1024 * 4096
        fl3 = 12 * (core + qkv + o + ffn)
        out["c3_decoder_stack_12_layers"] = {
            "ms": round(ms3, 3), "tflops": round(fl3 / (ms3 * 1e-3) / 1e12, 2),
            "frac_of_fp32_mfma_peak": round(fl3 / (ms3 * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4),
            "tokens_per_s": round(4 * 4096 / (ms3 * 1e-3), 1), "gflop": round(fl3 / 1e9, 1)}
        del dev3, lm3
    if mgr is None and any(want(n) for n in EXTRA_LEGS[6:]):
        mgr = H.HipAccelerationManager(0)
    if want("c3_mha_one_sequence_dropin_host_arrays"):
        # drop-in manager path on one c3 sequence: host arrays in and out (PCIe inclusive)
        log("[bench] extras: drop-in manager (host arrays)")
        D, Hh, L = 1024, 16, 4096
        xs = np.random.default_rng(7).standard_normal((L, D), dtype=np.float32)
        wq, wk, wv, wo = (synth.xavier_uniform(60 + i, D, D) for i in range(4))
        bz = np.zeros(D, np.float32)

        def mha_host():
            q, k, v = mgr.ProjectQKV(xs, wq, bz, wk, bz, wv, bz)
            mgr.ApplyRotaryPositionEmbeddingInPlace(q, Hh, 10000.0, False)
            mgr.ApplyRotaryPositionEmbeddingInPlace(k, Hh, 10000.0, False)
            a = mgr.ScaledDotProductAttention(q, k, v, Hh, None, True)
            return mgr.ProjectOutputBatch(a, wo, bz, L, D)

        # warm-up: the first calls after another leg's teardown (hundreds of MB of host
        # and pinned memory returned) run up to twice as long, so the timing starts
        # once the per-sequence cost is steady
        for _ in range(6):
            mha_host()
        s0 = mgr.transfer_stats()
        reps = 10
        t0 = time.perf_counter()
        for _ in range(reps):
            mha_host()
        dt = (time.perf_counter() - t0) / reps
        s1 = mgr.transfer_stats()
        core, qkv, o = mha_flops(1, L, D, Hh)
        pcie = pinned_pcie_bandwidth(N, st)
        out["c3_mha_one_sequence_dropin_host_arrays"] = {
            "ms": round(dt * 1e3, 3), "tflops": round((core + qkv + o) / dt / 1e12, 3),
            "h2d_mib_per_sequence": round((s1["h2d_bytes"] - s0["h2d_bytes"]) / reps / 2**20, 2),
            "d2h_mib_per_sequence": round((s1["d2h_bytes"] - s0["d2h_bytes"]) / reps / 2**20, 2),
            "h2d_mib_saved_per_sequence": round((s1["h2d_skipped_bytes"] - s0["h2d_skipped_bytes"]) / reps / 2**20, 2),
            "pinned_pcie_gbs": pcie, "host_copy_threads": H.host_copy_threads(),
            "note": "HipAccelerationManager with float[,]-style host arrays (PCIe included): each call "
                    "stages its transfers through pinned memory; returned activations stay on the device "
                    "and are uploaded again only when the shadow compare finds a host change; weights "
                    "stay resident"}
    if want("c5_time_series_model"):
        # c5: time-series regression transformer, full forward, B 256 x L 512
        log("[bench] extras: c5 time-series model")
        cfg5 = {"dim": 256, "heads": 8, "layers": 6, "ff": 1024, "max_seq": 512, "discrete": False,
                "input_dim": 5, "output_dim": 1}
        lm5, _ = host.language_model(cfg5, synth.continuous_lm_weights(cfg5, 21), mgr)
        dev5 = H.DeviceLanguageModel(lm5, 256)
        x5 = synth.random_walk_windows(31, 256, 512, 5).reshape(256 * 512, 5)
        ms5 = dev5.time_forward(x5, 256, 512, steps=5, warmup=2, continuous=True)
        core, qkv, o = mha_flops(256, 512, 256, 8)
        fl5 = 6 * (core + qkv + o + 4 * 256 * 512 * 256 * 1024) + 2 * 256 * 512 * 256 * (5 + 1)
        del dev5, lm5
        # the model's attention shape alone (d_h 32): flash kernel by events
        r5 = bench_mha(N, st, 10, 20, dict(batch=256, seq=512, dim=256, heads=8))
        core5 = mha_flops(256, 512, 256, 8)[0]
        fa5 = core5 / (r5["flash_ms"] * 1e-3) / 1e12
        tf5 = fl5 / (ms5 * 1e-3) / 1e12
        out["c5_time_series_model"] = {"ms": round(ms5, 3), "tflops": round(tf5, 2),
                                       "frac_of_fp32_mfma_peak": round(tf5 / FP32_MFMA_PEAK_TFLOPS, 4),
                                       "windows_per_s": round(256 / (ms5 * 1e-3), 1),
                                       "tokens_per_s": round(256 * 512 / (ms5 * 1e-3), 1),
                                       "attention_kernel_ms": round(r5["flash_ms"], 4),
                                       "attention_kernel_tflops": round(fa5, 2),
                                       "attention_kernel_frac_of_fp32_mfma_peak":
                                           round(fa5 / FP32_MFMA_PEAK_TFLOPS, 4)}
    if want("c1_text_model"):
        # c1: README text model, forward of 4 x 64 tokens and greedy generation of 20 tokens
        log("[bench] extras: c1 text model")
        cfg1 = {"vocab": 200, "dim": 64, "heads": 4, "layers": 2, "ff": 128, "max_seq": 64}
        lm1, _ = host.language_model(cfg1, synth.lm_weights(cfg1, 7), mgr)
        dev1 = H.DeviceLanguageModel(lm1, 4)
        ids = synth.token_ids(11, 4 * 64, 200).reshape(4, 64)
        ms1 = dev1.time_forward(ids, 4, 64, steps=50, warmup=50)
        dev1.GenerateGreedy(ids[:, :32], 20)
        t0 = time.perf_counter()
        for _ in range(5):
            dev1.GenerateGreedy(ids[:, :32], 20)
        gen_ms = (time.perf_counter() - t0) / 5 * 1e3
        # forward matmul FLOPs: 2 layers of MHA and FFN 64 -> 128 -> 64, and the LM head
        core1, qkv1, o1 = mha_flops(4, 64, 64, 4)
        fl1 = 2 * (core1 + qkv1 + o1 + 4 * 256 * 64 * 128) + 2 * 256 * 64 * 200
        tf1 = fl1 / (ms1 * 1e-3) / 1e12
        out["c1_text_model"] = {"forward_ms": round(ms1, 4),
                                "forward_tokens_per_s": round(256 / (ms1 * 1e-3), 1),
                                "forward_tflops": round(tf1, 3),
                                "forward_frac_of_fp32_mfma_peak": round(tf1 / FP32_MFMA_PEAK_TFLOPS, 5),
                                "note": "latency-bound (44 MFLOP per forward)",
                                "generate_20_tokens_batch4_ms": round(gen_ms, 3),
                                "generated_tokens_per_s": round(80 / (gen_ms * 1e-3), 1)}
    return out


def host_cpu_info():
    """The host's processor count as .NET's Environment.ProcessorCount reads it
    on Linux (the CPUs in the process's affinity mask, lowered to the cgroup
    CPU quota when one is set), which AccelerationMutliThreadCPU uses as its
    degree of parallelism (AccelerationMutliThreadCPU.cs:61-69), plus nproc and
    the CPU model.  The threads used are that count, capped at this box's CPU
    share for one GPU when the box announces one through OMP_NUM_THREADS."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = os.cpu_count() or 1
    quota = None
    try:
        q, p = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = max(1, -(-int(q) // int(p)))
    except (OSError, ValueError):
        pass
    proc_count = min(affinity, quota) if quota else affinity
    share = os.environ.get("OMP_NUM_THREADS", "")
    share = int(share) if share.isdigit() and int(share) > 0 else None
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    used = min(proc_count, share) if share else proc_count
    return {"processor_count": proc_count, "nproc": affinity, "os_cpu_count": os.cpu_count(),
            "cgroup_cpu_quota": quota, "box_cpu_share": share, "threads_used": used, "cpu_model": model}


def pinned_pcie_bandwidth(N, st, mib=256, reps=5):
    """Host<->device copy rate between pinned host memory and HBM (GB/s), the
    bound of the drop-in manager's staged transfers."""
    lib = N.lib()
    nbytes = mib << 20
    hp = C.c_void_p()
    N.check(lib.cdml_host_alloc_pinned(C.byref(hp), nbytes))
    d = N.DeviceBuffer(nbytes)
    res = {}
    try:
        for name, fn, args in (("h2d", lib.cdml_memcpy_h2d_async, (d.ptr, hp.value)),
                               ("d2h", lib.cdml_memcpy_d2h_async, (hp.value, d.ptr))):
            N.check(fn(*args, nbytes, st.handle))
            st.synchronize()
            e0, e1 = N.Event(), N.Event()
            e0.record(st)
            for _ in range(reps):
                N.check(fn(*args, nbytes, st.handle))
            e1.record(st)
            ms = e0.elapsed_ms(e1) / reps
            res[name] = round(nbytes / (ms * 1e-3) / 1e9, 1)
    finally:
        d.free()
        lib.cdml_host_free_pinned(hp.value)
    return res


def _mt_mha(O, x, ws, bs, H):
    """MultiHeadAttention.Forward's calls on the multi-threaded restatement:
    ProjectQKV, RoPE of Q and K, causal ScaledDotProductAttention,
    ProjectOutputBatch (AccelerationMutliThreadCPU.cs:798-831, 3910-3985,
    1991-2098, 2331-2359)."""
    q, k, v = O.project_qkv(x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], mt=True)
    q, k = O.rope(q, H, mt=True), O.rope(k, H, mt=True)
    return O.project_output_batch(O.sdpa(q, k, v, H, causal=True, mt=True), ws[3], bs[3], mt=True)


def _mt_block(O, x, ws, bs, ff, H):
    """TransformerBlock.Forward (TransformerBlock.cs:35-44) on the
    multi-threaded restatement: MHA, residual LayerNorm, FFN [D, FF, D] with
    ReLU (BatchDotProductAddBias, :1694-1740), residual LayerNorm
    (:3988-4018)."""
    g, z = np.ones(x.shape[1], np.float32), np.zeros(x.shape[1], np.float32)
    n1 = O.residual_layernorm(x, _mt_mha(O, x, ws, bs, H), g, z, mt=True)
    h = O.activation(O.batch_dot_add_bias(ff[0], n1, ff[1], mt=True), 3)
    return O.residual_layernorm(n1, O.batch_dot_add_bias(ff[2], h, ff[3], mt=True), g, z, mt=True)


def _timed_units(fn, units, reps=1):
    """One untimed warm-up call on a full-size unit, then `reps` timed passes
    over all `units`; returns the seconds of each pass."""
    fn(units[0])
    out = []
    for _ in range(reps):
        t0 = time.perf_counter()
        for u in units:
            fn(u)
        out.append(time.perf_counter() - t0)
    return out


def cpu_baseline(sample_seqs=3):
    """The multi-threaded CPU restatement of AccelerationMutliThreadCPU's
    ProjectQKV / RoPE / ScaledDotProductAttention / ProjectOutputBatch
    (oracle/refcpu_mt.c) on `sample_seqs` of the c3 batch's sequences, one
    LanguageModel.Forward-style call per sequence, after one untimed
    full-size sequence.  Timed, not checked."""
    from oracle import oracle as O
    from cdml import synth

    host = host_cpu_info()
    threads = host["threads_used"]
    O.set_threads(threads)
    L, D, H = C3["seq"], C3["dim"], C3["heads"]
    rng = np.random.default_rng(5)
    ws = [synth.xavier_uniform(30 + i, D, D) for i in range(4)]
    bs = [np.zeros(D, np.float32)] * 4
    xs = [rng.standard_normal((L, D), dtype=np.float32) for _ in range(sample_seqs)]
    dt = _timed_units(lambda x: _mt_mha(O, x, ws, bs, H), xs)[0]
    core, qkv, out = mha_flops(sample_seqs, L, D, H)
    return dict(value=(core + qkv + out) / dt / 1e12, unit="TFLOP/s", cores=threads, kind="port",
                seconds=dt, host=host,
                sample=f"{sample_seqs} of the 4 c3 sequences (L 4096, D 1024, H 16), full MHA forward "
                       f"through the C restatement of AccelerationMutliThreadCPU (-O2, no fast-math), "
                       f"after one untimed full-size sequence, "
                       f"{threads} threads (Environment.ProcessorCount equivalent {host['processor_count']}, "
                       f"nproc {host['nproc']}, box share {host['box_cpu_share']}) on {host['cpu_model']}, "
                       f"{dt:.1f} s")


def cpu_baseline_other_configs(threads, c3_mha_s_per_seq):
    """The same restatement on bounded samples of the other configs, each
    after one untimed full-size unit (a sequence, a window, a decode row):

    * c2: the MHA layer forward, 4 of the 16 sequences, 3 timed passes.
    * c3: one decoder layer (MHA + residual LayerNorm + FFN 4096 + residual
      LayerNorm) on one sequence; the MHA-only layer is the headline leg.  The
      4-sequence 12-layer stack time is extrapolated from these and labelled so.
    * c5: the MHA layer and the whole decoder layer, 64 of the 256 windows
      each; the 6-layer figure is extrapolated.
    * c4: the decode step, whose reference (LanguageModel.DecoderSelfAttention-
      Step) is inline and single-threaded: sequentially over 8 of the 64 rows
      as the reference runs it, and with the rows spread over the threads
      (labelled); 3 timed passes each.
    * c1: the config-1 text model through the single-threaded restatement of
      LanguageModel.Forward (4 sequences of 64 tokens) and Generate (greedy,
      20 new tokens after 32-token prompts), 3 timed passes.
    Timed, not checked."""
    from oracle import oracle as O
    from cdml import synth

    out = {}
    rng = np.random.default_rng(6)
    r6 = lambda v: round(v, 6)
    # c2: MHA layer
    B, L, D, H, n = 16, 1024, 512, 8, 4
    ws = [synth.xavier_uniform(40 + i, D, D) for i in range(4)]
    bs = [np.zeros(D, np.float32)] * 4
    xs = [rng.standard_normal((L, D), dtype=np.float32) for _ in range(n)]
    t = _timed_units(lambda x: _mt_mha(O, x, ws, bs, H), xs, reps=3)
    core, qkv, o = mha_flops(n, L, D, H)
    med = float(np.median(t))
    out["c2"] = {"value": r6((core + qkv + o) / med / 1e12), "unit": "TFLOP/s", "seconds_per_pass": [r6(v) for v in t],
                 "sample": f"{n} of the {B} sequences (L {L}, D {D}, H {H}), MHA layer forward, one untimed "
                           f"sequence then 3 timed passes (median), {threads} threads"}
    # c3 and c5: MHA layer, and MHA + FFN + 2 LayerNorms
    for name, (B, L, D, H, FF, nl, n) in (("c3", (4, 4096, 1024, 16, 4096, 12, 1)),
                                          ("c5", (256, 512, 256, 8, 1024, 6, 64))):
        ws = [synth.xavier_uniform(50 + i, D, D) for i in range(4)]
        bs = [np.zeros(D, np.float32)] * 4
        ff = [synth.xavier_uniform(60, FF, D), np.zeros(FF, np.float32), synth.xavier_uniform(61, D, FF),
              np.zeros(D, np.float32)]
        xs = [rng.standard_normal((L, D), dtype=np.float32) for _ in range(n)]
        core, qkv, o = mha_flops(n, L, D, H)
        mha_fl = core + qkv + o
        ffn_fl = 2 * 2 * n * L * D * FF
        leg = {}
        if name == "c5":
            t_mha = _timed_units(lambda x: _mt_mha(O, x, ws, bs, H), xs)[0]
            leg["mha_layer"] = {"value": r6(mha_fl / t_mha / 1e12), "unit": "TFLOP/s", "seconds": r6(t_mha)}
        else:
            t_mha = c3_mha_s_per_seq * n
            leg["mha_layer"] = {"value": r6(mha_fl / t_mha / 1e12), "unit": "TFLOP/s", "seconds": r6(t_mha),
                                "from": "the headline cpu_baseline leg"}
        t_blk = _timed_units(lambda x: _mt_block(O, x, ws, bs, ff, H), xs)[0]
        leg["decoder_layer"] = {"value": r6((mha_fl + ffn_fl) / t_blk / 1e12), "unit": "TFLOP/s",
                                "seconds": r6(t_blk)}
        per_seq = t_blk / n
        leg[f"stack_{nl}_layers_batch_{B}_extrapolated"] = {
            "seconds": round(per_seq * nl * B, 2), "tokens_per_s": round(B * L / (per_seq * nl * B), 1),
            "how": f"extrapolated: the timed decoder layer's seconds per sequence x {nl} layers x {B} "
                   f"sequences, not run"}
        leg["sample"] = (f"{n} of the {B} sequences (L {L}, D {D}, H {H}, FF {FF}), one untimed sequence per "
                         f"form, {threads} threads")
        out[name] = leg
    # c4: decode
    B, T, D, H = 8, C4["t"], C4["dim"], C4["heads"]
    q = rng.standard_normal((B, D), dtype=np.float32)
    kc = rng.standard_normal((B, T, D), dtype=np.float32)
    vc = rng.standard_normal((B, T, D), dtype=np.float32)
    lens = np.full(B, T, np.int32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D // H)))
    nbytes = decode_bytes(B, T, D)
    dec = {}
    for label, parallel in (("sequential", False), ("parallel_over_batch", True)):
        O.decode_attention_batch(q[:1], kc[:1], vc[:1], lens[:1], H, scale, parallel)  # one full-size row
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            O.decode_attention_batch(q, kc, vc, lens, H, scale, parallel)
            ts.append(time.perf_counter() - t0)
        dt = float(np.median(ts))
        dec[label] = {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s",
                      "ms_per_step_of_64": round(dt / B * 64 * 1e3, 3)}
    dec["sample"] = (f"{B} of the 64 decode rows (KV {T}, D {D}, H {H}), one untimed row then 3 timed passes "
                     f"(median); the sequential form runs one thread as the reference's inline step does, the "
                     f"parallel one spreads the rows over {threads} threads")
    out["c4_decode"] = dec
    # c1: the README text model, forward and greedy generation
    cfg = {"vocab": 200, "dim": 64, "heads": 4, "layers": 2, "ff": 128, "max_seq": 64}
    lm = O.LanguageModel(cfg, synth.lm_weights(cfg, 5, biased=True))
    ids = synth.token_ids(7, 4 * 64, 200).reshape(4, 64)
    fwd = _timed_units(lambda s: lm.forward(s), list(ids), reps=3)
    gen = _timed_units(lambda s: lm.generate_greedy(s[:32], 20), list(ids), reps=3)
    out["c1"] = {"forward_ms": round(float(np.median(fwd)) * 1e3, 3),
                 "generate_20_tokens_batch4_ms": round(float(np.median(gen)) * 1e3, 3),
                 "tokens_per_s_generate": round(4 * 20 / float(np.median(gen)), 1), "cores": 1,
                 "sample": "the whole config (4 sequences of 64 tokens; 4 prompts of 32 tokens, 20 greedy tokens "
                           "each, one sequence at a time as LanguageModel.Forward / Generate run), single-threaded "
                           "restatement of AccelerationCPU, one untimed sequence then 3 timed passes (median)"}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--only", default="",
                    help="run only these comma-separated legs of " + ", ".join(EXTRA_LEGS) +
                         " and print their figures (no headline metric line); for kernel traces")
    args = ap.parse_args()
    only = {n for n in args.only.split(",") if n}
    if only - set(EXTRA_LEGS):
        ap.error(f"--only: unknown legs {sorted(only - set(EXTRA_LEGS))}")
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the attention path is single-device by design "
              "(batch x head shards need no exchange); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from cdml import native as N

    N.init(0)
    info = N.device_info(0)
    log(f"[bench] device {info['name']} {info['arch']} CUs {info['compute_units']} "
        f"sclk {info['max_clock_mhz']} MHz")
    st = N.Stream()
    if only:
        # profiling mode: the selected legs alone, so a kernel trace holds only their launches
        print(json.dumps({"other_configs": extras(N, st, only)}), flush=True)
        return

    mha = bench_mha(N, st, args.steps, args.warmup)
    core, qkv, out = mha_flops(**C3)
    total = core + qkv + out
    ms_per_step = mha["wall_s"] / args.steps * 1e3
    value = total / (ms_per_step * 1e-3) / 1e12
    flash_tflops = core / (mha["flash_ms"] * 1e-3) / 1e12
    traffic_c3, prov_c3 = measured_traffic("flash_c3")
    res = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: x ~ N(0,1), Wq/Wk/Wv/Wo Xavier-uniform, zero biases, causal",
        "config": {"workload": "c3 causal MHA layer forward (QKV proj + RoPE + flash SDPA + out proj)",
                   "batch": C3["batch"], "seq_len": C3["seq"], "d_model": C3["dim"],
                   "heads": C3["heads"], "head_dim": C3["dim"] // C3["heads"], "parallelism": "none"},
        "frac_of_fp32_mfma_peak": round(value / FP32_MFMA_PEAK_TFLOPS, 4),
        "selfcheck": {"rows": "sequence 0, rows 0-63, against float64 numpy", "tolerance": "1e-4 + 1e-3 |ref|",
                      "max_abs_err": mha["selfcheck_max_abs_err"]},
        "tokens_per_s": round(C3["batch"] * C3["seq"] / (ms_per_step * 1e-3), 1),
        "kernels_ms": {"project_qkv_rope": round(mha["qkv_ms"], 4), "flash_sdpa": round(mha["flash_ms"], 4),
                       "out_proj": round(mha["out_ms"], 4), "step_events": round(mha["dev_ms"], 4)},
        "roofline": {"kernel": "flash_fwd_kernel (cdml_sdpa_fwd, c3)", "bound": "mfma",
                     "achieved": round(flash_tflops, 3), "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(flash_tflops / FP32_MFMA_PEAK_TFLOPS, 4),
                     "traffic": traffic_c3, "traffic_provenance": prov_c3,
                     "algorithmic_per_launch": core},
        "device": {k: info[k] for k in ("name", "arch", "compute_units", "max_clock_mhz")},
    }
    if not args.no_decode:
        log("[bench] c4 decode")
        dec = bench_decode(N, st, max(args.steps, 10), args.warmup)
        nbytes = decode_bytes(C4["batch"], C4["t"], C4["dim"])
        gbs = nbytes / (dec["ms"] * 1e-3) / 1e9
        traffic_c4, prov_c4 = measured_traffic("decode_c4")
        res["decode"] = {"workload": "c4 decode step (B 64, KV 8192, 16 heads x 128)",
                         "ms": round(dec["ms"], 4), "tokens_per_s": round(C4["batch"] / (dec["ms"] * 1e-3), 1),
                         "roofline": {"kernel": "decode_split_kernel + decode_combine_vec_kernel", "bound": "hbm",
                                      "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                      "frac": round(gbs / HBM_PEAK_GBS, 4),
                                      "traffic": traffic_c4, "traffic_provenance": prov_c4,
                                      "algorithmic_per_launch": nbytes}}
    if not args.no_extras:
        log("[bench] extras")
        res["other_configs"] = extras(N, st, only)
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (multi-threaded restatement)")
        cb = cpu_baseline()
        res["cpu_baseline"] = {k: (round(v, 6) if isinstance(v, float) else v) for k, v in cb.items()}
        res["cpu_baseline"]["other_configs"] = cpu_baseline_other_configs(cb["cores"], cb["seconds"] / 3)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()

"""Throughput of the fused-op hot path on one MI355X.

Workload (one step): SwiGLU forward + backward on gate, up [8192, 6144] bf16
and RoPE forward + backward on q [4, 16, 2048, 128], k [4, 8, 2048, 128]
bf16 with positions 0..2047, theta 1e6, cos/sin computed in-kernel. Inputs
~N(0, 1) drawn on the CPU from seeded generators, resident in HBM before the
timed region; consecutive steps alternate between two copies of every input
(1 GB each), so no step re-reads operands the previous step left in the
256 MB MALL.

value = algorithmic bytes per step / time per step, where algorithmic bytes
count each input read once and each output written once:
  SwiGLU fwd 3*N*I*2 + bwd 5*N*I*2 = 805,306,368 B
  RoPE   fwd (read + write q, k) + bwd (same) = 201,326,592 B
roofline: the dominant kernel (SwiGLU backward, 503,316,480 B per launch),
its launch duration measured cold (MALL and L2 flushed by a 512 MB write
before each of 25 reps, median, HIP events on its stream), against 8 TB/s.
cpu_baseline: the oracle (a CPU restatement of the reference's torch ops)
on a bounded sample of the same workload, on the host's cores;
cpu_baselines: the same per config (RMSNorm, SwiGLU, RoPE, LoRA backward,
FLCE, train step) on bounded samples; --cpu-full runs them at full shape.
breakdown: each op's cold median (and warm back-to-back) launch time; plus,
outside the step, RMSNorm fp32, the residual add + RMSNorm and the q/k norm
+ RoPE (all cold); chunked FLCE fwd+bwd (hidden [8192, 2048], lm_head
[151936, 2048], chunk 8192: 15.29 TFLOP, with its peak extra memory) and
the fused LoRA backward of a Qwen3-style 2B layer (QKV + MLP, rank 16:
774.2 GFLOP), as TFLOP/s against the 2.5 PFLOP/s bf16 peak (medians of 20
reps); and the 4-layer Qwen3-style LoRA train step (batch 4 x 2048 tokens,
every fused op patched in, FLCE loss, AdamW on the adapters) in tokens/s.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--no-mfma-ops]
       [--no-train-step] [--train-step-only] [--cpu-full] [--pmc-probe] [--pmc-mfma-probe]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
N_TOK, INTER = 8192, 6144
RB, RHQ, RHK, RS, RD = 4, 16, 8, 2048, 128
THETA = 1e6
SWIGLU_FWD_BYTES = 3 * N_TOK * INTER * 2
SWIGLU_BWD_BYTES = 5 * N_TOK * INTER * 2
ROPE_DIR_BYTES = 2 * RB * (RHQ + RHK) * RS * RD * 2       # read + write q and k
STEP_BYTES = SWIGLU_FWD_BYTES + SWIGLU_BWD_BYTES + 2 * ROPE_DIR_BYTES
METRIC = "fused-op fwd+bwd GB/s (% HBM peak); LoRA layer train-step tokens/sec"


def seeded(shape, seed, dtype):
    import torch
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32).to(dtype)


FLCE_N, FLCE_H, FLCE_V, FLCE_CHUNK = 8192, 2048, 151936, 8192
FLCE_FLOP = 3 * 2 * FLCE_N * FLCE_V * FLCE_H                 # logits, dH, dW
LORA_N, LORA_H, LORA_KV, LORA_I, LORA_R = 8192, 2048, 1024, 6144, 16
LORA_BWD_FLOP = 774_167_855_104                             # QKV + MLP backward, necessary FLOPs
MFMA_PEAK_TFLOPS = 2500.0


def gpu_randn(shape, seed, dev, scale=1.0, dtype=None):
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    t = torch.randn(*shape, generator=g, device=dev, dtype=torch.float32)
    if scale != 1.0:
        t.mul_(scale)
    return t.to(dtype or torch.bfloat16)


def time_launches(fn, stream, reps):
    """Average milliseconds per call over `reps` back-to-back calls (events on
    the stream the kernels are launched on): the warm rate, operands partly
    resident in the MALL / L2 when they fit there."""
    import torch
    fn()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        fn()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


FLUSH_BYTES = 512 << 20   # twice the 256 MB MALL, far beyond the 8 x 4 MB L2


class ColdTimer:
    """Launch time with the MALL and L2 flushed before every rep: each rep
    writes a 512 MB buffer and reads another, then runs fn; the same flush is timed alone in
    interleaved reps. time(fn) = median over reps of (flush + fn) minus the
    median of (flush alone), from events on the launch stream; no event sits
    between the flush and fn, so the inter-event gap of an event record does
    not land on fn, and fn's host-side launch is enqueued while the flush
    still runs."""

    def __init__(self, dev, stream):
        import torch
        self.stream = stream
        self.buf = torch.empty(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)
        self.rbuf = torch.ones(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)
        self.sink = torch.empty((), dtype=torch.float32, device=dev)

    def flush(self):
        import torch
        # the write evicts the op's data; the read of another 512 MB then
        # replaces the write's dirty lines with clean ones, so their
        # write-back happens inside the flush (timed and subtracted)
        self.buf.fill_(1.0)
        torch.sum(self.rbuf, dim=(0,), out=self.sink)

    def time(self, fn, reps=25):
        import statistics

        import torch
        fn()
        self.flush()
        torch.cuda.synchronize()
        E = torch.cuda.Event
        pairs = [[(E(enable_timing=True), E(enable_timing=True)) for _ in range(2)] for _ in range(reps)]
        for (fa, fb), (ta, tb) in pairs:
            fa.record(self.stream)
            self.flush()
            fb.record(self.stream)
            ta.record(self.stream)
            self.flush()
            fn()
            tb.record(self.stream)
        torch.cuda.synchronize()
        fl = [fa.elapsed_time(fb) for (fa, fb), _ in pairs]
        tot = [ta.elapsed_time(tb) for _, (ta, tb) in pairs]
        ops = sorted(t - f for t, f in zip(tot, fl))
        med = statistics.median(tot) - statistics.median(fl)
        return {"ms": med, "p10_ms": ops[len(ops) // 10], "p90_ms": ops[(9 * len(ops)) // 10],
                "reps": reps}


def time_rotating(fns, stream, rounds=6):
    """Average ms per launch over back-to-back launches that cycle through
    `fns` (the same op bound to different copies of its inputs, enough
    copies that their working set exceeds the 256 MB MALL, so every launch
    reads its operands from HBM), replayed from one captured HIP graph of
    rounds x len(fns) launches (no per-call host marshalling in the timed
    interval; same-stream kernels still run one after another)."""
    import torch
    n = rounds * len(fns)
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        for fn in fns:
            fn()
    stream.wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(rounds):
            for fn in fns:
                fn()
    g.replay()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(3):
        a.record(stream)
        g.replay()
        b.record(stream)
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) / n)
    del g
    return min(times)


COPY_BYTES = 256 << 20   # per copy: 256 MB read + 256 MB written


def copy_ceiling(dev, stream):
    """What a plain device-to-device copy sustains from HBM on this GPU
    (torch's copy_ of 256 MB, two source/destination pairs in rotation: a
    1 GB working set beyond the MALL), timed like the ops' rotating-input
    lines: the practical ceiling the streaming kernels' GB/s compare with."""
    import torch
    n = COPY_BYTES // 2
    pairs = [(torch.empty(n, dtype=torch.bfloat16, device=dev).fill_(1.0),
              torch.empty(n, dtype=torch.bfloat16, device=dev)) for _ in range(2)]
    ms = time_rotating([lambda s=s, d=d: d.copy_(s) for s, d in pairs], stream)
    nbytes = 2 * COPY_BYTES
    del pairs
    return {"bytes": nbytes, "us": round(ms * 1e3, 2), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "what": "torch copy_ of 256 MB bf16 (read + write), 2 pairs in rotation, graph replay"}


def rotating_copies(nbytes_per_launch):
    """Input copies needed so one round of launches touches > 512 MB."""
    return max(2, -(-(FLUSH_BYTES) // max(nbytes_per_launch, 1)))


def cold_line(res, nbytes=None, flop=None, rot_ms=None):
    """Fields of one cold-timed op: the rotating-input launch time (us,
    GB/s, hbm_frac: what the kernel sustains from HBM) when given, and the
    flushed single-launch median (flushed_us, with p10/p90 and GB/s, which
    also holds the launch's dispatch gap)."""
    out = {}
    if rot_ms is not None and nbytes:
        out["us"] = round(rot_ms * 1e3, 2)
        out["GB/s"] = round(nbytes / (rot_ms * 1e-3) / 1e9, 1)
        out["hbm_frac"] = round(nbytes / (rot_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    out.update({"flushed_us": round(res["ms"] * 1e3, 2), "flushed_p10_us": round(res["p10_ms"] * 1e3, 2),
                "flushed_p90_us": round(res["p90_ms"] * 1e3, 2)})
    if nbytes:
        out["flushed_GB/s"] = round(nbytes / (res["ms"] * 1e-3) / 1e9, 1)
    if flop:
        out["TFLOP/s"] = round(flop / (res["ms"] * 1e-3) / 1e12, 1)
    return out


TIMING_NOTE = ("us / GB/s / hbm_frac: back-to-back launches cycling through copies of the inputs "
               "whose working set exceeds the 256 MB MALL (every launch reads HBM), replayed from a "
               "captured graph; flushed_*: MALL/L2 flushed before each rep by a 512 MB write then "
               "a 512 MB read (caches clean, none of the op's data), median of 25 reps of "
               "(flush + op) minus the median of (flush alone), dispatch gap included")


RMS_N, RMS_H = 8192, 2048
RMS_FWD_BYTES = 2 * RMS_N * RMS_H * 4 + RMS_H * 4 + RMS_N * 4          # x, w in; y, rrms out
RMS_BWD_BYTES = 3 * RMS_N * RMS_H * 4 + 2 * RMS_H * 4 + RMS_N * 4      # x, dy, w, rrms in; dx, dw out


def bench_rmsnorm(dev, timer):
    """RMSNorm fwd and bwd, fp32 x [8192, 2048], weight 1 + 0.1 N(0, 1),
    eps 1e-6 (rrms saved by the forward, as the autograd Function does)."""
    from metal_liger_amd import hip_ops
    import torch
    x = gpu_randn((RMS_N, RMS_H), 40, dev, dtype=torch.float32)
    w = (1.0 + 0.1 * gpu_randn((RMS_H,), 41, dev, dtype=torch.float32))
    dy = gpu_randn((RMS_N, RMS_H), 42, dev, dtype=torch.float32)
    _, rrms = hip_ops.rms_norm_fwd(x, w, 1e-6)
    f = timer.time(lambda: hip_ops.rms_norm_fwd(x, w, 1e-6))
    b = timer.time(lambda: hip_ops.rms_norm_bwd(x, w, dy, rrms, 1e-6))
    C = rotating_copies(RMS_FWD_BYTES)
    cp = [(x.clone(), dy.clone(), rrms.clone()) for _ in range(C)]
    rf = time_rotating([lambda t=t: hip_ops.rms_norm_fwd(t[0], w, 1e-6) for t in cp], timer.stream)
    rb = time_rotating([lambda t=t: hip_ops.rms_norm_bwd(t[0], w, t[1], t[2], 1e-6) for t in cp],
                       timer.stream)
    del cp
    tot = rf + rb
    return {"fwd": cold_line(f, RMS_FWD_BYTES, rot_ms=rf), "bwd": cold_line(b, RMS_BWD_BYTES, rot_ms=rb),
            "fwd_bwd_GB/s": round((RMS_FWD_BYTES + RMS_BWD_BYTES) / (tot * 1e-3) / 1e9, 1),
            "fwd_bwd_hbm_frac": round((RMS_FWD_BYTES + RMS_BWD_BYTES) / (tot * 1e-3) / 1e9
                                      / HBM_PEAK_GBS, 4),
            "bwd_note": "includes the fixed-order dW partial-row reduction launch"}


ADD_N, ADD_H = 8192, 2048
ADD_FWD_BYTES = 4 * ADD_N * ADD_H * 2 + ADD_H * 2 + ADD_N * 4      # x, res, w in; sum, y, rrms out
ADD_BWD_BYTES = 4 * ADD_N * ADD_H * 2 + 2 * ADD_H * 2 + ADD_N * 4  # sum, dy, dsum, w, rrms in; dx, dw out


def bench_add_rmsnorm(dev, timer):
    """Residual add fused into RMSNorm (a decoder layer's post-attention
    step), bf16 hidden states [8192, 2048], bf16 weight 1 + 0.1 N(0, 1),
    eps 1e-6; beside it the unfused pair (torch's add, then the fused norm;
    the norm's backward, then torch's add)."""
    from metal_liger_amd import hip_ops
    x = gpu_randn((ADD_N, ADD_H), 45, dev)
    res = gpu_randn((ADD_N, ADD_H), 46, dev)
    w = 1.0 + 0.1 * gpu_randn((ADD_H,), 47, dev)
    dy = gpu_randn((ADD_N, ADD_H), 48, dev)
    ds = gpu_randn((ADD_N, ADD_H), 49, dev)
    _, total, rrms = hip_ops.rms_norm_add_fwd(x, res, w, 1e-6)
    f = timer.time(lambda: hip_ops.rms_norm_add_fwd(x, res, w, 1e-6))
    b = timer.time(lambda: hip_ops.rms_norm_bwd(total, w, dy, rrms, 1e-6, dsum=ds))
    C = rotating_copies(ADD_FWD_BYTES)
    cp = [(x.clone(), res.clone(), total.clone(), dy.clone(), ds.clone(), rrms.clone())
          for _ in range(C)]
    rf = time_rotating([lambda t=t: hip_ops.rms_norm_add_fwd(t[0], t[1], w, 1e-6) for t in cp],
                       timer.stream)
    rb = time_rotating([lambda t=t: hip_ops.rms_norm_bwd(t[2], w, t[3], t[5], 1e-6, dsum=t[4])
                        for t in cp], timer.stream)
    ruf = time_rotating([lambda t=t: hip_ops.rms_norm_fwd(t[0] + t[1], w, 1e-6) for t in cp],
                        timer.stream)
    rub = time_rotating([lambda t=t: hip_ops.rms_norm_bwd(t[2], w, t[3], t[5], 1e-6)[0] + t[4]
                         for t in cp], timer.stream)
    del cp
    return {"fwd": cold_line(f, ADD_FWD_BYTES, rot_ms=rf), "bwd": cold_line(b, ADD_BWD_BYTES, rot_ms=rb),
            "unfused_fwd_us": round(ruf * 1e3, 2), "unfused_bwd_us": round(rub * 1e3, 2)}


def flce_reference_peak_bytes(N, V, H, chunk):
    """Peak extra device memory of the reference's Function in its backward
    (ops/fused_linear_cross_entropy.py:159-185): fp32 copies of hidden and
    weight, fp32 grad_hidden and grad_weight, about three live fp32 [N, chunk]
    temporaries (logit_chunk, prob_chunk, the masked product) and the final
    bf16 cast of grad_weight while its fp32 buffer is alive."""
    return 2 * N * H * 4 + 2 * V * H * 4 + 3 * N * chunk * 4 + V * H * 2


def bench_flce(dev, timer, reps=20, token_chunk=None):
    """Fused linear cross-entropy fwd + bwd as the autograd Function runs it:
    hidden [8192, 2048], lm_head [151936, 2048] ~N(0, 0.02), no bias, 10% of
    labels ignored; the forward forms loss, dH and dW in one pass (logits
    computed once), the backward applies grad_output. 15.29 TFLOP of
    necessary GEMM work (logits, dH, dW) per fwd+bwd. Peak extra memory: the
    allocator's peak above the inputs during one fwd + bwd (workspace plus
    the dH / dW outputs)."""
    import torch

    from metal_liger_amd import hip_ops
    h = gpu_randn((FLCE_N, FLCE_H), 10, dev)
    w = gpu_randn((FLCE_V, FLCE_H), 11, dev, 0.02)
    g = torch.Generator(device=dev).manual_seed(12)
    lab = torch.randint(0, FLCE_V, (FLCE_N,), generator=g, device=dev)
    lab[torch.rand(FLCE_N, generator=g, device=dev) < 0.1] = -100
    one = torch.ones((), device=dev)
    state = {}

    def fwd():
        state["f"] = hip_ops.flce_fwd_grad(h, w, lab, token_chunk=token_chunk)

    def bwd():
        _, _, _, dh, dw = state["f"]
        hip_ops.flce_scale_grads(one, dh, dw)

    fwd()
    torch.cuda.synchronize()
    state.clear()
    torch.cuda.empty_cache()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    fwd()
    bwd()
    torch.cuda.synchronize()
    peak_extra = torch.cuda.max_memory_allocated() - base
    f = timer.time(fwd, reps)
    b = timer.time(bwd, reps)
    tot = f["ms"] + b["ms"]
    tf = FLCE_FLOP / (tot * 1e-3) / 1e12
    T = token_chunk or hip_ops.flce_token_chunk(FLCE_N, FLCE_V)
    ws = hip_ops._hip.query("ml_flce_fwd_grad_workspace_bytes", FLCE_N, FLCE_V, FLCE_H, T, 1)
    del h, w, lab, state
    torch.cuda.empty_cache()
    return {"fwd_ms": round(f["ms"], 3), "bwd_ms": round(b["ms"], 3), "TFLOP/s": round(tf, 1),
            "mfma_frac": round(tf / MFMA_PEAK_TFLOPS, 4), "flop": FLCE_FLOP, "token_chunk": T,
            "peak_extra_bytes": int(peak_extra), "workspace_bytes": int(ws),
            "grad_output_bytes": (FLCE_N + FLCE_V) * FLCE_H * 2,
            "full_logits_bf16_bytes": FLCE_N * FLCE_V * 2,
            "peak_extra_over_full_logits": round(peak_extra / (FLCE_N * FLCE_V * 2), 4),
            "workspace_over_full_logits": round(ws / (FLCE_N * FLCE_V * 2), 4),
            "reference_model_peak_extra_bytes": flce_reference_peak_bytes(FLCE_N, FLCE_V, FLCE_H,
                                                                          FLCE_CHUNK),
            "reps": reps, "timing": "median of reps (flush before each)"}


QKN_DIR_TABLE_BYTES = 2 * RB * RS * RD * 2                  # cos + sin [B, S, D] bf16
QKN_FWD_BYTES = 2 * RB * (RHQ + RHK) * RS * RD * 2 + QKN_DIR_TABLE_BYTES    # x in, y out
QKN_BWD_BYTES = 3 * RB * (RHQ + RHK) * RS * RD * 2 + QKN_DIR_TABLE_BYTES    # x, dy in; dx out


def bench_qk_norm_rope(dev, timer):
    """Qwen3 q_norm / k_norm fused with RoPE at the RoPE config: q [4, 16,
    2048, 128], k [4, 8, 2048, 128] bf16 as HF's transposed views of the
    projections, bf16 weights 1 + 0.1 N(0, 1), bf16 theta-1e6 tables [4,
    2048, 128] broadcast over heads; backward with the weight gradients."""
    import torch

    from metal_liger_amd import hip_ops
    q = gpu_randn((RB, RS, RHQ, RD), 60, dev).transpose(1, 2)
    k = gpu_randn((RB, RS, RHK, RD), 61, dev).transpose(1, 2)
    wq = 1.0 + 0.1 * gpu_randn((RD,), 62, dev)
    wk = 1.0 + 0.1 * gpu_randn((RD,), 63, dev)
    inv = hip_ops.rope_inv_freq(RD, THETA, dev)
    ang = torch.arange(RS, device=dev, dtype=torch.float32).unsqueeze(-1) * inv
    emb = torch.cat((ang, ang), -1).unsqueeze(0).expand(RB, RS, RD)
    cos = emb.cos().to(torch.bfloat16).unsqueeze(1)
    sin = emb.sin().to(torch.bfloat16).unsqueeze(1)
    dq = gpu_randn((RB, RHQ, RS, RD), 64, dev)
    dk = gpu_randn((RB, RHK, RS, RD), 65, dev)
    f = timer.time(lambda: hip_ops.qk_norm_rope_fwd(q, k, wq, wk, cos, sin, 1e-6))
    b = timer.time(lambda: hip_ops.qk_norm_rope_bwd(q, k, wq, wk, cos, sin, 1e-6, dq, dk))
    C = rotating_copies(QKN_FWD_BYTES)
    cp = [(q.clone(memory_format=torch.preserve_format), k.clone(memory_format=torch.preserve_format),
           dq.clone(), dk.clone()) for _ in range(C)]
    rf = time_rotating([lambda t=t: hip_ops.qk_norm_rope_fwd(t[0], t[1], wq, wk, cos, sin, 1e-6)
                        for t in cp], timer.stream)
    rb = time_rotating([lambda t=t: hip_ops.qk_norm_rope_bwd(t[0], t[1], wq, wk, cos, sin, 1e-6,
                                                             t[2], t[3]) for t in cp], timer.stream)
    del cp
    return {"fwd": cold_line(f, QKN_FWD_BYTES, rot_ms=rf), "bwd": cold_line(b, QKN_BWD_BYTES, rot_ms=rb),
            "bwd_note": "includes the dw partial-row reduction launch"}


def bench_lora_bwd(dev, timer, reps=20):
    """Fused LoRA backward of a Qwen3-style 2B layer (QKV + MLP): X [8192, 2048],
    Wq [2048, 2048], Wk/Wv [1024, 2048], Wgate/Wup [6144, 2048], Wdown
    [2048, 6144] ~N(0, 0.02), rank 16, alpha 32, A ~N(0, 1/16), B ~N(0, 0.02);
    forward intermediates made by the library's forward ops beforehand."""
    from metal_liger_amd import hip_ops
    N, H, KV, I, r = LORA_N, LORA_H, LORA_KV, LORA_I, LORA_R
    s = 2.0
    x = gpu_randn((N, H), 20, dev)
    outs = (H, KV, KV)
    Wqkv = [gpu_randn((o, H), 21 + i, dev, 0.02) for i, o in enumerate(outs)]
    a_qkv = gpu_randn((3 * r, H), 24, dev, 0.25)
    Bqkv = [gpu_randn((o, r), 25 + i, dev, 0.02) for i, o in enumerate(outs)]
    dqkv = [gpu_randn((N, o), 28 + i, dev) for i, o in enumerate(outs)]
    xa = hip_ops.lora_xa(x, a_qkv)
    WG, WU = gpu_randn((I, H), 31, dev, 0.02), gpu_randn((I, H), 32, dev, 0.02)
    WD = gpu_randn((H, I), 33, dev, 0.02)
    a_gu = gpu_randn((2 * r, H), 34, dev, 0.25)
    a_d = gpu_randn((r, I), 35, dev, 0.25)
    BG, BU = gpu_randn((I, r), 36, dev, 0.02), gpu_randn((I, r), 37, dev, 0.02)
    BD = gpu_randn((H, r), 38, dev, 0.02)
    dy = gpu_randn((N, H), 39, dev)
    xa_gu = hip_ops.lora_xa(x, a_gu)
    gate = hip_ops.lora_linear_out(x, WG, xa_gu[:, :r], BG * s)
    up = hip_ops.lora_linear_out(x, WU, xa_gu[:, r:], BU * s)
    hmid = hip_ops.swiglu_fwd(gate, up)
    ha_d = hip_ops.lora_xa(hmid, a_d)

    def qkv():
        hip_ops.lora_qkv_bwd(x, dqkv, Wqkv, a_qkv, Bqkv, [s, s, s], xa, r)

    def mlp():  # h recomputed from gate and up, as the autograd path calls it
        hip_ops.lora_mlp_bwd(x, gate, up, None, dy, WG, WU, WD, a_gu, a_d, BG, BU, BD,
                             [s, s, s], xa_gu, ha_d, r)

    q = timer.time(qkv, reps)
    m = timer.time(mlp, reps)
    tot = q["ms"] + m["ms"]
    tf = LORA_BWD_FLOP / (tot * 1e-3) / 1e12
    return {"qkv_ms": round(q["ms"], 3), "mlp_ms": round(m["ms"], 3), "TFLOP/s": round(tf, 1),
            "mfma_frac": round(tf / MFMA_PEAK_TFLOPS, 4), "flop": LORA_BWD_FLOP,
            "tokens_per_s": round(N / (tot * 1e-3), 1), "reps": reps,
            "timing": "median of reps (flush before each)"}


def build_train_model(dev, layers=None, efficient_attention=True):
    """The 4-layer Qwen3-style LoRA train-step model (tests/qwen_tiny.py,
    build_train_config: hidden 2048, 16 q / 8 kv heads, head_dim 128, MLP
    6144, vocab 151936, tied embeddings, rank-16 LoRA on q, k, v, o, gate,
    up, down, bf16) with every fused op patched in and, with
    efficient_attention, its grouped-query attention on SDPA's
    memory-efficient kernel (otherwise transformers' own SDPA call); only the
    adapters train."""
    from metal_liger_amd import apply_metal_liger_to_qwen3vl
    from tests import qwen_tiny
    model = qwen_tiny.build_train_config(dev, layers or qwen_tiny.TRAIN_LAYERS)
    model = apply_metal_liger_to_qwen3vl(model, fuse_qk_norm_rope=True, fuse_lm_loss=True,
                                         fuse_residual_norm=True,
                                         efficient_attention=efficient_attention)
    qwen_tiny.freeze_all_but_lora(model)
    return model


def bench_train_step(dev, steps=5, warmup=2, efficient_attention=True):
    """4-layer Qwen3-style LoRA train step: token ids [4, 2048] uniform in
    [0, 151936), forward through the patched decoder (fused RMSNorm, SwiGLU,
    LoRA QKV / MLP / o_proj, q/k norm + RoPE from the rotary module's tables,
    the post-attention residual add fused into its norm),
    next-token loss from model(input_ids, labels=input_ids) by the chunked
    fused linear cross-entropy (transformers' label shift: the last position
    of each sequence ignored; no logits formed), backward, AdamW on the
    adapters.
    Attention is torch's scaled_dot_product_attention: with
    efficient_attention over key / value heads repeated to the 16 query
    heads, on its memory-efficient kernel; without it, transformers' own GQA
    call (enable_gqa, the flash kernel). Either way an unavailable kernel
    raises instead of falling back to the batched-matmul path. tokens/s =
    8192 / step time."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from tests import qwen_tiny
    model = build_train_model(dev, efficient_attention=efficient_attention)
    model.train()
    params = [p for p in model.parameters() if p.requires_grad]
    opt = torch.optim.AdamW(params, lr=1e-4, foreach=True)
    ids = qwen_tiny.train_ids(dev)

    def step():
        opt.zero_grad(set_to_none=True)
        # use_cache=False: a training forward keeps no KV cache (with the
        # config's default the model would copy every layer's keys and values
        # into one, 2 x 33.5 MB per layer per step, for nothing)
        out = model(input_ids=ids, labels=ids, use_cache=False)
        if out.logits is not None:
            raise RuntimeError("train step: the fused loss hook did not run")
        loss = out.loss
        loss.backward()
        opt.step()
        return loss

    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        for _ in range(warmup):
            loss = step()
        torch.cuda.synchronize()
        first = loss.item()
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = step()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
    last = loss.item()
    del model, opt, params
    torch.cuda.empty_cache()
    if not (math.isfinite(first) and math.isfinite(last)):
        raise RuntimeError(f"train step: non-finite loss {first} -> {last}")
    n_tok = qwen_tiny.TRAIN_B * qwen_tiny.TRAIN_S
    return {"layers": qwen_tiny.TRAIN_LAYERS, "tokens": n_tok, "ms_per_step": round(dt * 1e3, 2),
            "tokens_per_s": round(n_tok / dt, 1), "loss_first": round(first, 4),
            "loss_last": round(last, 4), "steps": steps, "warmup": warmup,
            "includes": "fwd + FLCE loss (model(input_ids, labels=input_ids, use_cache=False)) + bwd + AdamW on LoRA params",
            "attention": ("torch SDPA, memory-efficient kernel, key/value heads repeated "
                          "(efficient_attention=True)" if efficient_attention else
                          "transformers' SDPA call with enable_gqa (flash kernel; "
                          "efficient_attention=False)")}


def pmc_probe(dev):
    """Launch sequence for rocprofv3 --pmc traffic counting: 3 copies of a
    1 GiB buffer (the calibration: a plain copy reads and writes exactly
    1 GiB each), then 5 launches each of the SwiGLU backward and forward on
    gate, up, dy [8192, 6144] bf16, RoPE (positions, in-kernel cos/sin) on
    q [4, 16, 2048, 128], k [4, 8, 2048, 128] bf16, RMSNorm forward and
    backward on x [8192, 2048] fp32, and the fused q/k norm + RoPE forward
    and backward (with weight gradients) on the same q, k as HF's transposed
    views with bf16 tables [4, 2048, 128], and the residual add + RMSNorm
    forward and backward on bf16 [8192, 2048]."""
    import torch

    from metal_liger_amd import hip_ops
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    gate = gpu_randn((N_TOK, INTER), 0, dev)
    up = gpu_randn((N_TOK, INTER), 1, dev)
    dy = gpu_randn((N_TOK, INTER), 2, dev)
    q = gpu_randn((RB, RHQ, RS, RD), 3, dev)
    k = gpu_randn((RB, RHK, RS, RD), 4, dev)
    pos = torch.arange(RS, device=dev)
    inv = hip_ops.rope_inv_freq(RD, THETA, dev)
    x = gpu_randn((RMS_N, RMS_H), 40, dev, dtype=torch.float32)
    w = 1.0 + 0.1 * gpu_randn((RMS_H,), 41, dev, dtype=torch.float32)
    gx = gpu_randn((RMS_N, RMS_H), 42, dev, dtype=torch.float32)
    _, rrms = hip_ops.rms_norm_fwd(x, w, 1e-6)
    hq = gpu_randn((RB, RS, RHQ, RD), 60, dev).transpose(1, 2)
    hk = gpu_randn((RB, RS, RHK, RD), 61, dev).transpose(1, 2)
    nwq = 1.0 + 0.1 * gpu_randn((RD,), 62, dev)
    nwk = 1.0 + 0.1 * gpu_randn((RD,), 63, dev)
    cos = gpu_randn((RB, 1, RS, RD), 64, dev)
    sin = gpu_randn((RB, 1, RS, RD), 65, dev)
    ax = gpu_randn((ADD_N, ADD_H), 45, dev)
    ares = gpu_randn((ADD_N, ADD_H), 46, dev)
    aw = 1.0 + 0.1 * gpu_randn((ADD_H,), 47, dev)
    ady = gpu_randn((ADD_N, ADD_H), 48, dev)
    ads = gpu_randn((ADD_N, ADD_H), 49, dev)
    _, atot, arr = hip_ops.rms_norm_add_fwd(ax, ares, aw, 1e-6)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    for fn in (lambda: hip_ops.swiglu_bwd(gate, up, dy),
               lambda: hip_ops.swiglu_fwd(gate, up),
               lambda: hip_ops.rope_pos(q, k, pos, inv, 1.0),
               lambda: hip_ops.rms_norm_fwd(x, w, 1e-6),
               lambda: hip_ops.rms_norm_bwd(x, w, gx, rrms, 1e-6),
               lambda: hip_ops.qk_norm_rope_fwd(hq, hk, nwq, nwk, cos, sin, 1e-6),
               lambda: hip_ops.qk_norm_rope_bwd(hq, hk, nwq, nwk, cos, sin, 1e-6, q, k),
               lambda: hip_ops.rms_norm_add_fwd(ax, ares, aw, 1e-6),
               lambda: hip_ops.rms_norm_bwd(atot, aw, ady, arr, 1e-6, dsum=ads)):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
    print("pmc probe: 3 x 1 GiB copy; 5 x each of swiglu_bwd, swiglu_fwd [8192, 6144] bf16, "
          "rope_pos q/k bf16, rms_norm fwd, bwd [8192, 2048] fp32, qk_norm_rope fwd, bwd bf16, "
          "rms_norm add fwd, bwd [8192, 2048] bf16", flush=True)


class _RunOnce:
    """Stands in for ColdTimer where only the launches matter (PMC probes)."""

    def time(self, fn, reps=1):
        fn()
        return {"ms": 1.0, "p10_ms": 1.0, "p90_ms": 1.0, "reps": 1}


def pmc_mfma_probe(dev):
    """Launch sequence for rocprofv3 --pmc matrix-core counting: one warm-up
    and one measured call each of the one-pass FLCE forward (loss, dH, dW;
    hidden [8192, 2048], lm_head [151936, 2048]) and of the LoRA QKV and MLP
    backward of the Qwen3-style 2B layer."""
    import torch

    from metal_liger_amd import hip_ops
    h = gpu_randn((FLCE_N, FLCE_H), 10, dev)
    w = gpu_randn((FLCE_V, FLCE_H), 11, dev, 0.02)
    g = torch.Generator(device=dev).manual_seed(12)
    lab = torch.randint(0, FLCE_V, (FLCE_N,), generator=g, device=dev)
    for _ in range(2):
        out = hip_ops.flce_fwd_grad(h, w, lab)
    torch.cuda.synchronize()
    del out, h, w, lab
    torch.cuda.empty_cache()
    bench_lora_bwd(dev, _RunOnce(), 1)
    torch.cuda.synchronize()
    print("pmc mfma probe: 2 x flce_fwd_grad, 2 x (lora qkv bwd + mlp bwd)", flush=True)


def load_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed
    rocprofv3 PMC summary (FETCH_SIZE / WRITE_SIZE scaled by the copy-kernel
    calibration); None when not measured."""
    path = os.path.join(ROOT, "profiles", "traffic_swiglu_bwd.json")
    try:
        with open(path) as f:
            d = json.load(f)
        return int(d["hbm_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def host_cpu():
    """os.cpu_count(), torch's thread count and the CPU model of this host."""
    import torch
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
            "model": model}


def _time_cpu(fn, warmup, reps):
    import statistics
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline(seconds: float):
    """Oracle (reference torch ops restated, CPU) on the headline step at its
    full shape: SwiGLU fwd + bwd on [8192, 6144] and RoPE fwd + bwd on q
    [4,16,2048,128], k [4,8,2048,128] (tables built as the HF rotary module
    does, cast to bf16 as HF does), repeated for about `seconds`."""
    import torch

    from oracle import reference_ops as ref

    n = N_TOK
    g = seeded((n, INTER), 0, torch.bfloat16)
    u = seeded((n, INTER), 1, torch.bfloat16)
    dy = seeded((n, INTER), 2, torch.bfloat16)
    q = seeded((RB, RHQ, RS, RD), 3, torch.bfloat16)
    k = seeded((RB, RHK, RS, RD), 4, torch.bfloat16)
    gq = seeded((RB, RHQ, RS, RD), 5, torch.bfloat16)
    gk = seeded((RB, RHK, RS, RD), 6, torch.bfloat16)
    pos = torch.arange(RS)
    sample_bytes = 8 * n * INTER * 2 + 2 * 2 * RB * (RHQ + RHK) * RS * RD * 2
    assert sample_bytes == STEP_BYTES

    def once():
        out, sig = ref.swiglu_forward(g, u)
        ref.swiglu_backward(g, u, sig, dy)
        cos, sin = ref.rope_tables(pos, RD, THETA)
        cos, sin = cos.to(torch.bfloat16), sin.to(torch.bfloat16)
        ref.rope_forward(q, cos, sin)
        ref.rope_forward(k, cos, sin)
        ref.rope_backward(gq, cos, sin, torch.bfloat16)
        ref.rope_backward(gk, cos, sin, torch.bfloat16)

    once()  # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        once()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per = el / reps
    return {
        "value": round(sample_bytes / per / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"full shape: oracle torch-CPU SwiGLU fwd+bwd on [{n}, {INTER}] bf16 + RoPE "
                   f"fwd+bwd on q [{RB},{RHQ},{RS},{RD}], k [{RB},{RHK},{RS},{RD}] bf16 (tables "
                   f"built per call), {reps} reps in {el:.1f} s, {sample_bytes} algorithmic bytes "
                   "per rep"),
        "host": host_cpu(),
    }


def cpu_baselines(full: bool):
    """The oracle (the reference's torch ops restated, run on this host's CPU
    with all of torch's threads) on every config. full=False: bounded
    samples (RMSNorm at full size; SwiGLU and RoPE on a quarter, LoRA on an
    eighth, FLCE on a sixteenth of the tokens; the train step at batch 1 x
    256), 1 warm-up + 3 reps (FLCE: 1 rep; train step: 1 warm-up + 1 rep),
    ~15 s on an 8-core host; full=True: every config at its full shape, 1
    warm-up + 3 reps for RMSNorm, SwiGLU, RoPE and LoRA, 1 rep for FLCE and
    the train step. Each value is in the unit of the GPU line it stands
    beside; the sample is named."""
    import torch

    from oracle import reference_ops as ref
    torch.manual_seed(0)
    out = {"host": host_cpu(), "full_shapes": full}
    bf = torch.bfloat16

    # RMSNorm fp32 [8192, 2048] fwd + bwd
    x = seeded((RMS_N, RMS_H), 40, torch.float32)
    w = 1.0 + 0.1 * seeded((RMS_H,), 41, torch.float32)
    gy = seeded((RMS_N, RMS_H), 42, torch.float32)

    def rms():
        y, r = ref.rms_norm_forward(x, w, 1e-6)
        ref.rms_norm_backward(x, w, r, gy)
    t = _time_cpu(rms, 1, 3)
    out["rmsnorm_fp32"] = {"GB/s": round((RMS_FWD_BYTES + RMS_BWD_BYTES) / t / 1e9, 2),
                           "sample": f"x [{RMS_N}, {RMS_H}] fp32 fwd+bwd", "s_per_rep": round(t, 3)}

    # SwiGLU bf16 [n, 6144] fwd + bwd
    n = N_TOK if full else N_TOK // 4
    g = seeded((n, INTER), 0, bf)
    u = seeded((n, INTER), 1, bf)
    dyy = seeded((n, INTER), 2, bf)

    def swg():
        o, sig = ref.swiglu_forward(g, u)
        ref.swiglu_backward(g, u, sig, dyy)
    t = _time_cpu(swg, 1, 3)
    out["swiglu_bf16"] = {"GB/s": round(8 * n * INTER * 2 / t / 1e9, 2),
                          "sample": f"gate/up [{n}, {INTER}] bf16 fwd+bwd", "s_per_rep": round(t, 3)}
    del g, u, dyy

    # RoPE bf16 fwd + bwd, tables built per call
    b = RB if full else 1
    q = seeded((b, RHQ, RS, RD), 3, bf)
    k = seeded((b, RHK, RS, RD), 4, bf)
    pos = torch.arange(RS)

    def rope():
        cos, sin = ref.rope_tables(pos, RD, THETA)
        cos, sin = cos.to(bf), sin.to(bf)
        ref.rope_forward(q, cos, sin), ref.rope_forward(k, cos, sin)
        ref.rope_backward(q, cos, sin, bf), ref.rope_backward(k, cos, sin, bf)
    t = _time_cpu(rope, 1, 3)
    out["rope_bf16"] = {"GB/s": round(2 * 2 * b * (RHQ + RHK) * RS * RD * 2 / t / 1e9, 2),
                        "sample": f"q [{b},{RHQ},{RS},{RD}], k [{b},{RHK},{RS},{RD}] bf16 fwd+bwd",
                        "s_per_rep": round(t, 3)}
    del q, k

    # LoRA backward of the Qwen3-style layer (QKV + MLP), rank 16
    nl = LORA_N if full else LORA_N // 8
    H, KV, I, r = LORA_H, LORA_KV, LORA_I, LORA_R
    X = seeded((nl, H), 20, bf)
    qkv = [(seeded((o, H), 21 + i, bf) * 0.02, seeded((r, H), 24 + i, bf) * 0.25,
            seeded((o, r), 27 + i, bf) * 0.02, 2.0) for i, o in enumerate((H, KV, KV))]
    dqkv = [seeded((nl, o), 30 + i, bf) for i, o in enumerate((H, KV, KV))]
    mlp = [(seeded((I, H), 33, bf) * 0.02, seeded((r, H), 34, bf) * 0.25, seeded((I, r), 35, bf) * 0.02, 2.0),
           (seeded((I, H), 36, bf) * 0.02, seeded((r, H), 37, bf) * 0.25, seeded((I, r), 38, bf) * 0.02, 2.0),
           (seeded((H, I), 39, bf) * 0.02, seeded((r, I), 40, bf) * 0.25, seeded((H, r), 41, bf) * 0.02, 2.0)]
    fq = [t_ for p in qkv for t_ in p]
    fm = [t_ for p in mlp for t_ in p]
    dY = seeded((nl, H), 42, bf)
    _, gate, up, hmid = ref.lora_mlp_forward(X, *fm)

    def lora():
        ref.lora_qkv_backward(X, *dqkv, *fq)
        ref.lora_mlp_backward(X, gate, up, hmid, dY, *fm)
    t = _time_cpu(lora, 1, 3)
    lf = LORA_BWD_FLOP * nl / LORA_N
    out["lora_bwd_layer"] = {"TFLOP/s": round(lf / t / 1e12, 3), "tokens_per_s": round(nl / t, 1),
                             "sample": f"X [{nl}, {H}] (QKV + MLP backward, rank {r}) bf16",
                             "s_per_rep": round(t, 3)}
    del X, qkv, mlp, gate, up, hmid, dqkv, dY

    # FLCE fwd + bwd over the full vocabulary (chunk 8192), fp32 inside
    nf = FLCE_N if full else FLCE_N // 16
    hf = seeded((nf, FLCE_H), 10, bf)
    wf = seeded((FLCE_V, FLCE_H), 11, bf) * 0.02
    gl = torch.Generator().manual_seed(12)
    lab = torch.randint(0, FLCE_V, (nf,), generator=gl)
    lab[torch.rand(nf, generator=gl) < 0.1] = -100

    def flce():
        loss, lse, mask = ref.flce_forward(hf, wf, lab, None, -100, FLCE_CHUNK)
        ref.flce_backward(hf, wf, lab, lse, mask, torch.tensor(1.0), None, FLCE_CHUNK)
    t = _time_cpu(flce, 0, 1)
    ff = 3 * 2 * nf * FLCE_V * FLCE_H
    out["flce_fwd_bwd"] = {"TFLOP/s": round(ff / t / 1e12, 3),
                           "sample": f"hidden [{nf}, {FLCE_H}], lm_head [{FLCE_V}, {FLCE_H}] bf16",
                           "s_per_rep": round(t, 3)}
    del hf, wf

    # 4-layer Qwen3-style LoRA train step (unpatched HF model: the same math
    # as the reference's patched model, whose fused ops are torch on the CPU)
    from tests import qwen_tiny
    bs, sl = (qwen_tiny.TRAIN_B, qwen_tiny.TRAIN_S) if full else (1, 256)
    model = qwen_tiny.build_train_config(torch.device("cpu"), attn="sdpa")
    model.train()
    params = [p for p in model.parameters() if p.requires_grad]
    opt = torch.optim.AdamW(params, lr=1e-4)
    ids = torch.randint(0, qwen_tiny.TRAIN_V, (bs, sl), generator=torch.Generator().manual_seed(0))

    def step():
        opt.zero_grad(set_to_none=True)
        model(input_ids=ids, labels=ids).loss.backward()
        opt.step()
    t = _time_cpu(step, 0 if full else 1, 1)
    out["train_step_4layer"] = {"tokens_per_s": round(bs * sl / t, 1),
                                "sample": f"batch {bs} x seq {sl}, bf16, fwd + loss + bwd + AdamW",
                                "s_per_rep": round(t, 3)}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-full", action="store_true",
                    help="only the CPU baselines of every config at full shape (one JSON line)")
    ap.add_argument("--cpu-samples", action="store_true",
                    help="CPU baselines of the configs on bounded samples of their shapes "
                         "instead of the full shapes (the default; ~30 s of host time)")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="only the launch sequence used for rocprofv3 --pmc traffic counting")
    ap.add_argument("--pmc-mfma-probe", action="store_true",
                    help="only the FLCE / LoRA-backward launches used for rocprofv3 --pmc "
                         "matrix-core counting")
    ap.add_argument("--no-mfma-ops", action="store_true",
                    help="skip the FLCE / LoRA-backward lines of the breakdown")
    ap.add_argument("--no-train-step", action="store_true",
                    help="skip the 4-layer Qwen3 LoRA train-step line")
    ap.add_argument("--train-step-only", action="store_true",
                    help="only the 4-layer Qwen3 LoRA train step (one JSON line)")
    args = ap.parse_args()
    if args.cpu_full:
        print(json.dumps({"cpu_baselines": cpu_baselines(full=True)}), flush=True)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: metal_liger_amd has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch

    from metal_liger_amd import hip_ops

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.pmc_probe:
        pmc_probe(dev)
        return
    if args.pmc_mfma_probe:
        pmc_mfma_probe(dev)
        return
    if args.train_step_only:
        print(json.dumps({"train_step_4layer": bench_train_step(dev)}), flush=True)
        return
    bf = torch.bfloat16
    gate = seeded((N_TOK, INTER), 0, bf).to(dev)
    up = seeded((N_TOK, INTER), 1, bf).to(dev)
    dy = seeded((N_TOK, INTER), 2, bf).to(dev)
    q = seeded((RB, RHQ, RS, RD), 3, bf).to(dev)
    k = seeded((RB, RHK, RS, RD), 4, bf).to(dev)
    gq = seeded((RB, RHQ, RS, RD), 5, bf).to(dev)
    gk = seeded((RB, RHK, RS, RD), 6, bf).to(dev)
    pos = torch.arange(RS, device=dev)
    inv = hip_ops.rope_inv_freq(RD, THETA, dev)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)
    ops = {
        "swiglu_fwd": lambda: hip_ops.swiglu_fwd(gate, up),
        "swiglu_bwd": lambda: hip_ops.swiglu_bwd(gate, up, dy),
        "rope_fwd": lambda: hip_ops.rope_pos(q, k, pos, inv, 1.0),
        "rope_bwd": lambda: hip_ops.rope_pos(gq, gk, pos, inv, -1.0),
    }
    # Consecutive steps alternate between two copies of every input (1 GB
    # of operands each): a step never re-reads what the previous step left
    # in the 256 MB MALL, so every step streams its bytes from HBM.
    step_inputs = [(gate, up, dy, q, k, gq, gk),
                   tuple(t.clone() for t in (gate, up, dy, q, k, gq, gk))]

    def step(i):
        g_, u_, d_, q_, k_, gq_, gk_ = step_inputs[i % len(step_inputs)]
        hip_ops.swiglu_fwd(g_, u_)
        hip_ops.swiglu_bwd(g_, u_, d_)
        hip_ops.rope_pos(q_, k_, pos, inv, 1.0)
        hip_ops.rope_pos(gq_, gk_, pos, inv, -1.0)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # Timed region: exactly K steps, no per-kernel events (each event record
    # inserts ~4.6 us of idle time between kernels on this GPU).
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(args.steps):
        step(args.warmup + i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms_step = e0.elapsed_time(e1) / args.steps

    # Per-kernel launch duration, cold (ColdTimer: MALL / L2 flushed before
    # each of 25 reps, median), and warm (20 back-to-back launches).
    timer = ColdTimer(dev, stream)
    per_op, warm, rot = {}, {}, {}
    C = rotating_copies(ROPE_DIR_BYTES)
    rot_in = [(gate.clone(), up.clone(), dy.clone(), q.clone(), k.clone()) for _ in range(C)]
    rot_ops = {
        "swiglu_fwd": lambda t: hip_ops.swiglu_fwd(t[0], t[1]),
        "swiglu_bwd": lambda t: hip_ops.swiglu_bwd(t[0], t[1], t[2]),
        "rope_fwd": lambda t: hip_ops.rope_pos(t[3], t[4], pos, inv, 1.0),
        "rope_bwd": lambda t: hip_ops.rope_pos(t[3], t[4], pos, inv, -1.0),
    }
    for name, fn in ops.items():
        per_op[name] = timer.time(fn)
        warm[name] = time_launches(fn, stream, 20)
        rot[name] = time_rotating([lambda t=t, f=rot_ops[name]: f(t) for t in rot_in], stream)
    del rot_in, step_inputs

    ms_step = wall * 1e3 / args.steps
    value = STEP_BYTES / (wall / args.steps) / 1e9
    op_bytes = {"swiglu_fwd": SWIGLU_FWD_BYTES, "swiglu_bwd": SWIGLU_BWD_BYTES,
                "rope_fwd": ROPE_DIR_BYTES, "rope_bwd": ROPE_DIR_BYTES}
    breakdown = {n: dict(cold_line(per_op[n], op_bytes[n], rot_ms=rot[n]),
                         warm_us=round(warm[n] * 1e3, 2)) for n in per_op}
    breakdown["timing"] = TIMING_NOTE + ("; warm_us: mean of 20 back-to-back eager launches of "
                                         "the same inputs")
    breakdown["gpu_ms_per_step"] = round(gpu_ms_step, 4)
    breakdown["rmsnorm_fp32"] = bench_rmsnorm(dev, timer)
    breakdown["qk_norm_rope_bf16"] = bench_qk_norm_rope(dev, timer)
    breakdown["add_rmsnorm_bf16"] = bench_add_rmsnorm(dev, timer)
    if not args.no_mfma_ops:
        breakdown["flce_fwd_bwd"] = bench_flce(dev, timer)
        breakdown["lora_bwd_layer"] = bench_lora_bwd(dev, timer)
    if not args.no_train_step:
        breakdown["train_step_4layer"] = bench_train_step(dev)
        # the same step with transformers' own attention call: what the fused
        # ops alone give, without the opt-in attention routing
        breakdown["train_step_4layer_hf_attention"] = bench_train_step(dev,
                                                                       efficient_attention=False)
    breakdown["hbm_copy_ceiling"] = copy_ceiling(dev, stream)
    dom_ms = rot["swiglu_bwd"]
    achieved = SWIGLU_BWD_BYTES / (dom_ms * 1e-3) / 1e9
    roofline = {
        "kernel": "swiglu_bwd_vec<bf16> (ml_swiglu_bwd)",
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": load_traffic(),
        "algorithmic_bytes_per_launch": SWIGLU_BWD_BYTES,
        "launch_us": round(dom_ms * 1e3, 2),
        "flushed_launch_us": round(per_op["swiglu_bwd"]["ms"] * 1e3, 2),
        "timing": ("back-to-back launches over 2 copies of gate/up/dy (1 GB, beyond the MALL), "
                   "replayed from a captured graph; flushed_launch_us: median of 25 launches each "
                   "after a 512 MB write + 512 MB read flush, dispatch gap included"),
    }
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": ("SwiGLU + RoPE fwd+bwd bf16: gate/up [8192, 6144]; RoPE q [4,16,2048,128], "
                         "k [4,8,2048,128], positions 0..2047, theta 1e6, cos/sin in-kernel"),
            "bytes_per_step": STEP_BYTES,
            "hbm_frac": round(value / HBM_PEAK_GBS, 4),
            "inputs": "two copies of every input, alternating per step (each step reads HBM, not the MALL)",
        },
        "roofline": roofline,
        "breakdown": breakdown,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        line["cpu_baselines"] = cpu_baselines(full=not args.cpu_samples)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

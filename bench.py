"""Throughput of the fused-op hot path on one MI355X.

Workload (one step): SwiGLU forward + backward on gate, up [8192, 6144] bf16
and RoPE forward + backward on q [4, 16, 2048, 128], k [4, 8, 2048, 128]
bf16 with positions 0..2047, theta 1e6, cos/sin computed in-kernel. Inputs
~N(0, 1) drawn on the CPU from seeded generators, resident in HBM before the
timed region.

value = algorithmic bytes per step / time per step, where algorithmic bytes
count each input read once and each output written once:
  SwiGLU fwd 3*N*I*2 + bwd 5*N*I*2 = 805,306,368 B
  RoPE   fwd (read + write q, k) + bwd (same) = 201,326,592 B
roofline: the dominant kernel (SwiGLU backward, 503,316,480 B per launch),
its average launch duration from HIP events on its stream around 20
back-to-back launches, against 8 TB/s.
cpu_baseline: the oracle (a CPU restatement of the reference's torch ops)
on a bounded sample of the same workload, on the host's cores.
breakdown: each op's average launch time; plus, outside the step, chunked
FLCE fwd+bwd (hidden [8192, 2048], lm_head [151936, 2048], chunk 8192:
15.29 TFLOP) and the fused LoRA backward of a Qwen3-style 2B layer (QKV +
MLP, rank 16: 774.2 GFLOP), as TFLOP/s against the 2.5 PFLOP/s bf16 peak;
and the 4-layer Qwen3-style LoRA train step (batch 4 x 2048 tokens, every
fused op patched in, FLCE loss, AdamW on the adapters) in tokens/s.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--no-mfma-ops] [--no-train-step]
       [--train-step-only] [--pmc-probe] [--pmc-mfma-probe]
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
    the stream the kernels are launched on)."""
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


def time_graph(fn, stream, reps):
    """Average milliseconds per call of fn replayed from one captured HIP
    graph of `reps` calls: the launches' own GPU time, without the host-side
    argument marshalling of each call. Falls back to time_launches (and says
    so) when the capture fails."""
    import torch
    try:
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            fn()
        stream.wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                fn()
        g.replay()
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        g.replay()
        b.record(stream)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / reps
        del g
        return ms, "graph replay"
    except RuntimeError:
        return time_launches(fn, stream, reps), "eager launches (graph capture failed)"


RMS_N, RMS_H = 8192, 2048
RMS_FWD_BYTES = 2 * RMS_N * RMS_H * 4 + RMS_H * 4 + RMS_N * 4          # x, w in; y, rrms out
RMS_BWD_BYTES = 3 * RMS_N * RMS_H * 4 + 2 * RMS_H * 4 + RMS_N * 4      # x, dy, w, rrms in; dx, dw out


def bench_rmsnorm(dev, stream, reps):
    """RMSNorm fwd and bwd, fp32 x [8192, 2048], weight 1 + 0.1 N(0, 1),
    eps 1e-6 (rrms saved by the forward, as the autograd Function does)."""
    import torch

    from metal_liger_amd import hip_ops
    x = gpu_randn((RMS_N, RMS_H), 40, dev, dtype=torch.float32)
    w = (1.0 + 0.1 * gpu_randn((RMS_H,), 41, dev, dtype=torch.float32))
    dy = gpu_randn((RMS_N, RMS_H), 42, dev, dtype=torch.float32)
    _, rrms = hip_ops.rms_norm_fwd(x, w, 1e-6)
    f_ms = time_launches(lambda: hip_ops.rms_norm_fwd(x, w, 1e-6), stream, reps)
    b_ms = time_launches(lambda: hip_ops.rms_norm_bwd(x, w, dy, rrms, 1e-6), stream, reps)
    return {"fwd_us": round(f_ms * 1e3, 2), "fwd_GB/s": round(RMS_FWD_BYTES / (f_ms * 1e-3) / 1e9, 1),
            "bwd_us": round(b_ms * 1e3, 2), "bwd_GB/s": round(RMS_BWD_BYTES / (b_ms * 1e-3) / 1e9, 1)}


ADD_N, ADD_H = 8192, 2048
ADD_FWD_BYTES = 4 * ADD_N * ADD_H * 2 + ADD_H * 2 + ADD_N * 4      # x, res, w in; sum, y, rrms out
ADD_BWD_BYTES = 4 * ADD_N * ADD_H * 2 + 2 * ADD_H * 2 + ADD_N * 4  # sum, dy, dsum, w, rrms in; dx, dw out


def bench_add_rmsnorm(dev, stream, reps):
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
    f_ms, how = time_graph(lambda: hip_ops.rms_norm_add_fwd(x, res, w, 1e-6), stream, reps)
    b_ms, _ = time_graph(lambda: hip_ops.rms_norm_bwd(total, w, dy, rrms, 1e-6, dsum=ds), stream, reps)
    uf_ms, _ = time_graph(lambda: hip_ops.rms_norm_fwd(x + res, w, 1e-6), stream, reps)
    ub_ms, _ = time_graph(lambda: hip_ops.rms_norm_bwd(total, w, dy, rrms, 1e-6)[0] + ds, stream, reps)
    return {"fwd_us": round(f_ms * 1e3, 2), "fwd_GB/s": round(ADD_FWD_BYTES / (f_ms * 1e-3) / 1e9, 1),
            "bwd_us": round(b_ms * 1e3, 2), "bwd_GB/s": round(ADD_BWD_BYTES / (b_ms * 1e-3) / 1e9, 1),
            "unfused_fwd_us": round(uf_ms * 1e3, 2), "unfused_bwd_us": round(ub_ms * 1e3, 2),
            "timing": how}


def bench_flce(dev, stream, reps, token_chunk=None):
    """Fused linear cross-entropy fwd + bwd as the autograd Function runs it:
    hidden [8192, 2048], lm_head [151936, 2048] ~N(0, 0.02), no bias, 10% of
    labels ignored; the forward forms loss, dH and dW in one pass (logits
    computed once), the backward applies grad_output. 15.29 TFLOP of
    necessary GEMM work (logits, dH, dW) per fwd+bwd."""
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

    f_ms = time_launches(fwd, stream, reps)
    b_ms = time_launches(bwd, stream, reps)
    tot = f_ms + b_ms
    tf = FLCE_FLOP / (tot * 1e-3) / 1e12
    T = token_chunk or hip_ops.flce_token_chunk(FLCE_N, FLCE_V)
    del h, w, lab, state
    torch.cuda.empty_cache()
    return {"fwd_ms": round(f_ms, 3), "bwd_ms": round(b_ms, 3), "TFLOP/s": round(tf, 1),
            "mfma_frac": round(tf / MFMA_PEAK_TFLOPS, 4), "flop": FLCE_FLOP, "token_chunk": T}


QKN_DIR_TABLE_BYTES = 2 * RB * RS * RD * 2                  # cos + sin [B, S, D] bf16
QKN_FWD_BYTES = 2 * RB * (RHQ + RHK) * RS * RD * 2 + QKN_DIR_TABLE_BYTES    # x in, y out
QKN_BWD_BYTES = 3 * RB * (RHQ + RHK) * RS * RD * 2 + QKN_DIR_TABLE_BYTES    # x, dy in; dx out


def bench_qk_norm_rope(dev, stream, reps):
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
    f_ms, how = time_graph(lambda: hip_ops.qk_norm_rope_fwd(q, k, wq, wk, cos, sin, 1e-6), stream, reps)
    b_ms, _ = time_graph(lambda: hip_ops.qk_norm_rope_bwd(q, k, wq, wk, cos, sin, 1e-6, dq, dk),
                         stream, reps)
    return {"fwd_us": round(f_ms * 1e3, 2), "fwd_GB/s": round(QKN_FWD_BYTES / (f_ms * 1e-3) / 1e9, 1),
            "bwd_us": round(b_ms * 1e3, 2), "bwd_GB/s": round(QKN_BWD_BYTES / (b_ms * 1e-3) / 1e9, 1),
            "bwd_note": "includes the dw partial-row reduction launch", "timing": how}


def bench_lora_bwd(dev, stream, reps):
    """Fused LoRA backward of a Qwen3-style 2B layer (QKV + MLP): X [8192, 2048],
    Wq [2048, 2048], Wk/Wv [1024, 2048], Wgate/Wup [6144, 2048], Wdown
    [2048, 6144] ~N(0, 0.02), rank 16, alpha 32, A ~N(0, 1/16), B ~N(0, 0.02);
    forward intermediates made by the library's forward ops beforehand."""
    import torch

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

    def mlp():
        hip_ops.lora_mlp_bwd(x, gate, up, hmid, dy, WG, WU, WD, a_gu, a_d, BG, BU, BD,
                             [s, s, s], xa_gu, ha_d, r)

    q_ms = time_launches(qkv, stream, reps)
    m_ms = time_launches(mlp, stream, reps)
    tot = q_ms + m_ms
    tf = LORA_BWD_FLOP / (tot * 1e-3) / 1e12
    return {"qkv_ms": round(q_ms, 3), "mlp_ms": round(m_ms, 3), "TFLOP/s": round(tf, 1),
            "mfma_frac": round(tf / MFMA_PEAK_TFLOPS, 4), "flop": LORA_BWD_FLOP,
            "tokens_per_s": round(N / (tot * 1e-3), 1)}


def build_train_model(dev, layers=None):
    """The 4-layer Qwen3-style LoRA train-step model (tests/qwen_tiny.py,
    build_train_config: hidden 2048, 16 q / 8 kv heads, head_dim 128, MLP
    6144, vocab 151936, tied embeddings, rank-16 LoRA on q, k, v, o, gate,
    up, down, bf16) with every fused op patched in; only the adapters
    train."""
    from metal_liger_amd import apply_metal_liger_to_qwen3vl
    from tests import qwen_tiny
    model = qwen_tiny.build_train_config(dev, layers or qwen_tiny.TRAIN_LAYERS)
    model = apply_metal_liger_to_qwen3vl(model, fuse_qk_norm_rope=True, fuse_lm_loss=True,
                                         fuse_residual_norm=True)
    qwen_tiny.freeze_all_but_lora(model)
    return model


def bench_train_step(dev, steps=5, warmup=2):
    """4-layer Qwen3-style LoRA train step: token ids [4, 2048] uniform in
    [0, 151936), forward through the patched decoder (fused RMSNorm, SwiGLU,
    LoRA QKV / MLP / o_proj, q/k norm + RoPE from the rotary module's tables,
    the post-attention residual add fused into its norm),
    next-token loss from model(input_ids, labels=input_ids) by the chunked
    fused linear cross-entropy (transformers' label shift: the last position
    of each sequence ignored; no logits formed), backward, AdamW on the
    adapters.
    Attention is torch's scaled_dot_product_attention restricted to its
    flash / memory-efficient kernels (an unavailable kernel raises instead of
    falling back to the batched-matmul path). tokens/s = 8192 / step time."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from tests import qwen_tiny
    model = build_train_model(dev)
    model.train()
    params = [p for p in model.parameters() if p.requires_grad]
    opt = torch.optim.AdamW(params, lr=1e-4, foreach=True)
    ids = qwen_tiny.train_ids(dev)

    def step():
        opt.zero_grad(set_to_none=True)
        out = model(input_ids=ids, labels=ids)
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
    if not (math.isfinite(first) and math.isfinite(last)):
        raise RuntimeError(f"train step: non-finite loss {first} -> {last}")
    n_tok = qwen_tiny.TRAIN_B * qwen_tiny.TRAIN_S
    return {"layers": qwen_tiny.TRAIN_LAYERS, "tokens": n_tok, "ms_per_step": round(dt * 1e3, 2),
            "tokens_per_s": round(n_tok / dt, 1), "loss_first": round(first, 4),
            "loss_last": round(last, 4), "steps": steps, "warmup": warmup,
            "includes": "fwd + FLCE loss (model(input_ids, labels=input_ids)) + bwd + AdamW on LoRA params",
            "attention": "torch SDPA (flash / mem-efficient)"}


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
    stream = torch.cuda.current_stream(dev)
    bench_lora_bwd(dev, stream, 1)
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


def cpu_baseline(seconds: float):
    """Oracle (reference torch ops restated, CPU) on a bounded sample:
    SwiGLU on 1024 of the 8192 tokens, RoPE on batch 1 of 4 (tables built
    as the HF rotary module does, cast to bf16 as HF does)."""
    import torch

    from oracle import reference_ops as ref

    n = 1024
    g = seeded((n, INTER), 0, torch.bfloat16)
    u = seeded((n, INTER), 1, torch.bfloat16)
    dy = seeded((n, INTER), 2, torch.bfloat16)
    q = seeded((1, RHQ, RS, RD), 3, torch.bfloat16)
    k = seeded((1, RHK, RS, RD), 4, torch.bfloat16)
    gq = seeded((1, RHQ, RS, RD), 5, torch.bfloat16)
    gk = seeded((1, RHK, RS, RD), 6, torch.bfloat16)
    pos = torch.arange(RS)
    sample_bytes = 8 * n * INTER * 2 + 2 * 2 * (RHQ + RHK) * RS * RD * 2

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
        "sample": (f"oracle torch-CPU SwiGLU fwd+bwd on [{n}, {INTER}] bf16 + RoPE fwd+bwd on "
                   f"q [1,{RHQ},{RS},{RD}], k [1,{RHK},{RS},{RD}] bf16 (tables built per call), "
                   f"{reps} reps in {el:.1f} s, {sample_bytes} algorithmic bytes per rep"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
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

    def step():
        for fn in ops.values():
            fn()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # Timed region: exactly K steps, no per-kernel events (each event record
    # inserts ~4.6 us of idle time between kernels on this GPU).
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms_step = e0.elapsed_time(e1) / args.steps

    # Per-kernel launch duration: HIP events on the kernel's stream around
    # 20 back-to-back launches of that kernel alone, eagerly and replayed
    # from a captured graph; the smaller of the two is kept (eager launches
    # of the ~17 us RoPE kernel are timed through each call's host-side
    # argument marshalling, a graph adds ~1.5 us between its nodes).
    reps = 20
    per_op, how = {}, {}
    for name, fn in ops.items():
        eager = time_launches(fn, stream, reps)
        graph, gh = time_graph(fn, stream, reps)
        per_op[name], how[name] = (graph, gh) if graph < eager else (eager, "eager launches")

    ms_step = wall * 1e3 / args.steps
    value = STEP_BYTES / (wall / args.steps) / 1e9
    op_bytes = {"swiglu_fwd": SWIGLU_FWD_BYTES, "swiglu_bwd": SWIGLU_BWD_BYTES,
                "rope_fwd": ROPE_DIR_BYTES, "rope_bwd": ROPE_DIR_BYTES}
    breakdown = {n: {"us": round(per_op[n] * 1e3, 2),
                     "GB/s": round(op_bytes[n] / (per_op[n] * 1e-3) / 1e9, 1), "timing": how[n]}
                 for n in per_op}
    breakdown["gpu_ms_per_step"] = round(gpu_ms_step, 4)
    breakdown["rmsnorm_fp32"] = bench_rmsnorm(dev, stream, reps)
    breakdown["qk_norm_rope_bf16"] = bench_qk_norm_rope(dev, stream, reps)
    breakdown["add_rmsnorm_bf16"] = bench_add_rmsnorm(dev, stream, reps)
    if not args.no_mfma_ops:
        breakdown["flce_fwd_bwd"] = bench_flce(dev, stream, 5)
        breakdown["lora_bwd_layer"] = bench_lora_bwd(dev, stream, 10)
    if not args.no_train_step:
        breakdown["train_step_4layer"] = bench_train_step(dev)
    dom_ms = per_op["swiglu_bwd"]
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
        "avg_launch_us": round(dom_ms * 1e3, 2),
        "timing": how["swiglu_bwd"],
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
        },
        "roofline": roofline,
        "breakdown": breakdown,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

/*
 * metal_liger_amd — C ABI of the MI355X (gfx950) fused-op library.
 *
 * This is the drop-in boundary that replaces the reference's native bridge
 * (the pybind module `metal_liger_ext`, declared in csrc/metal_liger_ops.h:13-36
 * and bound in csrc/bindings.mm:10-33) and the pure-torch bodies of the
 * autograd functions in ops/fused_*.py.
 *
 * Conventions (every entry point):
 *   - Plain pointers and sizes only. Device pointers are `void*`; sizes,
 *     strides and leading dimensions are int64_t and count ELEMENTS.
 *   - The caller allocates every output and every workspace; the library
 *     allocates no device memory. `*_workspace_bytes` queries give the size.
 *   - `stream` is a hipStream_t (NULL = the default stream). Work is enqueued
 *     asynchronously in stream order; nothing synchronizes with the host.
 *   - Return value 0 = success. Non-zero = error; ml_last_error() returns a
 *     thread-local message (the reference raised RuntimeError through
 *     TORCH_CHECK / std::runtime_error, csrc/rms_norm_metal.mm:116-117,
 *     csrc/swiglu_metal.mm:71-72; the Python layer raises RuntimeError with
 *     this message).
 *   - All arithmetic is fp32 internally; outputs are rounded once (RNE) to
 *     their storage dtype.
 */
#ifndef METAL_LIGER_AMD_H
#define METAL_LIGER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ML_ABI_VERSION 6

/* dtype tags */
#define ML_F32 0
#define ML_BF16 1
#define ML_F16 2

/* status codes */
#define ML_OK 0
#define ML_ERR_INVALID 1 /* bad argument (shape, dtype, pointer, size) */
#define ML_ERR_HIP 2     /* a HIP runtime call or kernel launch failed */

/* ABI version of the loaded library (== ML_ABI_VERSION it was built with). */
int ml_abi_version(void);

/* Thread-local message describing the last failed call on this thread. */
const char* ml_last_error(void);

/* ------------------------------------------------------------------ RMSNorm
 * Replaces metal_rms_norm_forward (csrc/metal_liger_ops.h:13-17,
 * csrc/rms_norm_metal.mm:110-160) and the math of
 * _FusedRMSNormFunction.forward (ops/fused_rms_norm.py:31-41).
 *
 *   rrms[r] = 1 / sqrt(mean_c(x[r,c]^2) + eps)
 *   y[r,c]  = (x[r,c] * rrms[r]) * w[c]        (rounded to x's dtype)
 *
 * x, y: [rows, cols] with row strides ldx / ldy (last dim contiguous).
 * w: [cols] of w_dtype. rrms: [rows] fp32 (may be NULL if not needed).
 */
int ml_rmsnorm_fwd(const void* x, int64_t ldx, const void* w, void* y, int64_t ldy,
                   float* rrms, int64_t rows, int64_t cols, float eps, int x_dtype,
                   int w_dtype, void* stream);

/* Workspace for ml_rmsnorm_bwd (fp32 per-block dW partials), in bytes. */
size_t ml_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols);

/*
 * Replaces metal_rms_norm_backward (csrc/metal_liger_ops.h:19-24,
 * csrc/rms_norm_metal.mm:164-214) and _FusedRMSNormFunction.backward
 * (ops/fused_rms_norm.py:43-60).
 *
 *   gw  = dy * w
 *   dx  = gw * r - (x * mean_c(gw * x)) * r^3          (x's dtype)
 *   dw  = sum_r dy * (x * r)                            (w's dtype)
 *
 * r is read from rrms when non-NULL, else recomputed from x and eps (the
 * reference native backward recomputes it, kernels/rms_norm.metal:106-200).
 * dy shares x's dtype. dw is reduced deterministically: fp32 per-block
 * partials in `workspace`, then a fixed-order second pass.
 */
int ml_rmsnorm_bwd(const void* x, int64_t ldx, const void* w, const void* dy, int64_t lddy,
                   const float* rrms, float eps, void* dx, int64_t lddx, void* dw,
                   void* workspace, size_t workspace_bytes, int64_t rows, int64_t cols,
                   int x_dtype, int w_dtype, void* stream);

/*
 * ml_rmsnorm_bwd without a workspace argument: no counterpart in the
 * reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * dW partials live in the library's own 8 MiB device array, one per GPU,
 * held until the process ends; min(rows, 256) * cols * 4 must not exceed
 * it (cols <= 8192 once rows >= 256), else the call fails with an error
 * and launches nothing. Calls allocate nothing.
 * Calls that overlap on one GPU share the array and race; the stream must
 * belong to the current device.
 */
int ml_rmsnorm_bwd_noalloc(const void* x, int64_t ldx, const void* w, const void* dy,
                           int64_t lddy, const float* rrms, float eps, void* dx, int64_t lddx,
                           void* dw, int64_t rows, int64_t cols, int x_dtype, int w_dtype,
                           void* stream);

/*
 * Residual add fused into the norm after it: the decoder layer's
 * `hidden = residual + attn_out; post_attention_layernorm(hidden)`
 * (transformers modeling_qwen3.py, Qwen3DecoderLayer.forward; the step that
 * follows the reference's LoRA o_proj, ops/fused_lora.py:26 "LoRA_W").
 * No single reference function: it fuses torch's add with
 * _FusedRMSNormFunction.forward (ops/fused_rms_norm.py:31-41).
 *
 *   sum[r,c] = x[r,c] + residual[r,c]                  (rounded to x's dtype)
 *   y, rrms  = ml_rmsnorm_fwd of that rounded sum
 *
 * residual shares x's dtype; sum may not alias x or residual.
 */
int ml_rmsnorm_add_fwd(const void* x, int64_t ldx, const void* residual, int64_t ldr,
                       const void* w, void* sum, int64_t lds, void* y, int64_t ldy, float* rrms,
                       int64_t rows, int64_t cols, float eps, int x_dtype, int w_dtype,
                       void* stream);

/*
 * Backward of ml_rmsnorm_add_fwd: the norm's VJP at the saved sum plus the
 * gradient dsum the sum receives from the residual branch, rounded once:
 *
 *   dx = (gw * r - (sum * mean_c(gw * sum)) * r^3) + dsum   (x's dtype)
 *   dw as ml_rmsnorm_bwd; workspace from ml_rmsnorm_bwd_workspace_bytes.
 *
 * dx is the gradient of both x and residual (autograd's add backward gives
 * each the sum's gradient). dx may not alias sum, dy or dsum.
 */
int ml_rmsnorm_add_bwd(const void* sum, int64_t lds, const void* w, const void* dy,
                       int64_t lddy, const void* dsum, int64_t ldd, const float* rrms, float eps,
                       void* dx, int64_t lddx, void* dw, void* workspace, size_t workspace_bytes,
                       int64_t rows, int64_t cols, int x_dtype, int w_dtype, void* stream);

/* ------------------------------------------------------------------- SwiGLU
 * Replaces metal_swiglu_forward (csrc/metal_liger_ops.h:27-30,
 * csrc/swiglu_metal.mm:66-100) and _FusedSwiGLUFunction.forward
 * (ops/fused_swiglu.py:26-35).
 *
 *   out = (gate * sigmoid(gate)) * up                   (n contiguous elements)
 */
int ml_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n, int dtype,
                  void* stream);

/*
 * Replaces metal_swiglu_backward (csrc/metal_liger_ops.h:32-36,
 * csrc/swiglu_metal.mm:106-144) and _FusedSwiGLUFunction.backward
 * (ops/fused_swiglu.py:37-50). sigmoid(gate) is recomputed, not stored.
 *
 *   dup   = dy * (gate * s)
 *   dgate = ((dy * up) * s) * (1 + gate * (1 - s)),    s = sigmoid(gate)
 *
 * dy may be the same buffer as dgate (the backward then runs in place).
 */
int ml_swiglu_bwd(const void* gate, const void* up, const void* dy, void* dgate, void* dup,
                  int64_t n, int dtype, void* stream);

/* --------------------------------------------------------------------- RoPE
 * Rotate-half rotary embedding over one or two [B, H, S, D] tensors (q and,
 * optionally, k — they share B, S, D and the angle source).
 *
 * geom (9 int64 per tensor): {B, H, S, in_sb, in_sh, in_ss, out_sb, out_sh,
 * out_ss}; the D dimension is contiguous (stride 1) in input and output.
 *
 *   y[..j]      = x[j] * c[j]      - x[j+D/2] * sgn * s[j]
 *   y[..j+D/2]  = x[j+D/2] * c[j+D/2] + x[j] * sgn * s[j+D/2]
 *
 * sgn = +1 applies the rotation (forward); sgn = -1 applies the reference's
 * backward, rotate_half with -sin (ops/fused_rope.py:48-57).
 */

/*
 * Table mode: cos/sin given as tensors broadcastable to [B, H, S, D]
 * (replaces _FusedRoPEFunction / _apply_rotary_fused, ops/fused_rope.py:22-75,
 * :110-127). cs_geom (6 int64): {cos_sb, cos_sh, cos_ss, sin_sb, sin_sh, sin_ss}
 * (0 for broadcast dims); the D dimension of cos/sin is contiguous.
 * out_dtype must be the promotion of x_dtype and cs_dtype.
 */
int ml_rope_table(const void* q, void* q_out, const int64_t* q_geom, const void* k, void* k_out,
                  const int64_t* k_geom, int64_t D, const void* cos, const void* sin,
                  const int64_t* cs_geom, float sgn, int x_dtype, int cs_dtype, int out_dtype,
                  void* stream);

/*
 * Position mode: cos/sin computed in-kernel, angle = float(pos[b,s]) *
 * inv_freq[j mod D/2] (fp32, as the HF rotary module builds its tables) —
 * no table is read. positions: int64 [B, S] with strides pos_sb, pos_ss
 * (pos_sb = 0 to share one row). inv_freq: fp32 [D/2] device array.
 * Output dtype = x_dtype.
 */
int ml_rope_pos(const void* q, void* q_out, const int64_t* q_geom, const void* k, void* k_out,
                const int64_t* k_geom, int64_t D, const int64_t* positions, int64_t pos_sb,
                int64_t pos_ss, const float* inv_freq, float sgn, int x_dtype, void* stream);

/* ---------------------------------------------- q/k head-dim RMSNorm + RoPE
 * Qwen3 attention's q_norm / k_norm (transformers' Qwen3RMSNorm over the head
 * dimension) followed by rotate-half RoPE from cos/sin tables
 * (apply_rotary_pos_emb), q and k in one launch. The reference's patcher
 * leaves these norms unfused (patch.py:104-131 replaces only the layer
 * norms); the fused form replaces the sequence q_norm -> transpose ->
 * apply_rotary_pos_emb of the Qwen3 attention forward.
 *
 * Rows are [B, H, S, D] with D in {32, 64, 128, 256} contiguous; q and k share B,
 * S, D, eps and the tables. Per row (fp32 arithmetic, one rounding on store):
 *
 *   n = x * rsqrt(mean(x^2) + eps) * w
 *   y[j]     = n[j] c[j] - n[j+D/2] s[j]
 *   y[j+D/2] = n[j+D/2] c[j+D/2] + n[j] s[j+D/2]          (j < D/2)
 *
 * x, y, the tables (and in the backward dy, dx) have dtype x_dtype; the
 * weights w [D] have x_dtype or fp32 (w_dtype). Every base pointer is 16-byte
 * aligned and every stride is a multiple of 16 bytes. Per-head tables (a
 * non-zero head stride) must cover max(Hq, Hk) heads.
 *
 * geom (9 int64 per tensor): {B, H, S, x_sb, x_sh, x_ss, y_sb, y_sh, y_ss}.
 * cs_geom (6 int64): {cos_sb, cos_sh, cos_ss, sin_sb, sin_sh, sin_ss}, 0 on
 * broadcast dimensions. k may be NULL (q only); a NULL k whose k_geom
 * describes no elements is an empty k (its weight gradient is zero).
 */
int ml_qk_norm_rope_fwd(const void* q, void* q_out, const int64_t* q_geom, const void* q_weight,
                        const void* k, void* k_out, const int64_t* k_geom, const void* k_weight,
                        int64_t D, float eps, const void* cos, const void* sin,
                        const int64_t* cs_geom, int x_dtype, int w_dtype, void* stream);

/*
 * Backward (exact for any tables): dx from dy, and optionally dw = sum over
 * rows of dn * x * rsqrt(mean(x^2) + eps) in w_dtype, where dn is dy rotated
 * back. geom (12 int64 per tensor): {B, H, S, x strides (b, h, s), dy strides,
 * dx strides}. dq_weight / dk_weight may be NULL to skip a weight gradient;
 * when either is requested the workspace holds
 * ml_qk_norm_rope_bwd_workspace_bytes(B, S, Hq, Hk, D) bytes. dw is summed in
 * a fixed order (deterministic).
 */
size_t ml_qk_norm_rope_bwd_workspace_bytes(int64_t B, int64_t S, int64_t Hq, int64_t Hk,
                                           int64_t D);
int ml_qk_norm_rope_bwd(const void* q, const void* dq_out, void* dq, const int64_t* q_geom,
                        const void* q_weight, void* dq_weight, const void* k, const void* dk_out,
                        void* dk, const int64_t* k_geom, const void* k_weight, void* dk_weight,
                        int64_t D, float eps, const void* cos, const void* sin,
                        const int64_t* cs_geom, int x_dtype, int w_dtype, void* workspace,
                        size_t workspace_bytes, void* stream);

/* ------------------------------------------- fused linear cross-entropy (FLCE)
 * Replaces _FusedLinearCrossEntropyFunction (ops/fused_linear_cross_entropy.py:
 * 82-185) and its chunk loops (:39-80). bf16 hidden [n_tokens, hidden_size]
 * (row stride ldh) and weight [vocab, hidden_size] (row stride ldw); optional
 * bias [vocab] (fp32 or bf16, bias_dtype; NULL for none); int64 labels
 * [n_tokens] where ignore_index marks ignored tokens. hidden_size and vocab
 * must be multiples of 8.
 *
 * Forward: loss = sum_valid (lse - z_label) / max(#valid, 1) (fp32 scalar),
 * lse fp32 [n_tokens], n_valid fp32 scalar (#valid tokens). No [tokens,
 * vocab] tensor is ever allocated; the workspace holds per-row partials.
 * Gradient outputs of the entry points below are written as 16-byte vectors
 * and must be 16-byte aligned (refused otherwise).
 */
size_t ml_flce_fwd_workspace_bytes(int64_t n_tokens, int64_t vocab);
int ml_flce_fwd(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const void* bias,
                int bias_dtype, const int64_t* labels, int64_t n_tokens, int64_t vocab,
                int64_t hidden_size, int64_t ignore_index, float* loss, float* lse, float* n_valid,
                void* workspace, size_t workspace_bytes, void* stream);

/*
 * Backward for d(loss) = *grad_loss (device fp32 scalar): d_hidden bf16
 * [n_tokens, hidden_size] and d_weight bf16 [vocab, hidden_size] (dense),
 * either may be NULL to skip it (a frozen lm_head skips the dW GEMMs). chunk
 * (multiple of 8) is the vocabulary slice whose bf16 dlogits are held at once:
 * the workspace is n_tokens * chunk * 2 bytes (+ an fp32 dH accumulator).
 * No bias gradient, as in the reference.
 */
size_t ml_flce_bwd_workspace_bytes(int64_t n_tokens, int64_t hidden_size, int64_t chunk,
                                   int need_dhidden);
int ml_flce_bwd(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const void* bias,
                int bias_dtype, const int64_t* labels, int64_t n_tokens, int64_t vocab,
                int64_t hidden_size, int64_t ignore_index, const float* lse, const float* n_valid,
                const float* grad_loss, int64_t chunk, void* d_hidden, void* d_weight,
                void* workspace, size_t workspace_bytes, void* stream);

/*
 * Loss and gradients in one call, with the logits computed once (the schedule
 * _FusedLinearCrossEntropyFunction uses; replaces its forward + backward,
 * ops/fused_linear_cross_entropy.py:93-185, whose backward recomputes every
 * logits chunk). Tokens go in chunks of token_chunk: per chunk one bf16
 * [token_chunk, vocab] workspace buffer holds exp(z - c) with one shift c
 * per row (the row's label logit + 30; rows whose values would leave the
 * safe range, a token loss above ~78 nats, are recomputed with their exact
 * max), so that the dlogits are a row factor times the buffer (label entry
 * rewritten): dH rows come from a split-K GEMM whose reduction applies the
 * row factors and dW accumulates (bf16) from the buffer and the
 * factor-scaled hidden rows. Outputs as ml_flce_fwd, plus d_hidden
 * [n_tokens, hidden_size] and d_weight [vocab, hidden_size] (bf16, dense;
 * either may be NULL) formed for d(loss) = 1. With both NULL this is the
 * loss-only forward (its workspace query still counts the buffer; the
 * smaller ml_flce_fwd is the loss-only entry point).
 */
size_t ml_flce_fwd_grad_workspace_bytes(int64_t n_tokens, int64_t vocab, int64_t hidden_size,
                                        int64_t token_chunk, int need_dhidden);
int ml_flce_fwd_grad(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                     const void* bias, int bias_dtype, const int64_t* labels, int64_t n_tokens,
                     int64_t vocab, int64_t hidden_size, int64_t ignore_index, int64_t token_chunk,
                     float* loss, float* lse, float* n_valid, void* d_hidden, void* d_weight,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * The upstream gradient of the loss (the grad_output of the reference's
 * backward, ops/fused_linear_cross_entropy.py:160-167) applied to gradients
 * from ml_flce_fwd_grad: d_hidden[0:n_hidden] and d_weight[0:n_weight] (bf16)
 * are multiplied by *grad_loss (device fp32 scalar) in place; nothing is
 * written when it equals 1. Either array may be NULL with its size 0.
 */
int ml_flce_scale_grads(const float* grad_loss, void* d_hidden, int64_t n_hidden, void* d_weight,
                        int64_t n_weight, void* stream);

/*
 * fp32 fused linear cross-entropy (hidden, weight, bias and both gradients
 * fp32; any H and V), with the reference's own vocabulary-chunked schedule
 * (ops/fused_linear_cross_entropy.py:39-80, :93-185): per chunk of `chunk`
 * vocabulary columns an fp32 [tokens, chunk] logits tile (the reference's
 * chunk), online (max, sum exp) partials, then per chunk again the
 * dlogits (softmax - one_hot) * mask / max(#valid, 1), dH += D W_c and
 * dW_c = D^T H. Outputs as ml_flce_fwd_grad (gradients for d(loss) = 1;
 * d_hidden / d_weight may be NULL). bias fp32 or NULL.
 */
size_t ml_flce_fwd_grad_f32_workspace_bytes(int64_t n_tokens, int64_t vocab, int64_t chunk);
int ml_flce_fwd_grad_f32(const float* hidden, int64_t ldh, const float* weight, int64_t ldw,
                         const float* bias, const int64_t* labels, int64_t n_tokens,
                         int64_t vocab, int64_t hidden_size, int64_t ignore_index, int64_t chunk,
                         float* loss, float* lse, float* n_valid, float* d_hidden,
                         float* d_weight, void* workspace, size_t workspace_bytes, void* stream);

/* ml_flce_scale_grads for fp32 gradients (16-byte aligned). */
int ml_flce_scale_grads_f32(const float* grad_loss, float* d_hidden, int64_t n_hidden,
                            float* d_weight, int64_t n_weight, void* stream);

/* ----------------------------------------------------------- fused LoRA bwd
 * Replaces _LoRA_QKV.backward (ops/fused_lora.py:121-171). Three adapters
 * (q, k, v) share the saved input X [n_tokens, in_features] (bf16). For
 * adapter i: dY[i] [n_tokens, out_features[i]], base W[i] [out, in], B[i]
 * [out, rank] (bf16), scale[i] a HOST float (PEFT's lora_alpha / r).
 * A_stack [3 rank, in] stacks A_q, A_k, A_v (bf16); XA [n_tokens, 3 rank] is
 * X A_stack^T from the forward. Outputs: dX bf16 [n_tokens, in];
 * dA fp32 [3 rank, in] (dA_q, dA_k, dA_v stacked); dB[i] fp32 [out, rank].
 * in_features, out_features and rank must be multiples of 8; dX is written
 * as 16-byte rows and must be 16-byte aligned. No gradient for the frozen
 * base weights, as in the reference.
 */
size_t ml_lora_qkv_bwd_workspace_bytes(int64_t n_tokens, int64_t in_features,
                                       const int64_t* out_features, int64_t rank);
int ml_lora_qkv_bwd(const void* X, int64_t n_tokens, int64_t in_features, const void* const* dY,
                    const int64_t* out_features, const void* const* W, const void* A_stack,
                    const void* const* B, const float* scale, const void* XA, int64_t rank,
                    void* dX, float* dA, float* const* dB, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * One projection with LoRA: the "LoRA_W" (output / o_proj) block the
 * reference announces but never implements (ops/fused_lora.py:26), with the
 * per-adapter formulas of _LoRA_QKV.backward (:121-171) and _lora_linear's
 * forward (:69-82): X [n_tokens, in_features], dY [n_tokens, out_features],
 * W [out, in], A [rank, in], B [out, rank] (bf16), scale a HOST float, XA =
 * X A^T [n_tokens, rank] from the forward. Outputs: dX bf16 [n, in] =
 * dY W + s (dY B) A; dA fp32 [rank, in] = s (dY B)^T X; dB fp32 [out, rank]
 * = s dY^T XA. Same size rules as ml_lora_qkv_bwd.
 */
size_t ml_lora_linear_bwd_workspace_bytes(int64_t n_tokens, int64_t in_features,
                                          int64_t out_features, int64_t rank);
int ml_lora_linear_bwd(const void* X, int64_t n_tokens, int64_t in_features, const void* dY,
                       int64_t out_features, const void* W, const void* A, const void* B,
                       float scale, const void* XA, int64_t rank, void* dX, float* dA, float* dB,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * Replaces _LoRA_MLP.backward (ops/fused_lora.py:209-266): SwiGLU MLP with
 * LoRA on gate / up / down. Saved from the forward (bf16): X [n, hidden],
 * gate / up / h [n, intermediate], XA_GU = X [A_G; A_U]^T [n, 2 rank],
 * hA_D = h A_D^T [n, rank]. Weights: WG, WU [intermediate, hidden], WD
 * [hidden, intermediate], A_GU [2 rank, hidden] (A_G; A_U), A_D [rank,
 * intermediate], BG, BU [intermediate, rank], BD [hidden, rank]; scale = HOST
 * floats {s_G, s_U, s_D}. Outputs: dX bf16 [n, hidden]; fp32 dA_GU [2 rank,
 * hidden], dA_D [rank, intermediate], dB_G, dB_U [intermediate, rank], dB_D
 * [hidden, rank] (dX 16-byte aligned: it is written as 16-byte rows).
 * dH = dY W_D + s_D (dY B_D) A_D is formed in bf16 and the SwiGLU backward
 * then runs over it in place.
 * h may be NULL: it is then silu(gate) * up rounded to bf16 exactly as
 * ml_swiglu_fwd forms it (the reference saves that product from its
 * forward, :197-204), recomputed from gate and up instead of read (at rank
 * 16 inside the pass that runs the SwiGLU backward; otherwise formed in the
 * workspace). A caller that passes h gets it used as given.
 */
size_t ml_lora_mlp_bwd_workspace_bytes(int64_t n_tokens, int64_t hidden, int64_t intermediate,
                                       int64_t rank);
int ml_lora_mlp_bwd(const void* X, int64_t n_tokens, int64_t hidden, int64_t intermediate,
                    const void* gate, const void* up, const void* h, const void* dY, const void* WG,
                    const void* WU, const void* WD, const void* A_GU, const void* A_D,
                    const void* BG, const void* BU, const void* BD, const float* scale,
                    const void* XA_GU, const void* hA_D, int64_t rank, void* dX, float* dA_GU,
                    float* dA_D, float* dB_G, float* dB_U, float* dB_D, void* workspace,
                    size_t workspace_bytes, void* stream);

/* X A^T for the adapters' stacked A matrices (the rank-r products of the
 * LoRA forwards: F.linear(x, A) in _lora_linear, ops/fused_lora.py:79-81):
 * X [n_tokens, in_features] bf16 (row stride ldx), A [rank_total,
 * in_features] bf16 dense, rank_total 1..64; XA [n_tokens, rank_total] bf16
 * (row stride ldo) = X A^T with fp32 accumulation. One pass over X (no
 * split-K partials). in_features and ldx multiples of 8, X and A 16-byte
 * aligned. */
int ml_lora_xa(const void* X, int64_t n_tokens, int64_t in_features, int64_t ldx, const void* A,
               int64_t rank_total, void* XA, int64_t ldo, void* stream);

/* --------------------------------------------------------------------- GEMM
 * bf16 MFMA GEMM (fp32 accumulation): C = alpha * A B + beta * C.
 * No reference counterpart: the reference's contractions are torch.mm /
 * F.linear calls inside ops/fused_linear_cross_entropy.py:44,64,78-79 and
 * ops/fused_lora.py:79-81,142-161,228-258; this is the engine those paths
 * run on here, exported for tests and for callers that need a plain product.
 *
 * a_layout 0: A is [M, K] row-major (element (m, k) at A[m * lda + k]);
 *          1: A is stored transposed, [K, M] row-major (A[k * lda + m]).
 * b_layout 0: B is stored transposed, [N, K] row-major (an nn.Linear weight);
 *          1: B is [K, N] row-major.
 * K (and every segment length) must be a multiple of 8, leading dimensions
 * multiples of 8, pointers 16-byte aligned, and M (N) a multiple of 8 when A
 * (B) is stored transposed. C is fp32 or bf16 (c_dtype), row-major with ldc;
 * a bf16 C needs ldc a multiple of 8 and a 16-byte aligned base (refused
 * otherwise), an fp32 C any ldc >= N.
 */
int ml_gemm_bf16(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, int a_layout,
                 const void* B, int64_t ldb, int b_layout, void* C, int64_t ldc, int c_dtype,
                 float alpha, float beta, void* stream);

/* Same product with K split into nseg (1..8) segments, segment s pairing
 * A_s (lda_s) with B_s (ldb_s) over k_lens[s]: C = alpha * sum_s A_s B_s + beta * C. */
int ml_gemm_bf16_segments(int64_t M, int64_t N, int nseg, const int64_t* k_lens,
                          const void* const* a_ptrs, const int64_t* ldas, const void* const* b_ptrs,
                          const int64_t* ldbs, int a_layout, int b_layout, void* C, int64_t ldc,
                          int c_dtype, float alpha, float beta, void* stream);

/* count (1..3) independent segmented products in ONE launch, A [M_g, K]
 * row-major (a_layout 0) for every product: product g has nseg[g] segments,
 * the next nseg[g] entries of k_lens / a_ptrs / ldas / b_ptrs / ldbs, and
 * writes C[g] (ldc[g]) = alpha * sum_s A_s B_s + beta * C[g]. For products
 * too small to fill the GPU on their own: the LoRA QKV forward's q, k and v
 * projections (ops/fused_lora.py:85-120 forms them one after another; k and
 * v have half as many 256 x 256 tiles as there are CUs) share rounds of
 * tiles. Same operand rules as ml_gemm_bf16_segments. */
int ml_gemm_bf16_segments_group(int count, const int64_t* M, const int64_t* N, const int* nseg,
                                const int64_t* k_lens, const void* const* a_ptrs,
                                const int64_t* ldas, const void* const* b_ptrs,
                                const int64_t* ldbs, int b_layout, void* const* C,
                                const int64_t* ldc, int c_dtype, float alpha, float beta,
                                void* stream);

/* Split-K form with a tile shape (tile_cfg 0: 256x256, 1: 256x32 for
 * rank-r outputs, 2: 64x256 for few-row outputs): ksplit slices of K write
 * fp32 partials to `workspace` (ml_gemm_splitk_workspace_bytes), summed in a
 * fixed order into C = alpha * A B + beta * C. Same operand rules as above. */
size_t ml_gemm_splitk_workspace_bytes(int64_t M, int64_t N, int64_t K, int ksplit);
int ml_gemm_bf16_splitk(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, int a_layout,
                        const void* B, int64_t ldb, int b_layout, void* C, int64_t ldc, int c_dtype,
                        float alpha, float beta, int tile_cfg, int ksplit, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * fp32 products for the fp32 forms of the LoRA and FLCE ops (the reference
 * runs _lora_linear / _LoRA_QKV / _LoRA_MLP in the activation dtype,
 * ops/fused_lora.py:69-266, and its FLCE in fp32,
 * ops/fused_linear_cross_entropy.py:108-109):
 *   C = alpha * sum_s op(A_s) op(B_s) + beta * C      (fp32 throughout,
 * v_mfma_f32_32x32x2_f32), layouts and K segments as ml_gemm_bf16_segments;
 * any M, N, K and leading dimensions.
 */
int ml_gemm_f32_segments(int64_t M, int64_t N, int nseg, const int64_t* k_lens,
                         const void* const* a_ptrs, const int64_t* ldas,
                         const void* const* b_ptrs, const int64_t* ldbs, int a_layout,
                         int b_layout, float* C, int64_t ldc, float alpha, float beta,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* METAL_LIGER_AMD_H */

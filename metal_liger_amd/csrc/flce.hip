// Fused linear cross-entropy for gfx950
// (ops/fused_linear_cross_entropy.py:39-185 of the reference).
//
// Two schedules share the kernels below.
//
// Loss and gradients in one pass (ml_flce_fwd_grad), over chunks of T tokens:
//   1. a shift per row, c = (label logit h . W[y], or the logit of entry 0
//      for a row without a label in range) + 30 (shift_kernel);
//   2. Z = H_c W^T (+ b) as a bf16 MFMA GEMM whose epilogue stores e =
//      exp(z - c) in bf16 ([T, vocab] buffer) and writes per-row, per
//      64-column (max z, sum e) partials;
//   3. a row pass: S = sum e, lse = c + log S, the masked loss terms, the row
//      factor alpha = mask / (n_valid S), the label entry rewritten as
//      exp(z_y - c) - S, and the scaled hidden rows alpha h. Then
//        dlogits = (softmax - one_hot) * mask / n_valid = diag(alpha) E'
//      with no pass over the [T, vocab] buffer. A row whose log S leaves
//      [-36, 48] (its cross-entropy against the pseudo label above 78 nats,
//      or a non-finite S) flags its 256-row tile; steps 2-3 run again for the
//      flagged tiles with c = the row's exact max (the launches are made
//      every chunk; without a flag their blocks return at once);
//   4. dH_c = diag(alpha) (E' W)  (split-K MFMA GEMM over the vocabulary,
//      the row factor applied in the fixed-order reduction; MN-major W);
//   5. dW  += E'^T (diag(alpha) H_c)  (MFMA GEMM, both operands MN-major;
//      accumulated in bf16 across token chunks).
//   The logits are computed once: three GEMMs (2 N V H FLOP each) in total,
//   against the four of a vocabulary-chunked schedule that must recompute
//   them after the logsumexp is known. The gradients are formed for
//   d(loss) = 1; ml_flce_scale_grads applies the actual upstream gradient.
//   Peak extra memory: one [T, vocab] bf16 buffer (no [tokens, vocab]
//   tensor exists; the reference keeps an fp32 copy of W, an fp32 dW and an
//   fp32 [tokens, chunk] logits chunk).
//
// Loss only (ml_flce_fwd) + vocabulary-chunked backward (ml_flce_bwd), for
// callers that keep only (lse, n_valid) between the passes:
//   forward: ONE logits GEMM over the whole vocabulary with the (m, s)
//   epilogue (nothing stored), the row pass and a fixed-order mean over
//   valid tokens (clamped at 1, :149).
//   backward, per vocabulary chunk of `chunk` columns (the reference's
//   chunk_size, :57-80): recompute the logits tile, write bf16 dlogits from
//   the epilogue, dH += D W_c (fp32 accumulator), dW_c = D^T H.
// dH / dW are skipped when not requested (frozen lm_head).
#include <math.h>

#include <algorithm>

#include "gemm_core.h"

namespace mla {
namespace flce {
namespace {

using namespace gemm;

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kColBlock = big::WN;  // columns per (max, sum) partial: one wave's sub-tile

__device__ __forceinline__ float exp_f(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

// Reductions over the 16 lanes of a group (the lanes that hold one row of a
// 16 x 16 accumulator tile), with DPP lane moves inside 16-lane rows:
// quad_perm [1,0,3,2] (xor 1), quad_perm [2,3,0,1] (xor 2), row_half_mirror
// (lane i <-> 7 - i in each half-row) and row_mirror (i <-> 15 - i); after
// the four steps every lane holds the result over its 16 lanes.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF,
                                                            0xF, false));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

__device__ __forceinline__ float grp16_max(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  return fmaxf(v, dpp_f<kDppMirror>(v));
}
__device__ __forceinline__ float grp16_sum(float v) {
  v += dpp_f<kDppXor1>(v);
  v += dpp_f<kDppXor2>(v);
  v += dpp_f<kDppHalfMirror>(v);
  return v + dpp_f<kDppMirror>(v);
}

template <typename TB>
__device__ __forceinline__ float bias_at(const TB* b, int64_t n) {
  return b ? to_f32(b[n]) : 0.f;
}

// ------------------------------------------------------------ forward epi --
// Loss only: each wave reduces its 64 logit columns to a (max, sum exp(z -
// max)) partial per row, pmax / psum [row * nblk + column block]; nothing
// else is stored. The label logits come from label_logit_kernel.
template <typename TB>
struct EpiRowLse {
  const TB* bias;
  float* pmax;  // [M][nblk]
  float* psum;  // [M][nblk]
  int M, V, nblk;

  template <bool FULL>
  __device__ __forceinline__ void rows(f32x4_t (&acc)[big::TM][big::TN], int m0, int n0,
                                       int lane) const {
    const int c = lane & 15;
    float bj[big::TN];
    bool okj[big::TN];
#pragma unroll
    for (int j = 0; j < big::TN; ++j) {
      const int n = n0 + 16 * j + c;
      okj[j] = FULL || n < V;
      bj[j] = bias ? (okj[j] ? to_f32(bias[n]) : 0.f) : 0.f;
    }
    const int nb = n0 / kColBlock;
#pragma unroll
    for (int i = 0; i < big::TM; ++i) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float z[big::TN];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < big::TN; ++j) {
          z[j] = okj[j] ? acc[i][j][v] + bj[j] : -INFINITY;
          mx = fmaxf(mx, z[j]);
        }
        mx = grp16_max(mx);  // finite: a wave's first column is always < V
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < big::TN; ++j) s += exp_f(z[j] - mx);  // 0 for columns past V
        s = grp16_sum(s);
        const int m = m0 + 16 * i + 4 * (lane >> 4) + v;
        if (c == 0 && m < M) {
          pmax[(int64_t)m * nblk + nb] = mx;
          psum[(int64_t)m * nblk + nb] = s;
        }
      }
    }
  }

  __device__ __forceinline__ void operator()(f32x4_t (&acc)[big::TM][big::TN], int m0, int n0,
                                             int lane, char*, int) const {
    // a wave whose 64 columns all lie past the vocabulary (in the last tile)
    // owns no partial slot
    if (n0 >= V) return;
    if (n0 + big::WN <= V)
      rows<true>(acc, m0, n0, lane);
    else
      rows<false>(acc, m0, n0, lane);
  }
};

// Reduction of x[k] (k < 16) over the 16 lanes of each 16-lane group, for
// 16 values at once, by recursive halving: four exchanges with the partner
// lane (row_mirror: c <-> 15 - c; row_half_mirror: c <-> c ^ 7; quad_perm
// xor 2 and xor 1), at each of which a lane keeps the half of its values
// selected by the bit in which it differs from its partner (bits 3, 2, 1, 0)
// and adds the partner's copy of that half. Lane c of the group ends with
// the reduction of value c (60 operations for 16 rows, against 128 for
// sixteen separate butterflies, and one result per lane instead of a copy
// of each in every lane).
template <bool MAX>
__device__ __forceinline__ float grp16_reduce16(float (&x)[16], int c) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  {
    const bool hi = (c >> 3) & 1;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float send = hi ? x[k] : x[k + 8];
      const float keep = hi ? x[k + 8] : x[k];
      x[k] = op(keep, dpp_f<kDppMirror>(send));
    }
  }
  {
    const bool hi = (c >> 2) & 1;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float send = hi ? x[k] : x[k + 4];
      const float keep = hi ? x[k + 4] : x[k];
      x[k] = op(keep, dpp_f<kDppHalfMirror>(send));
    }
  }
  {
    const bool hi = (c >> 1) & 1;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const float send = hi ? x[k] : x[k + 2];
      const float keep = hi ? x[k + 2] : x[k];
      x[k] = op(keep, dpp_f<kDppXor2>(send));
    }
  }
  const bool hi = c & 1;
  const float send = hi ? x[0] : x[1];
  const float keep = hi ? x[1] : x[0];
  return op(keep, dpp_f<kDppXor1>(send));
}

// One-pass (loss + gradients): every row m has a shift c_m chosen before
// the product (shift_kernel). The epilogue (r4 engine, a wave's whole 128 x
// 128 sub-tile at once) stores e = exp(z - c_m) in bf16 at E[m * ldE + n]
// and writes, per row and 128-column block, the max of z and the sum of e
// (fp32, before rounding): pmax / psum [m * nblk + block]. With one shift
// per row the stored values need no per-block rescaling afterwards: the
// dlogits of row m are alpha_m e' (e' = e with the label entry rewritten,
// alpha_m a row factor), so the row factor goes into the dH reduction and
// into the hidden rows of the dW product instead of a pass over the [T, V]
// buffer.
// tile_flags (optional): only row tiles with a nonzero flag are computed
// (the recomputation of rows whose shift was out of range).
constexpr int kShiftBlock = 128;  // columns per partial: one r4 wave's sub-tile

template <typename TB>
struct EpiShiftExp {
  const TB* bias;
  const float* shift;     // [M]
  const int* tile_flags;  // null: every tile
  float* pmax;            // [M][nblk]
  float* psum;            // [M][nblk]
  bf16* E;
  int64_t ldE;
  int M, V, nblk;

  __device__ __forceinline__ bool skip_tile(int tm) const {
    return tile_flags != nullptr && tile_flags[tm] == 0;
  }

  // acc[h][i][j][v]: row m0 + 16 i + 4 (lane / 16) + v, column n0 + 64 h +
  // 16 j + lane % 16. Each e is rounded to bf16 as soon as it is formed and
  // written to the wave's LDS (16 KB per 128 x 64 half, the staged layout of
  // stage_rows_bf16: column-major 16 x 16 blocks, 8-byte writes); the halves
  // are then read back as rows of 8 columns (transposing reads) and stored
  // with 16-byte stores.
  template <bool FULL>
  __device__ __forceinline__ void tile(const f32x4_t (&acc)[2][big::TM][4], int m0, int n0,
                                       int lane, char* lds) const {
    const int c = lane & 15, G = lane >> 4;
    const int mq = m0 + 4 * G;
    // the shifts of this lane's rows mq + 16 i + v, all loaded before the
    // first is used (16-byte loads: m0 is a multiple of 128)
    f32x4_t csh[big::TM];
    if (m0 + 128 <= M) {
#pragma unroll
      for (int i = 0; i < big::TM; ++i) csh[i] = *reinterpret_cast<const f32x4_t*>(shift + mq + 16 * i);
    } else {
#pragma unroll
      for (int i = 0; i < big::TM; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) csh[i][v] = mq + 16 * i + v < M ? shift[mq + 16 * i + v] : 0.f;
    }
    float bj[2][4];
    bool okj[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + 64 * h + 16 * j + c;
        okj[h][j] = FULL || n < V;
        bj[h][j] = bias ? (okj[h][j] ? to_f32(bias[n]) : 0.f) : 0.f;
      }
    char* wr = lds + (c * 16 + 4 * G) * 2;
    const int nb = n0 / kShiftBlock;
#pragma unroll
    for (int b = 0; b < 2; ++b) {  // rows of i = 4 b .. 4 b + 3: 16 per lane group
      float xm[16], xs[16];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int i = 4 * b + ii;
        float cl[4], mx[4], sm[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          cl[v] = csh[i][v] * kLog2e;
          mx[v] = -INFINITY;
          sm[v] = 0.f;
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            bf16x4_t w;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              float z = acc[h][i][j][v];
              if (bias) z += bj[h][j];
              if (!FULL) z = okj[h][j] ? z : -INFINITY;
              mx[v] = fmaxf(mx[v], z);
              const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(z, kLog2e, -cl[v]));  // 0 past V
              sm[v] += e;
              w[v] = static_cast<bf16>(e);
            }
            *reinterpret_cast<bf16x4_t*>(wr + h * r4::EPI_BYTES + (i * 4 + j) * 512) = w;
          }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          xm[4 * ii + v] = mx[v];
          xs[4 * ii + v] = sm[v];
        }
      }
      // lane c of group G gets row 16 (4 b + c / 4) + 4 G + c % 4
      const float rm = grp16_reduce16<true>(xm, c);
      const float rs = grp16_reduce16<false>(xs, c);
      const int m = m0 + 16 * (4 * b + (c >> 2)) + 4 * G + (c & 3);
      if (m < M) {
        pmax[(int64_t)m * nblk + nb] = rm;
        psum[(int64_t)m * nblk + nb] = rs;
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's writes are in LDS
    __builtin_amdgcn_wave_barrier();
    typedef __attribute__((address_space(3))) i16x4_t* lp;
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    const int L = lane & 15, a = L >> 2, bq = L & 3;
    const int cb = 8 * ((lane >> 4) & 1);
    const int jo = lane >> 5;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const char* rd = lds + h * r4::EPI_BYTES + jo * 512 + ((cb + a) * 16 + 4 * bq) * 2;
#pragma unroll
      for (int q = 0; q < big::TM * 2; ++q) {
        const int i = q >> 1, jp = q & 1;
        const char* blk = rd + (i * 4 + 2 * jp) * 512;
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lp)(blk));
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lp)(blk + 4 * 32));
        const int m = m0 + 16 * i + L;
        const int n = n0 + 64 * h + 16 * (2 * jp + jo) + cb;
        if (m >= M) continue;
        bf16* dst = E + (int64_t)m * ldE + n;
        if (FULL || n + 8 <= V) {
          *reinterpret_cast<i16x8_t*>(dst) = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        } else {
#pragma unroll
          for (int k = 0; k < 8; ++k)
            if (n + k < V) dst[k] = __builtin_bit_cast(bf16, k < 4 ? lo[k] : hi[k - 4]);
        }
      }
    }
  }

  __device__ __forceinline__ void full_tile(f32x4_t (&acc)[2][big::TM][4], int m0, int n0,
                                            int lane, char* lds) const {
    if (n0 >= V) return;  // no partial slot, nothing to store
    if (n0 + kShiftBlock <= V)
      tile<true>(acc, m0, n0, lane, lds);
    else
      tile<false>(acc, m0, n0, lane, lds);
  }
};

// zy[t] = h_t . W[label_t] (+ b[label_t]) for a label in [0, V), else 0
// (the label logit, as the reference forms it from the gathered weight rows,
// ops/fused_linear_cross_entropy.py:131-134). One wave per token; H % 8 == 0.
template <typename TB>
__global__ __launch_bounds__(256) void label_logit_kernel(
    const bf16* __restrict__ hidden, int64_t ldh, const bf16* __restrict__ weight, int64_t ldw,
    const TB* __restrict__ bias, const int64_t* __restrict__ labels, int M, int64_t V, int H,
    float* __restrict__ zy) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int64_t lab = labels[row];
  if (lab < 0 || lab >= V) {
    if (lane == 0) zy[row] = 0.f;
    return;
  }
  const bf16* h = hidden + (int64_t)row * ldh;
  const bf16* w = weight + lab * ldw;
  float acc = 0.f;
  for (int k = lane * 8; k < H; k += 64 * 8) {
    float a[8], b[8];
    load_n<bf16, 8>(h + k, a);
    load_n<bf16, 8>(w + k, b);
#pragma unroll
    for (int q = 0; q < 8; ++q) acc += a[q] * b[q];
  }
  acc = wave_sum(acc);
  if (lane == 0) zy[row] = acc + (bias ? to_f32(bias[lab]) : 0.f);
}

// n_valid = #(labels != ignore), as fp32 (one block).
__global__ __launch_bounds__(1024) void count_valid_kernel(const int64_t* __restrict__ labels, int M,
                                                           int64_t ignore, float* __restrict__ n_valid) {
  __shared__ float sc[16];
  float c = 0.f;
  for (int i = threadIdx.x; i < M; i += 1024) c += labels[i] != ignore ? 1.f : 0.f;
  c = wave_sum(c);
  if ((threadIdx.x & 63) == 0) sc[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int i = 0; i < 16; ++i) t += sc[i];
    n_valid[0] = t;
  }
}

// ------------------------------------------------ one pass: row shifts --
// The shift of a row is its pseudo-label logit plus kShiftMargin: the label
// logit z_y for a label in [0, V), else the logit of vocabulary entry 0. With
// c = z_p + kShiftMargin, log S = log sum_v exp(z_v - c) = (lse - z_p) -
// kShiftMargin, and lse - z_p >= 0 (lse is at least every logit). A row is
// computed from its shift when log S lies in [kLogSMin, kLogSMax], i.e.
// when its cross-entropy against the pseudo label is at most 78 nats:
//   - every stored e = exp(z - c) <= S <= e^48 and the dH sums of e W stay
//     far inside fp32;
//   - S >= e^-36 keeps the row's largest e (>= S / V) a normal bf16 number
//     with 39 e-folds of normal range below it: entries lost to underflow
//     carry < e^-39 of the row's largest probability;
//   - the row factor alpha = mask / (n_valid S) and the scaled hidden rows
//     alpha h stay normal for any n_valid < 2^31.
// Rows outside the window (and non-finite S) flag their 256-row tile and are
// recomputed with c = the row's exact max (then S is in [1, V]).
constexpr float kShiftMargin = 30.f;
constexpr float kLogSMin = -36.f, kLogSMax = 48.f;

// zy[t] = h_t . W[label_t] (+ b) for a label in [0, V), else 0; shift[t] =
// the pseudo-label logit + kShiftMargin. Block 0 also clears the chunk's
// n_flags tile flags. One wave per token; H % 8 == 0.
template <typename TB>
__global__ __launch_bounds__(256) void shift_kernel(
    const bf16* __restrict__ hidden, int64_t ldh, const bf16* __restrict__ weight, int64_t ldw,
    const TB* __restrict__ bias, const int64_t* __restrict__ labels, int M, int64_t V, int H,
    float* __restrict__ zy, float* __restrict__ shift, int* __restrict__ tile_flags, int n_flags) {
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < n_flags; i += 256) tile_flags[i] = 0;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int64_t lab = labels[row];
  const bool inrange = lab >= 0 && lab < V;
  const int64_t idx = inrange ? lab : 0;
  const bf16* h = hidden + (int64_t)row * ldh;
  const bf16* w = weight + idx * ldw;
  float acc = 0.f;
  for (int k = lane * 8; k < H; k += 64 * 8) {
    float a[8], b[8];
    load_n<bf16, 8>(h + k, a);
    load_n<bf16, 8>(w + k, b);
#pragma unroll
    for (int q = 0; q < 8; ++q) acc += a[q] * b[q];
  }
  acc = wave_sum(acc) + (bias ? to_f32(bias[idx]) : 0.f);
  if (lane == 0) {
    zy[row] = inrange ? acc : 0.f;
    shift[row] = acc + kShiftMargin;
  }
}

// One wave per row of a chunk: merges the row's partials (fixed order) into
// M = max z and S = sum exp(z - c), then, for a row in the window (or, in
// the RECOMPUTE pass, any row of a flagged tile):
//   lse = c + log S, the loss term (lse - z_y for a valid label in range, 0
//   for ignore_index, NaN for a label out of range), the row factor
//   alpha = [label != ignore] / (max(n_valid, 1) S) (so that alpha e =
//   softmax * mask / #valid), the label entry rewritten as e' = exp(z_y - c)
//   - S (alpha e' = (p_y - 1) * mask / #valid, from the fp32 label logit),
//   and the scaled hidden row Hs = alpha h (bf16; the dW product's operand).
// A row outside the window (first pass) flags its tile and takes c = M.
template <bool RECOMPUTE>
__global__ __launch_bounds__(256) void finalize_kernel(
    const float* __restrict__ pmax, const float* __restrict__ psum, int nblk,
    float* __restrict__ shift, const float* __restrict__ zy, const int64_t* __restrict__ labels,
    int64_t ignore, int M, int64_t V, const float* __restrict__ n_valid, bf16* __restrict__ E,
    int64_t ldE, const bf16* __restrict__ hidden, int64_t ldh, int H, bf16* __restrict__ Hs,
    float* __restrict__ alpha, int* __restrict__ tile_flags, float* __restrict__ lse,
    float* __restrict__ loss_row, float* __restrict__ valid_row) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  if (RECOMPUTE && tile_flags[row >> 8] == 0) return;
  const float* pm = pmax + (int64_t)row * nblk;
  const float* ps = psum + (int64_t)row * nblk;
  float mx = -INFINITY, s = 0.f;
  for (int b0 = 4 * lane; b0 < nblk; b0 += 256) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (b0 + u < nblk) {
        mx = fmaxf(mx, pm[b0 + u]);
        s += ps[b0 + u];
      }
    }
  }
  mx = wave_max(mx);
  s = wave_sum(s);
  const float c = shift[row];
  const float lS = logf(s);  // NaN / -inf / +inf fail the window test
  if (!RECOMPUTE && !(lS >= kLogSMin && lS <= kLogSMax)) {
    if (lane == 0) {
      tile_flags[row >> 8] = 1;
      shift[row] = mx;
    }
    return;
  }
  const int64_t lab = labels[row];
  const bool valid = lab != ignore;
  const bool inrange = lab >= 0 && lab < V;
  const float sc = valid ? 1.0f / fmaxf(n_valid[0], 1.0f) : 0.f;
  const float a = sc / s;
  if (lane == 0) {
    const float L = c + lS;
    lse[row] = L;
    loss_row[row] = valid ? (inrange ? L - zy[row] : NAN) : 0.f;
    valid_row[row] = valid ? 1.f : 0.f;
    alpha[row] = a;
    if (valid && inrange) E[(int64_t)row * ldE + lab] = from_f32<bf16>(exp_f(zy[row] - c) - s);
  }
  const bf16* h = hidden + (int64_t)row * ldh;
  bf16* hs = Hs + (int64_t)row * H;
  for (int k = lane * 8; k < H; k += 64 * 8) {
    float x[8];
    load_n<bf16, 8>(h + k, x);
#pragma unroll
    for (int q = 0; q < 8; ++q) x[q] *= a;
    store_n<bf16, 8>(hs + k, x);
  }
}

// x *= g[0] for bf16 or fp32 arrays (skipped as a whole when g[0] == 1).
// The vector loop needs x 16-byte aligned (the caller checks).
template <typename T>
__global__ __launch_bounds__(256) void scale_kernel(T* __restrict__ x, int64_t n,
                                                    const float* __restrict__ g) {
  constexpr int V = 16 / sizeof(T);
  const float s = g[0];
  if (s == 1.0f) return;
  const int64_t nv = n / V;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nv; i += (int64_t)gridDim.x * 256) {
    float v[V];
    load_n_nt<T, V>(x + i * V, v);
#pragma unroll
    for (int k = 0; k < V; ++k) v[k] *= s;
    store_n_nt<T, V>(x + i * V, v);
  }
  for (int64_t i = nv * V + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256)
    x[i] = from_f32<T>(to_f32(x[i]) * s);
}

// One wave per row: merge the row's partials into lse and its loss term.
// One pass, each lane folding four partials per step into a running
// (max, sum exp(. - max)); empty partials (s = 0: columns past V) are skipped.
__global__ __launch_bounds__(256) void lse_reduce_kernel(
    const float* __restrict__ pmax, const float* __restrict__ psum, int nblk,
    const float* __restrict__ zy, const int64_t* __restrict__ labels, int64_t ignore, int M,
    int64_t V, float* __restrict__ lse, float* __restrict__ loss_row, float* __restrict__ valid_row) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const float* pm = pmax + (int64_t)row * nblk;
  const float* ps = psum + (int64_t)row * nblk;
  float mx = -INFINITY, s = 0.f;
  for (int b0 = 4 * lane; b0 < nblk; b0 += 256) {
    float m4[4], s4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const bool ok = b0 + u < nblk;
      m4[u] = ok ? pm[b0 + u] : -INFINITY;
      s4[u] = ok ? ps[b0 + u] : 0.f;
    }
    float mn = mx;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (s4[u] > 0.f) mn = fmaxf(mn, m4[u]);
    if (mn == -INFINITY) continue;
    float t = s > 0.f ? s * expf(mx - mn) : 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (s4[u] > 0.f) t += s4[u] * expf(m4[u] - mn);
    mx = mn;
    s = t;
  }
  const float M_ = wave_max(mx);
  s = wave_sum(s > 0.f ? s * expf(mx - M_) : 0.f);
  if (lane == 0) {
    const float L = M_ + logf(s);
    const int64_t lab = labels[row];
    const bool valid = lab != ignore;
    const bool inrange = lab >= 0 && lab < V;
    lse[row] = L;
    // an out-of-range label (not ignore_index) poisons the loss with NaN
    loss_row[row] = valid ? (inrange ? L - zy[row] : NAN) : 0.f;
    valid_row[row] = valid ? 1.f : 0.f;
  }
}

// Fixed-order mean over valid tokens (one block).
__global__ __launch_bounds__(1024) void loss_mean_kernel(const float* __restrict__ loss_row,
                                                         const float* __restrict__ valid_row, int M,
                                                         float* __restrict__ loss,
                                                         float* __restrict__ n_valid) {
  __shared__ float sl[16], sv[16];
  float a = 0.f, c = 0.f;
  for (int i = threadIdx.x; i < M; i += 1024) {
    a += loss_row[i];
    c += valid_row[i];
  }
  a = wave_sum(a);
  c = wave_sum(c);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sl[w] = a;
    sv[w] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float ta = 0.f, tc = 0.f;
    for (int i = 0; i < 16; ++i) {
      ta += sl[i];
      tc += sv[i];
    }
    loss[0] = ta / fmaxf(tc, 1.0f);
    n_valid[0] = tc;
  }
}

// ----------------------------------------------------------- backward epi --
// d = (exp(z - lse) - [col == label]) * mask * (grad / n_valid), to bf16
// (staged epilogue, 16-byte stores).
template <typename TB>
struct EpiDlogit {
  const TB* bias;  // chunk-relative (bias + c0) or null
  const int64_t* labels;
  int64_t ignore;
  const float* lse;
  const float* grad;     // [1] d loss
  const float* n_valid;  // [1]
  bf16* D;
  int64_t ldd;
  int M, C;
  int64_t c0;

  __device__ __forceinline__ void operator()(f32x4_t (&acc)[big::TM][big::TN], int m0, int n0,
                                             int lane, char* lds, int) const {
    const int c = lane & 15;
    const float scale = grad[0] / fmaxf(n_valid[0], 1.0f);
    float bj[big::TN];
#pragma unroll
    for (int j = 0; j < big::TN; ++j) {
      const int n = n0 + 16 * j + c;
      bj[j] = n < C ? bias_at(bias, n) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < big::TM; ++i) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + 16 * i + 4 * (lane >> 4) + v;
        const int64_t lab = m < M ? labels[m] : ignore;
        const float sc = lab != ignore ? scale : 0.f;
        const float L = m < M ? lse[m] : 0.f;
#pragma unroll
        for (int j = 0; j < big::TN; ++j) {
          const int n = n0 + 16 * j + c;
          float p = exp_f((acc[i][j][v] + bj[j]) - L);
          if (c0 + n == lab) p -= 1.0f;
          acc[i][j][v] = p * sc;
        }
      }
    }
    constexpr int B = 2;  // stores only
    stage_rows_bf16<B>(
        lds, lane, m0, n0, [&](int i, int j, int v) { return acc[i][j][v]; },
        [&](const int (&m)[B], const int (&n)[B], const float (&x)[B][8]) {
#pragma unroll
          for (int q = 0; q < B; ++q)
            if (m[q] < M && n[q] < C) store_row8_bf16(D + (int64_t)m[q] * ldd + n[q], n[q], C, x[q]);
        });
  }
};

__global__ __launch_bounds__(256) void cast_f32_bf16_kernel(const float* __restrict__ src,
                                                            bf16* __restrict__ dst, int64_t n) {
  const int64_t nv = n / 4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nv; i += (int64_t)gridDim.x * 256) {
    float v[4];
    load_n<float, 4>(src + i * 4, v);
    store_n<bf16, 4>(dst + i * 4, v);
  }
  for (int64_t i = nv * 4 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256)
    dst[i] = from_f32<bf16>(src[i]);
}

__global__ __launch_bounds__(256) void zero_bf16_kernel(bf16* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    p[i] = from_f32<bf16>(0.f);
}

__global__ __launch_bounds__(256) void zero_f32_kernel(float* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    p[i] = 0.f;
}

__global__ void empty_loss_kernel(float* loss, float* n_valid) {
  loss[0] = 0.f;
  n_valid[0] = 0.f;
}

// ----------------------------------------------- fp32 (vocabulary chunks) --
// The fp32 form follows the reference's own schedule
// (ops/fused_linear_cross_entropy.py:39-80): per vocabulary chunk an fp32
// logits tile [N, C] from the fp32 matrix-core GEMM, reduced per row to a
// (max, sum exp) partial that lse_reduce_kernel merges; then, per chunk
// again, the logits recomputed and turned into dlogits in place, dH += D W_c
// and dW_c = D^T H. Every value is fp32; the logits tile is the reference's
// [N, chunk] fp32 chunk.

// pmax / psum [row * nblk + blk] = (max_j z, sum_j exp(z - max)) over the C
// logits of row `row` (z = Z + bias). One wave per row.
template <typename TB>
__global__ __launch_bounds__(256) void chunk_partials_f32_kernel(
    const float* __restrict__ Z, int64_t ldz, int rows, int C, const TB* __restrict__ bias,
    float* __restrict__ pmax, float* __restrict__ psum, int nblk, int blk) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* z = Z + (int64_t)row * ldz;
  float mx = -INFINITY;
  for (int j = lane; j < C; j += 64) mx = fmaxf(mx, z[j] + (bias ? to_f32(bias[j]) : 0.f));
  mx = wave_max(mx);
  float sm = 0.f;
  for (int j = lane; j < C; j += 64) sm += expf((z[j] + (bias ? to_f32(bias[j]) : 0.f)) - mx);
  sm = wave_sum(sm);
  if (lane == 0) {
    pmax[(int64_t)row * nblk + blk] = mx;
    psum[(int64_t)row * nblk + blk] = sm;
  }
}

// zy[t] = h_t . W[label_t] (+ b[label_t]) in fp32 for a label in [0, V),
// else 0; any H. One wave per token.
template <typename TB>
__global__ __launch_bounds__(256) void label_logit_f32_kernel(
    const float* __restrict__ hidden, int64_t ldh, const float* __restrict__ weight, int64_t ldw,
    const TB* __restrict__ bias, const int64_t* __restrict__ labels, int M, int64_t V, int H,
    float* __restrict__ zy) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int64_t lab = labels[row];
  if (lab < 0 || lab >= V) {
    if (lane == 0) zy[row] = 0.f;
    return;
  }
  const float* h = hidden + (int64_t)row * ldh;
  const float* w = weight + lab * ldw;
  float acc = 0.f;
  for (int k = lane; k < H; k += 64) acc += h[k] * w[k];
  acc = wave_sum(acc);
  if (lane == 0) zy[row] = acc + (bias ? to_f32(bias[lab]) : 0.f);
}

// In place over the fp32 logits tile of columns c0 .. c0 + C - 1:
// d = (exp(z + b - lse) - [c0 + j == label]) * [label != ignore] / max(n_valid, 1)
// (the reference's softmax minus one-hot with its mask and 1 / #valid scale,
// :67-76, for grad_output = 1). One block of 256 per row and column segment.
template <typename TB>
__global__ __launch_bounds__(256) void chunk_dlogit_f32_kernel(
    float* __restrict__ Z, int64_t ldz, int rows, int C, int64_t c0, const TB* __restrict__ bias,
    const float* __restrict__ lse, const int64_t* __restrict__ labels, int64_t ignore,
    const float* __restrict__ n_valid) {
  const int row = blockIdx.y;
  if (row >= rows) return;
  const int64_t lab = labels[row];
  const float scale = lab != ignore ? 1.0f / fmaxf(n_valid[0], 1.0f) : 0.f;
  const float L = lse[row];
  float* z = Z + (int64_t)row * ldz;
  for (int j = blockIdx.x * 256 + threadIdx.x; j < C; j += gridDim.x * 256) {
    float p = expf((z[j] + (bias ? to_f32(bias[j]) : 0.f)) - L);
    if (c0 + j == lab) p -= 1.0f;
    z[j] = p * scale;
  }
}

// -------------------------------------------------------------- host side --
struct FwdWs {
  float *pmax, *psum, *zy, *loss_row, *valid_row;
};

int64_t nblocks(int64_t V) { return (V + kColBlock - 1) / kColBlock; }

size_t fwd_ws_bytes(int64_t M, int64_t V) {
  return (size_t)(M * (2 * nblocks(V) + 3)) * sizeof(float);
}

size_t bwd_ws_bytes(int64_t M, int64_t H, int64_t chunk, bool need_dh) {
  const size_t d = (size_t)(M * chunk) * 2;
  const size_t d_al = (d + 255) / 256 * 256;
  return d_al + (need_dh ? (size_t)(M * H) * 4 : 0);
}

int check_common(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                 const int64_t* labels, int64_t M, int64_t V, int64_t H, int bias_dtype) {
  ML_CHECK(M >= 0 && V > 0 && H > 0, "flce: bad sizes tokens=%lld vocab=%lld hidden=%lld",
           (long long)M, (long long)V, (long long)H);
  ML_CHECK(M < (1LL << 31) && V < (1LL << 31), "flce: sizes too large");
  ML_CHECK(H % 8 == 0, "flce: hidden size must be a multiple of 8 (got %lld)", (long long)H);
  ML_CHECK(V % 8 == 0, "flce: vocab size must be a multiple of 8 (got %lld)", (long long)V);
  ML_CHECK(M == 0 || (hidden && labels), "flce: null hidden / labels");
  ML_CHECK(weight, "flce: null weight");
  ML_CHECK(ldh >= H && ldw >= H, "flce: leading dimension smaller than hidden size");
  ML_CHECK(bias_dtype == ML_F32 || bias_dtype == ML_BF16, "flce: bias dtype must be fp32 or bf16");
  return ML_OK;
}

template <typename TB>
int fwd_impl(const bf16* hidden, int64_t ldh, const bf16* weight, int64_t ldw, const TB* bias,
             const int64_t* labels, int M, int V, int H, int64_t ignore, float* loss, float* lse,
             float* n_valid, char* ws, hipStream_t st) {
  const int nblk = (int)nblocks(V);
  FwdWs w;
  w.pmax = reinterpret_cast<float*>(ws);
  w.psum = w.pmax + (int64_t)M * nblk;
  w.zy = w.psum + (int64_t)M * nblk;
  w.loss_row = w.zy + M;
  w.valid_row = w.loss_row + M;

  Segment seg{{hidden, ldh}, {weight, ldw}, H};
  Problem pb;
  int rc = make_problem<R4Cfg>(pb, M, V, 1, &seg, kKMajor, kKMajor, 0);
  if (rc) return rc;
  EpiRowLse<TB> epi{bias, w.pmax, w.psum, M, V, nblk};
  gemm_kernel<R4Cfg, kKMajor, kKMajor, EpiRowLse<TB>>
      <<<dim3(grid_blocks(pb)), R4Cfg::THREADS, 0, st>>>(pb, epi);
  ML_LAUNCH_CHECK();
  label_logit_kernel<TB><<<dim3((M + 3) / 4), 256, 0, st>>>(hidden, ldh, weight, ldw, bias, labels,
                                                            M, V, H, w.zy);
  ML_LAUNCH_CHECK();
  lse_reduce_kernel<<<dim3((M + 3) / 4), 256, 0, st>>>(w.pmax, w.psum, nblk, w.zy, labels, ignore,
                                                       M, V, lse, w.loss_row, w.valid_row);
  ML_LAUNCH_CHECK();
  loss_mean_kernel<<<1, 1024, 0, st>>>(w.loss_row, w.valid_row, M, loss, n_valid);
  ML_LAUNCH_CHECK();
  return ML_OK;
}

// ------------------------------------------ loss + gradients in one pass --
// Split count of the dH product (K = the vocabulary) over its 256 x 256
// tiles. One workgroup per CU runs at a time, so a launch takes
// ceil(tiles * ks / CUs) rounds of items 1 / ks of K long, and every split
// writes (then the reduction reads) fp32 partials of the chunk's dH. The
// count minimises the estimated time of both (ties to fewer splits):
//   rounds * V / ks * (us per vocabulary column of a 256 x 256 item at
//   ~1.2 PFLOP/s over 256 CUs) + ks * T * H * (8 B at ~6 TB/s).
// (A fixed target of work items left 264 items at 2736-token chunks: a
// second round of 8 items as long as the first, +34% on the product.)
constexpr int kDhCUs = 256;                             // MI355X
constexpr double kDhUsPerColumn = 2.0 * 65536 / 4.6875e6;  // us
constexpr double kDhUsPerPartial = 8.0 / 6.0e6;             // us per token x hidden
constexpr int kDhMaxSplit = 64;

int dh_ksplit(int T, int H, int V) {
  const int tiles = ((T + 255) / 256) * ((H + 255) / 256);
  const int k64 = (V + kBK - 1) / kBK;
  const int kmax = std::min(k64, kDhMaxSplit);
  int best = 1;
  double best_cost = 0.0;
  for (int ks = 1; ks <= kmax; ++ks) {
    const int64_t rounds = ((int64_t)tiles * ks + kDhCUs - 1) / kDhCUs;
    const double cost = (double)rounds * V / ks * kDhUsPerColumn +
                        (double)ks * T * H * kDhUsPerPartial;
    if (ks == 1 || cost < best_cost) {
      best = ks;
      best_cost = cost;
    }
  }
  return best;
}

// dH split-K partial bytes for a chunk of Tc tokens.
size_t dh_part_bytes(int64_t Tc, int64_t H, int64_t V) {
  const int ks = dh_ksplit((int)Tc, (int)H, (int)V);
  const int k64 = (int)((V + kBK - 1) / kBK);
  const int kps = (k64 + ks - 1) / ks;
  const int splits = (k64 + kps - 1) / kps;
  return (size_t)splits * Tc * H * 4;
}

struct GradWs {
  bf16* E;                           // [T, V]
  float *pmax, *psum;                // [T, nblk]
  float *zy, *loss_row, *valid_row;  // [N]
  float *shift, *alpha;              // [T]
  bf16* Hs;                          // [T, H]: alpha-scaled hidden rows
  int* tile_flags;                   // [ceil(T / 256)]
  float* part;                       // dH split-K partials
  size_t part_bytes;
};

int n_tile_flags(int64_t T) { return (int)((T + 255) / 256); }

// Workspace layout (base == nullptr: size only). T = tokens per chunk.
size_t grad_ws_layout(int64_t N, int64_t V, int64_t H, int64_t T, bool need_dh, GradWs* w,
                      char* base) {
  auto al = [](size_t b) { return (b + 255) / 256 * 256; };
  const int64_t nblk = nblocks(V);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += al(bytes);
    return p;
  };
  char* e = take((size_t)(T * V) * 2);
  char* pm = take((size_t)(T * nblk) * 4);
  char* ps = take((size_t)(T * nblk) * 4);
  char* zy = take((size_t)N * 4);
  char* lr = take((size_t)N * 4);
  char* vr = take((size_t)N * 4);
  char* sh = take((size_t)T * 4);
  char* al_ = take((size_t)T * 4);
  char* hs = take((size_t)(T * H) * 2);
  char* fl = take((size_t)n_tile_flags(T) * 4);
  size_t part = 0;
  if (need_dh) {
    part = dh_part_bytes(T, H, V);
    if (N % T) part = std::max(part, dh_part_bytes(N % T, H, V));
  }
  char* pt = take(part);
  if (w) {
    w->E = reinterpret_cast<bf16*>(e);
    w->pmax = reinterpret_cast<float*>(pm);
    w->psum = reinterpret_cast<float*>(ps);
    w->zy = reinterpret_cast<float*>(zy);
    w->loss_row = reinterpret_cast<float*>(lr);
    w->valid_row = reinterpret_cast<float*>(vr);
    w->shift = reinterpret_cast<float*>(sh);
    w->alpha = reinterpret_cast<float*>(al_);
    w->Hs = reinterpret_cast<bf16*>(hs);
    w->tile_flags = reinterpret_cast<int*>(fl);
    w->part = reinterpret_cast<float*>(pt);
    w->part_bytes = part;
  }
  return off;
}

template <typename TB>
int fwd_grad_impl(const bf16* hidden, int64_t ldh, const bf16* weight, int64_t ldw, const TB* bias,
                  const int64_t* labels, int N, int V, int H, int64_t ignore, int T, float* loss,
                  float* lse, float* n_valid, bf16* d_hidden, bf16* d_weight, char* ws,
                  hipStream_t st) {
  GradWs w;
  grad_ws_layout(N, V, H, T, d_hidden != nullptr, &w, ws);
  const int nblk = (int)nblocks(V);                                // loss only: 64 columns
  const int nsb = (int)((V + kShiftBlock - 1) / kShiftBlock);       // one pass: 128 columns
  const bool grads = d_hidden || d_weight;
  count_valid_kernel<<<1, 1024, 0, st>>>(labels, N, ignore, n_valid);
  ML_LAUNCH_CHECK();
  int rc;
  for (int t0 = 0; t0 < N; t0 += T) {
    const int Tc = N - t0 < T ? N - t0 : T;
    const bf16* hc = hidden + (int64_t)t0 * ldh;
    const int64_t* lc = labels + t0;
    const unsigned row_blocks = (unsigned)((Tc + 3) / 4);
    Segment seg{{hc, ldh}, {weight, ldw}, H};
    Problem pb;
    rc = make_problem<R4Cfg>(pb, Tc, V, 1, &seg, kKMajor, kKMajor, 0);
    if (rc) return rc;
    if (!grads) {  // loss only: (max, sum) partials, nothing stored
      EpiRowLse<TB> epi{bias, w.pmax, w.psum, Tc, V, nblk};
      gemm_kernel<R4Cfg, kKMajor, kKMajor, EpiRowLse<TB>>
          <<<dim3(grid_blocks(pb)), R4Cfg::THREADS, 0, st>>>(pb, epi);
      ML_LAUNCH_CHECK();
      label_logit_kernel<TB><<<row_blocks, 256, 0, st>>>(hc, ldh, weight, ldw, bias, lc, Tc, V, H,
                                                         w.zy + t0);
      ML_LAUNCH_CHECK();
      lse_reduce_kernel<<<row_blocks, 256, 0, st>>>(w.pmax, w.psum, nblk, w.zy + t0, lc, ignore,
                                                    Tc, V, lse + t0, w.loss_row + t0,
                                                    w.valid_row + t0);
      ML_LAUNCH_CHECK();
      continue;
    }
    // 1. row shifts (label logits) and cleared tile flags
    shift_kernel<TB><<<row_blocks, 256, 0, st>>>(hc, ldh, weight, ldw, bias, lc, Tc, V, H,
                                                 w.zy + t0, w.shift, w.tile_flags,
                                                 n_tile_flags(Tc));
    ML_LAUNCH_CHECK();
    // 2. logits, e = exp(z - c) in bf16, (max, sum e) partials (r4 engine),
    // 3. lse, loss terms, row factors, label entries, scaled hidden rows;
    // then the same two steps again for the row tiles a row flagged (their
    // blocks alone do work; for the others the launches return at once)
    for (int pass = 0; pass < 2; ++pass) {
      EpiShiftExp<TB> epi{bias, w.shift, pass ? w.tile_flags : nullptr, w.pmax, w.psum, w.E,
                          (int64_t)V, Tc, V, nsb};
      gemm_kernel<R4Cfg, kKMajor, kKMajor, EpiShiftExp<TB>>
          <<<dim3(grid_blocks(pb)), R4Cfg::THREADS, 0, st>>>(pb, epi);
      ML_LAUNCH_CHECK();
      if (pass == 0)
        finalize_kernel<false><<<row_blocks, 256, 0, st>>>(
            w.pmax, w.psum, nsb, w.shift, w.zy + t0, lc, ignore, Tc, V, n_valid, w.E, V, hc, ldh,
            H, w.Hs, w.alpha, w.tile_flags, lse + t0, w.loss_row + t0, w.valid_row + t0);
      else
        finalize_kernel<true><<<row_blocks, 256, 0, st>>>(
            w.pmax, w.psum, nsb, w.shift, w.zy + t0, lc, ignore, Tc, V, n_valid, w.E, V, hc, ldh,
            H, w.Hs, w.alpha, w.tile_flags, lse + t0, w.loss_row + t0, w.valid_row + t0);
      ML_LAUNCH_CHECK();
    }
    if (d_hidden) {  // 4. dH_c = diag(alpha) (E' W) (split-K over the vocabulary)
      Segment sd{{w.E, (int64_t)V}, {weight, ldw}, V};
      Problem pd;
      rc = make_problem<R4Cfg>(pd, Tc, H, 1, &sd, kKMajor, kMNMajor, 0, dh_ksplit(Tc, H, V));
      if (rc) return rc;
      ML_CHECK(splitk_ws_bytes(pd) <= w.part_bytes, "flce: dH partial workspace too small");
      rc = launch_splitk<R4Cfg, kKMajor, kMNMajor, bf16>(pd, w.part, d_hidden + (int64_t)t0 * H,
                                                          H, 1.0f, 0.0f, st, w.alpha);
      if (rc) return rc;
    }
    if (d_weight) {  // 5. dW (+)= E'^T (diag(alpha) H_c)
      Segment sw{{w.E, (int64_t)V}, {w.Hs, (int64_t)H}, Tc};
      Problem pw;
      rc = make_problem<BigCfg>(pw, V, H, 1, &sw, kMNMajor, kMNMajor, 0);
      if (rc) return rc;
      rc = launch_store<bf16>(pw, kMNMajor, kMNMajor, d_weight, H, 1.0f, t0 > 0 ? 1.0f : 0.0f, st);
      if (rc) return rc;
    }
  }
  loss_mean_kernel<<<1, 1024, 0, st>>>(w.loss_row, w.valid_row, N, loss, n_valid);
  ML_LAUNCH_CHECK();
  return ML_OK;
}

template <typename TB>
int bwd_impl(const bf16* hidden, int64_t ldh, const bf16* weight, int64_t ldw, const TB* bias,
             const int64_t* labels, int M, int V, int H, int64_t ignore, const float* lse,
             const float* n_valid, const float* grad, int chunk, bf16* d_hidden, bf16* d_weight,
             char* ws, hipStream_t st) {
  bf16* D = reinterpret_cast<bf16*>(ws);
  const size_t d_bytes = ((size_t)M * chunk * 2 + 255) / 256 * 256;
  float* dh32 = d_hidden ? reinterpret_cast<float*>(ws + d_bytes) : nullptr;
  for (int c0 = 0; c0 < V; c0 += chunk) {
    const int C = V - c0 < chunk ? V - c0 : chunk;
    const bf16* wc = weight + (int64_t)c0 * ldw;
    {  // 1. dlogits of this chunk
      Segment seg{{hidden, ldh}, {wc, ldw}, H};
      Problem pb;
      int rc = make_problem<BigCfg>(pb, M, C, 1, &seg, kKMajor, kKMajor, 0);
      if (rc) return rc;
      EpiDlogit<TB> epi{bias ? bias + c0 : nullptr, labels, ignore, lse, grad, n_valid, D,
                        (int64_t)chunk, M, C, (int64_t)c0};
      gemm_kernel<BigCfg, kKMajor, kKMajor, EpiDlogit<TB>>
          <<<dim3(grid_blocks(pb)), BigCfg::THREADS, 0, st>>>(pb, epi);
      ML_LAUNCH_CHECK();
    }
    if (dh32) {  // 2. dH (+)= D W_c
      Segment seg{{D, (int64_t)chunk}, {wc, ldw}, C};
      Problem pb;
      int rc = make_problem<BigCfg>(pb, M, H, 1, &seg, kKMajor, kMNMajor, 0);
      if (rc) return rc;
      rc = launch_store<float>(pb, kKMajor, kMNMajor, dh32, H, 1.0f, c0 > 0 ? 1.0f : 0.0f, st);
      if (rc) return rc;
    }
    if (d_weight) {  // 3. dW_c = D^T H
      Segment seg{{D, (int64_t)chunk}, {hidden, ldh}, M};
      Problem pb;
      int rc = make_problem<BigCfg>(pb, C, H, 1, &seg, kMNMajor, kMNMajor, 0);
      if (rc) return rc;
      rc = launch_store<bf16>(pb, kMNMajor, kMNMajor, d_weight + (int64_t)c0 * H, H, 1.0f, 0.0f,
                              st);
      if (rc) return rc;
    }
  }
  if (dh32) {
    const int64_t n = (int64_t)M * H;
    int64_t blocks = (n / 4 + 255) / 256;
    blocks = blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096;
    cast_f32_bf16_kernel<<<dim3((unsigned)blocks), 256, 0, st>>>(dh32, d_hidden, n);
    ML_LAUNCH_CHECK();
  }
  return ML_OK;
}

// fp32 workspace: the logits tile [N, chunk], partials [N, nblk] x 2, zy,
// loss_row, valid_row [N].
size_t f32_ws_layout(int64_t N, int64_t V, int64_t chunk, float** Z, float** pm, float** ps,
                     float** zy, float** lr, float** vr, char* base) {
  auto al = [](size_t b) { return (b + 255) / 256 * 256; };
  const int64_t nblk = (V + chunk - 1) / chunk;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += al(bytes);
    return reinterpret_cast<float*>(p);
  };
  float* z = take((size_t)(N * chunk) * 4);
  float* a = take((size_t)(N * nblk) * 4);
  float* b = take((size_t)(N * nblk) * 4);
  float* c = take((size_t)N * 4);
  float* d = take((size_t)N * 4);
  float* e = take((size_t)N * 4);
  if (Z) {
    *Z = z;
    *pm = a;
    *ps = b;
    *zy = c;
    *lr = d;
    *vr = e;
  }
  return off;
}

template <typename TB>
int fwd_grad_f32_impl(const float* hidden, int64_t ldh, const float* weight, int64_t ldw,
                      const TB* bias, const int64_t* labels, int N, int V, int H, int64_t ignore,
                      int chunk, float* loss, float* lse, float* n_valid, float* d_hidden,
                      float* d_weight, char* ws, hipStream_t st) {
  float *Z, *pm, *ps, *zy, *lr, *vr;
  f32_ws_layout(N, V, chunk, &Z, &pm, &ps, &zy, &lr, &vr, ws);
  const int nblk = (V + chunk - 1) / chunk;
  const unsigned row_blocks = (unsigned)((N + 3) / 4);
  count_valid_kernel<<<1, 1024, 0, st>>>(labels, N, ignore, n_valid);
  ML_LAUNCH_CHECK();
  auto logits = [&](int c0, int C) -> int {
    const int64_t kl = H;
    const void* a = hidden;
    const void* b = weight + (int64_t)c0 * ldw;
    return ml_gemm_f32_segments(N, C, 1, &kl, &a, &ldh, &b, &ldw, kKMajor, kKMajor, Z, chunk,
                                1.0f, 0.0f, st);
  };
  for (int blk = 0, c0 = 0; c0 < V; ++blk, c0 += chunk) {  // pass 1: partials
    const int C = V - c0 < chunk ? V - c0 : chunk;
    int rc = logits(c0, C);
    if (rc) return rc;
    chunk_partials_f32_kernel<TB><<<row_blocks, 256, 0, st>>>(Z, chunk, N, C,
                                                              bias ? bias + c0 : nullptr, pm, ps,
                                                              nblk, blk);
    ML_LAUNCH_CHECK();
  }
  label_logit_f32_kernel<TB><<<row_blocks, 256, 0, st>>>(hidden, ldh, weight, ldw, bias, labels, N,
                                                         V, H, zy);
  ML_LAUNCH_CHECK();
  lse_reduce_kernel<<<row_blocks, 256, 0, st>>>(pm, ps, nblk, zy, labels, ignore, N, V, lse, lr,
                                                 vr);
  ML_LAUNCH_CHECK();
  loss_mean_kernel<<<1, 1024, 0, st>>>(lr, vr, N, loss, n_valid);
  ML_LAUNCH_CHECK();
  if (!d_hidden && !d_weight) return ML_OK;
  for (int c0 = 0; c0 < V; c0 += chunk) {  // pass 2: gradients
    const int C = V - c0 < chunk ? V - c0 : chunk;
    int rc = logits(c0, C);
    if (rc) return rc;
    const unsigned segs = (unsigned)std::min<int64_t>((C + 255) / 256, 16);
    chunk_dlogit_f32_kernel<TB><<<dim3(segs, (unsigned)N), 256, 0, st>>>(
        Z, chunk, N, C, c0, bias ? bias + c0 : nullptr, lse, labels, ignore, n_valid);
    ML_LAUNCH_CHECK();
    const float* wc = weight + (int64_t)c0 * ldw;
    if (d_hidden) {  // dH (+)= D W_c
      const int64_t kl = C;
      const void* a = Z;
      const int64_t lda = chunk;
      const void* b = wc;
      rc = ml_gemm_f32_segments(N, H, 1, &kl, &a, &lda, &b, &ldw, kKMajor, kMNMajor, d_hidden, H,
                                1.0f, c0 > 0 ? 1.0f : 0.0f, st);
      if (rc) return rc;
    }
    if (d_weight) {  // dW_c = D^T H
      const int64_t kl = N;
      const void* a = Z;
      const int64_t lda = chunk;
      const void* b = hidden;
      rc = ml_gemm_f32_segments(C, H, 1, &kl, &a, &lda, &b, &ldh, kMNMajor, kMNMajor,
                                d_weight + (int64_t)c0 * H, H, 1.0f, 0.0f, st);
      if (rc) return rc;
    }
  }
  return ML_OK;
}

}  // namespace
}  // namespace flce
}  // namespace mla

using namespace mla;

extern "C" size_t ml_flce_fwd_grad_f32_workspace_bytes(int64_t n_tokens, int64_t vocab,
                                                      int64_t chunk) {
  if (n_tokens <= 0 || vocab <= 0 || chunk <= 0) return 0;
  return flce::f32_ws_layout(n_tokens, vocab, chunk, nullptr, nullptr, nullptr, nullptr, nullptr,
                             nullptr, nullptr);
}

extern "C" int ml_flce_fwd_grad_f32(const float* hidden, int64_t ldh, const float* weight,
                                    int64_t ldw, const float* bias, const int64_t* labels,
                                    int64_t n_tokens, int64_t vocab, int64_t hidden_size,
                                    int64_t ignore_index, int64_t chunk, float* loss, float* lse,
                                    float* n_valid, float* d_hidden, float* d_weight,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  ML_CHECK(n_tokens >= 0 && vocab > 0 && hidden_size > 0 && chunk > 0,
           "flce f32: bad sizes tokens=%lld vocab=%lld hidden=%lld chunk=%lld",
           (long long)n_tokens, (long long)vocab, (long long)hidden_size, (long long)chunk);
  ML_CHECK(n_tokens < (1LL << 31) && vocab < (1LL << 31) && hidden_size < (1LL << 31),
           "flce f32: sizes too large");
  ML_CHECK(n_tokens == 0 || (hidden && labels), "flce f32: null hidden / labels");
  ML_CHECK(weight && loss && n_valid, "flce f32: null weight / loss / n_valid");
  ML_CHECK(n_tokens == 0 || lse, "flce f32: null lse");
  ML_CHECK(ldh >= hidden_size && ldw >= hidden_size, "flce f32: leading dimension < hidden size");
  hipStream_t st = (hipStream_t)stream;
  if (n_tokens == 0) {
    flce::empty_loss_kernel<<<1, 1, 0, st>>>(loss, n_valid);
    ML_LAUNCH_CHECK();
    // an empty sum: zero gradients for the weight (dH is empty); a fill
    // kernel rather than a memset node, so the call can be graph-captured
    if (d_weight) {
      const int64_t n = vocab * hidden_size;
      int64_t blocks = (n + 255) / 256;
      blocks = blocks < 4096 ? blocks : 4096;
      flce::zero_f32_kernel<<<dim3((unsigned)blocks), 256, 0, st>>>(d_weight, n);
      ML_LAUNCH_CHECK();
    }
    return ML_OK;
  }
  const int64_t c = chunk < vocab ? chunk : vocab;
  const size_t need = ml_flce_fwd_grad_f32_workspace_bytes(n_tokens, vocab, c);
  ML_CHECK(workspace && workspace_bytes >= need, "flce f32: workspace too small (%zu < %zu)",
           workspace_bytes, need);
  return flce::fwd_grad_f32_impl<float>(hidden, ldh, weight, ldw, bias, labels, (int)n_tokens,
                                        (int)vocab, (int)hidden_size, ignore_index, (int)c, loss,
                                        lse, n_valid, d_hidden, d_weight,
                                        static_cast<char*>(workspace), st);
}

extern "C" int ml_flce_scale_grads_f32(const float* grad_loss, float* d_hidden, int64_t n_hidden,
                                       float* d_weight, int64_t n_weight, void* stream) {
  ML_CHECK(grad_loss, "flce: null grad_loss");
  ML_CHECK(n_hidden >= 0 && n_weight >= 0, "flce: negative sizes");
  ML_CHECK((n_hidden == 0 || d_hidden) && (n_weight == 0 || d_weight), "flce: null gradient");
  ML_CHECK((n_hidden == 0 || aligned16(d_hidden)) && (n_weight == 0 || aligned16(d_weight)),
           "flce: gradients must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  float* ptrs[2] = {d_hidden, d_weight};
  const int64_t ns[2] = {n_hidden, n_weight};
  for (int i = 0; i < 2; ++i) {
    if (ns[i] == 0) continue;
    int64_t blocks = (ns[i] / 4 + 255) / 256;
    blocks = blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096;
    flce::scale_kernel<float><<<dim3((unsigned)blocks), 256, 0, st>>>(ptrs[i], ns[i], grad_loss);
    ML_LAUNCH_CHECK();
  }
  return ML_OK;
}

extern "C" size_t ml_flce_fwd_workspace_bytes(int64_t n_tokens, int64_t vocab) {
  if (n_tokens <= 0 || vocab <= 0) return 0;
  return flce::fwd_ws_bytes(n_tokens, vocab);
}

extern "C" int ml_flce_fwd(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                           const void* bias, int bias_dtype, const int64_t* labels,
                           int64_t n_tokens, int64_t vocab, int64_t hidden_size,
                           int64_t ignore_index, float* loss, float* lse, float* n_valid,
                           void* workspace, size_t workspace_bytes, void* stream) {
  int rc = flce::check_common(hidden, ldh, weight, ldw, labels, n_tokens, vocab, hidden_size,
                              bias_dtype);
  if (rc) return rc;
  ML_CHECK(loss && n_valid && (n_tokens == 0 || lse), "flce: null output pointer");
  hipStream_t st = (hipStream_t)stream;
  if (n_tokens == 0) {
    flce::empty_loss_kernel<<<1, 1, 0, st>>>(loss, n_valid);
    ML_LAUNCH_CHECK();
    return ML_OK;
  }
  ML_CHECK(workspace && workspace_bytes >= flce::fwd_ws_bytes(n_tokens, vocab),
           "flce: forward workspace too small (%zu < %zu bytes)", workspace_bytes,
           flce::fwd_ws_bytes(n_tokens, vocab));
  const bf16* h = static_cast<const bf16*>(hidden);
  const bf16* w = static_cast<const bf16*>(weight);
  char* ws = static_cast<char*>(workspace);
  if (bias_dtype == ML_BF16)
    return flce::fwd_impl<bf16>(h, ldh, w, ldw, static_cast<const bf16*>(bias), labels,
                                (int)n_tokens, (int)vocab, (int)hidden_size, ignore_index, loss,
                                lse, n_valid, ws, st);
  return flce::fwd_impl<float>(h, ldh, w, ldw, static_cast<const float*>(bias), labels,
                               (int)n_tokens, (int)vocab, (int)hidden_size, ignore_index, loss, lse,
                               n_valid, ws, st);
}

extern "C" size_t ml_flce_bwd_workspace_bytes(int64_t n_tokens, int64_t hidden_size, int64_t chunk,
                                              int need_dhidden) {
  if (n_tokens <= 0 || hidden_size <= 0 || chunk <= 0) return 0;
  return flce::bwd_ws_bytes(n_tokens, hidden_size, chunk, need_dhidden != 0);
}

extern "C" int ml_flce_bwd(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                           const void* bias, int bias_dtype, const int64_t* labels,
                           int64_t n_tokens, int64_t vocab, int64_t hidden_size,
                           int64_t ignore_index, const float* lse, const float* n_valid,
                           const float* grad_loss, int64_t chunk, void* d_hidden, void* d_weight,
                           void* workspace, size_t workspace_bytes, void* stream) {
  int rc = flce::check_common(hidden, ldh, weight, ldw, labels, n_tokens, vocab, hidden_size,
                              bias_dtype);
  if (rc) return rc;
  ML_CHECK(chunk > 0 && chunk % 8 == 0 && chunk < (1LL << 31),
           "flce: chunk size must be a positive multiple of 8 (got %lld)", (long long)chunk);
  ML_CHECK((!d_hidden || aligned16(d_hidden)) && (!d_weight || aligned16(d_weight)),
           "flce: gradients must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  const int64_t H = hidden_size;
  if (n_tokens == 0) {
    // no tokens: dW is zero; dH is empty
    if (d_weight) {
      flce::zero_bf16_kernel<<<1024, 256, 0, st>>>(static_cast<bf16*>(d_weight), vocab * H);
      ML_LAUNCH_CHECK();
    }
    return ML_OK;
  }
  ML_CHECK(lse && n_valid && grad_loss, "flce: null saved tensors / grad");
  const size_t need = flce::bwd_ws_bytes(n_tokens, H, chunk, d_hidden != nullptr);
  ML_CHECK(workspace && workspace_bytes >= need, "flce: backward workspace too small (%zu < %zu)",
           workspace_bytes, need);
  if (!d_hidden && !d_weight) return ML_OK;
  const bf16* h = static_cast<const bf16*>(hidden);
  const bf16* w = static_cast<const bf16*>(weight);
  char* ws = static_cast<char*>(workspace);
  if (bias_dtype == ML_BF16)
    return flce::bwd_impl<bf16>(h, ldh, w, ldw, static_cast<const bf16*>(bias), labels,
                                (int)n_tokens, (int)vocab, (int)H, ignore_index, lse, n_valid,
                                grad_loss, (int)chunk, static_cast<bf16*>(d_hidden),
                                static_cast<bf16*>(d_weight), ws, st);
  return flce::bwd_impl<float>(h, ldh, w, ldw, static_cast<const float*>(bias), labels,
                               (int)n_tokens, (int)vocab, (int)H, ignore_index, lse, n_valid,
                               grad_loss, (int)chunk, static_cast<bf16*>(d_hidden),
                               static_cast<bf16*>(d_weight), ws, st);
}

extern "C" size_t ml_flce_fwd_grad_workspace_bytes(int64_t n_tokens, int64_t vocab,
                                                   int64_t hidden_size, int64_t token_chunk,
                                                   int need_dhidden) {
  if (n_tokens <= 0 || vocab <= 0 || hidden_size <= 0 || token_chunk <= 0) return 0;
  const int64_t T = token_chunk < n_tokens ? token_chunk : n_tokens;
  return flce::grad_ws_layout(n_tokens, vocab, hidden_size, T, need_dhidden != 0, nullptr, nullptr);
}

extern "C" int ml_flce_fwd_grad(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                                const void* bias, int bias_dtype, const int64_t* labels,
                                int64_t n_tokens, int64_t vocab, int64_t hidden_size,
                                int64_t ignore_index, int64_t token_chunk, float* loss, float* lse,
                                float* n_valid, void* d_hidden, void* d_weight, void* workspace,
                                size_t workspace_bytes, void* stream) {
  int rc = flce::check_common(hidden, ldh, weight, ldw, labels, n_tokens, vocab, hidden_size,
                              bias_dtype);
  if (rc) return rc;
  ML_CHECK(loss && n_valid && (n_tokens == 0 || lse), "flce: null output pointer");
  // dW is written as 16-byte row vectors; dH is scaled as 16-byte vectors later
  ML_CHECK((!d_hidden || aligned16(d_hidden)) && (!d_weight || aligned16(d_weight)),
           "flce: gradients must be 16-byte aligned");
  ML_CHECK(token_chunk > 0 && token_chunk < (1LL << 31), "flce: token_chunk must be positive");
  hipStream_t st = (hipStream_t)stream;
  const int64_t H = hidden_size;
  if (n_tokens == 0) {
    flce::empty_loss_kernel<<<1, 1, 0, st>>>(loss, n_valid);
    ML_LAUNCH_CHECK();
    if (d_weight) {
      flce::zero_bf16_kernel<<<1024, 256, 0, st>>>(static_cast<bf16*>(d_weight), vocab * H);
      ML_LAUNCH_CHECK();
    }
    return ML_OK;
  }
  const int64_t T = token_chunk < n_tokens ? token_chunk : n_tokens;
  ML_CHECK(T * vocab < (1LL << 40), "flce: token_chunk * vocab too large");
  const size_t need = ml_flce_fwd_grad_workspace_bytes(n_tokens, vocab, H, T, d_hidden != nullptr);
  ML_CHECK(workspace && workspace_bytes >= need, "flce: workspace too small (%zu < %zu bytes)",
           workspace_bytes, need);
  const bf16* h = static_cast<const bf16*>(hidden);
  const bf16* w = static_cast<const bf16*>(weight);
  char* ws = static_cast<char*>(workspace);
  if (bias_dtype == ML_BF16)
    return flce::fwd_grad_impl<bf16>(h, ldh, w, ldw, static_cast<const bf16*>(bias), labels,
                                     (int)n_tokens, (int)vocab, (int)H, ignore_index, (int)T, loss,
                                     lse, n_valid, static_cast<bf16*>(d_hidden),
                                     static_cast<bf16*>(d_weight), ws, st);
  return flce::fwd_grad_impl<float>(h, ldh, w, ldw, static_cast<const float*>(bias), labels,
                                    (int)n_tokens, (int)vocab, (int)H, ignore_index, (int)T, loss,
                                    lse, n_valid, static_cast<bf16*>(d_hidden),
                                    static_cast<bf16*>(d_weight), ws, st);
}

extern "C" int ml_flce_scale_grads(const float* grad_loss, void* d_hidden, int64_t n_hidden,
                                   void* d_weight, int64_t n_weight, void* stream) {
  ML_CHECK(grad_loss, "flce: null grad_loss");
  ML_CHECK(n_hidden >= 0 && n_weight >= 0, "flce: negative sizes");
  ML_CHECK((n_hidden == 0 || d_hidden) && (n_weight == 0 || d_weight), "flce: null gradient");
  ML_CHECK((n_hidden == 0 || aligned16(d_hidden)) && (n_weight == 0 || aligned16(d_weight)),
           "flce: gradients must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  void* ptrs[2] = {d_hidden, d_weight};
  const int64_t ns[2] = {n_hidden, n_weight};
  for (int i = 0; i < 2; ++i) {
    if (ns[i] == 0) continue;
    int64_t blocks = (ns[i] / 8 + 255) / 256;
    blocks = blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096;
    flce::scale_kernel<bf16><<<dim3((unsigned)blocks), 256, 0, st>>>(static_cast<bf16*>(ptrs[i]),
                                                                    ns[i], grad_loss);
    ML_LAUNCH_CHECK();
  }
  return ML_OK;
}

// RMSNorm forward / backward for gfx950.
//
// Math follows ops/fused_rms_norm.py:31-60 (fp32 accumulation, rrms saved
// in fp32, closed-form VJP). Layout and parallelisation are MI355X-native:
//
//  * fast path: one wave64 per row, the whole row held in registers. Lane l
//    owns 16-byte chunks l, l+64, l+128, ... so every load/store instruction
//    of a wave touches 1 KiB of contiguous HBM. Sum of squares and the
//    backward dot product are wave reductions (no LDS, no barrier).
//  * dW: each backward block accumulates its rows' g*(x*r) in registers
//    (lane-owned columns), folds its waves together through LDS in a fixed
//    tree order and writes one fp32 partial row; a second kernel sums the
//    partial rows in fixed order. No atomics, bit-reproducible run to run.
//  * generic path (any width, stride or alignment): one 256-thread block per
//    row with scalar accesses.
//  * residual form (Qwen3's `h = residual + attn_out; post_attention_layernorm(h)`):
//    the forward reads x and the residual, stores s = x + residual rounded
//    to x's dtype (what the separate add produces) and normalises that s;
//    the backward adds the gradient the sum receives from the residual
//    branch into dx before its one rounding. One pass each instead of an
//    add kernel plus a norm kernel (forward) and a norm kernel plus an add
//    (backward).
#include <initializer_list>

#include <mutex>

#include "common.h"

// Evaluate every product and sum exactly as written (one rounding each), as
// the reference's op-by-op torch evaluation does.
#pragma clang fp contract(off)

namespace mla {
namespace {

constexpr int kFwdWaves = 4;        // rows per forward block (one wave per row)
constexpr int kBwdWaves = 8;        // waves per backward block
constexpr int kMaxBwdBlocks = 256;  // dW partial rows (one 8-wave block per CU)
constexpr int kGenericThreads = 256;

// Column of chunk `it` for `lane`, clamped to the last valid chunk of the row.
__device__ __forceinline__ int clamp_col(int it, int lane, int cols, int vec) {
  const int c = (it * 64 + lane) * vec;
  return c < cols ? c : cols - vec;
}

__device__ __forceinline__ float block_sum_256(float v, float* red /* [4] */) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // red may still be read by a previous call
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// ------------------------------------------------------------ fast forward
// ADD: x <- round(x + res) first (stored to sum), as the residual form does.
template <typename TX, typename TW, int ITERS, bool ADD>
__global__ __launch_bounds__(64 * kFwdWaves) void rms_fwd_reg(
    const TX* __restrict__ x, int64_t ldx, const TX* __restrict__ res, int64_t ldr,
    TX* __restrict__ sum, int64_t lds, const TW* __restrict__ w, TX* __restrict__ y, int64_t ldy,
    float* __restrict__ rrms, int64_t rows, int cols, float eps) {
  constexpr int VEC = vec16<TX>();
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kFwdWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const TX* xr = x + row * ldx;

  // Chunks past the row end load the last valid chunk (no branch around the
  // load, so all ITERS loads are in flight together) and are zeroed after.
  float v[ITERS][VEC];
#pragma unroll
  for (int it = 0; it < ITERS; ++it) load_n_nt<TX, VEC>(xr + clamp_col(it, lane, cols, VEC), v[it]);
  if constexpr (ADD) {
    const TX* rr = res + row * ldr;
    float rv[ITERS][VEC];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) load_n_nt<TX, VEC>(rr + clamp_col(it, lane, cols, VEC), rv[it]);
    TX* sr = sum + row * lds;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[it][e] = to_f32(from_f32<TX>(v[it][e] + rv[it][e]));
      const int c = (it * 64 + lane) * VEC;
      if (c < cols) store_n_nt<TX, VEC>(sr + c, v[it]);
    }
  }
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    if ((it * 64 + lane) * VEC >= cols) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[it][e] = 0.f;
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int it = 0; it < ITERS; ++it)
#pragma unroll
    for (int e = 0; e < VEC; ++e) ss += v[it][e] * v[it][e];
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)cols + eps);
  if (rrms != nullptr && lane == 0) rrms[row] = r;

  TX* yr = y + row * ldy;
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int c = (it * 64 + lane) * VEC;
    if (c < cols) {
      float wv[VEC], o[VEC];
      load_n<TW, VEC>(w + c, wv);
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = (v[it][e] * r) * wv[e];
      store_n_nt<TX, VEC>(yr + c, o);
    }
  }
}

// --------------------------------------------------------- generic forward
// res == nullptr: plain norm of x. Otherwise each thread stores
// round(x + res) for its columns and normalises that.
template <typename TX, typename TW>
__global__ __launch_bounds__(kGenericThreads) void rms_fwd_generic(
    const TX* __restrict__ x, int64_t ldx, const TX* __restrict__ res, int64_t ldr,
    TX* __restrict__ sum, int64_t lds, const TW* __restrict__ w, TX* __restrict__ y, int64_t ldy,
    float* __restrict__ rrms, int64_t rows, int64_t cols, float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const TX* xr = x + row * ldx;
  const TX* rr = res == nullptr ? nullptr : res + row * ldr;
  TX* sr = res == nullptr ? nullptr : sum + row * lds;
  auto value = [&](int64_t c) -> float {
    return rr == nullptr ? to_f32(xr[c]) : to_f32(from_f32<TX>(to_f32(xr[c]) + to_f32(rr[c])));
  };
  float ss = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kGenericThreads) {
    const float xv = value(c);
    if (sr != nullptr) sr[c] = from_f32<TX>(xv);
    ss += xv * xv;
  }
  ss = block_sum_256(ss, red);
  const float r = 1.0f / sqrtf(ss / (float)cols + eps);
  if (rrms != nullptr && threadIdx.x == 0) rrms[row] = r;
  TX* yr = y + row * ldy;
  for (int64_t c = threadIdx.x; c < cols; c += kGenericThreads)
    yr[c] = from_f32<TX>((value(c) * r) * to_f32(w[c]));
}

// ------------------------------------------------------------ fast backward
// HAS_DRES: dx += dres (the residual form's second gradient) before rounding.
template <typename TX, typename TW, int ITERS, bool HAS_RRMS, bool HAS_DRES>
__global__ __launch_bounds__(64 * kBwdWaves) void rms_bwd_reg(
    const TX* __restrict__ x, int64_t ldx, const TW* __restrict__ w, const TX* __restrict__ dy,
    int64_t lddy, const TX* __restrict__ dres, int64_t ldd, const float* __restrict__ rrms,
    float eps, TX* __restrict__ dx, int64_t lddx, float* __restrict__ partial, int64_t rows,
    int cols) {
  constexpr int VEC = vec16<TX>();
  extern __shared__ float smem[];  // [kBwdWaves/2][cols]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  // w stays in registers when the row is short; wider rows re-read it from
  // L1 each row (it is shared by every wave of the CU) to avoid spills.
  constexpr bool W_IN_REGS = ITERS * VEC <= 32;
  float wv[W_IN_REGS ? ITERS : 1][VEC], acc[ITERS][VEC];
  auto load_w = [&](int it, float* dst) {
    load_n<TW, VEC>(w + clamp_col(it, lane, cols, VEC), dst);
    if ((it * 64 + lane) * VEC >= cols) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) dst[e] = 0.f;
    }
  };
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    if constexpr (W_IN_REGS) load_w(it, wv[it]);
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[it][e] = 0.f;
  }

  const float inv_cols = 1.0f / (float)cols;
  for (int64_t row = (int64_t)blockIdx.x * kBwdWaves + wave; row < rows;
       row += (int64_t)gridDim.x * kBwdWaves) {
    const TX* xr = x + row * ldx;
    const TX* gr = dy + row * lddy;
    float xv[ITERS][VEC], gv[ITERS][VEC], dv[HAS_DRES ? ITERS : 1][VEC];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int c = clamp_col(it, lane, cols, VEC);
      load_n_nt<TX, VEC>(xr + c, xv[it]);
      load_n_nt<TX, VEC>(gr + c, gv[it]);
      // (the tail chunk reads the last valid chunk; its result is not stored)
      if constexpr (HAS_DRES) load_n_nt<TX, VEC>(dres + row * ldd + c, dv[it]);
    }
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      if ((it * 64 + lane) * VEC >= cols) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) xv[it][e] = gv[it][e] = 0.f;
      }
    }
    float r;
    if constexpr (HAS_RRMS) {
      r = rrms[row];
    } else {
      float ss = 0.f;
#pragma unroll
      for (int it = 0; it < ITERS; ++it)
#pragma unroll
        for (int e = 0; e < VEC; ++e) ss += xv[it][e] * xv[it][e];
      ss = wave_sum(ss);
      r = 1.0f / sqrtf(ss * inv_cols + eps);
    }
    // gv becomes g * w in place (the reference's gw)
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      float wt[VEC];
      if constexpr (!W_IN_REGS) load_w(it, wt);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float wc = W_IN_REGS ? wv[W_IN_REGS ? it : 0][e] : wt[e];
        acc[it][e] += gv[it][e] * (xv[it][e] * r);
        gv[it][e] = gv[it][e] * wc;
      }
    }
    float dot = 0.f;
#pragma unroll
    for (int it = 0; it < ITERS; ++it)
#pragma unroll
      for (int e = 0; e < VEC; ++e) dot += gv[it][e] * xv[it][e];
    dot = wave_sum(dot);
    const float mean = dot / (float)cols;
    const float r3 = (r * r) * r;

    TX* dxr = dx + row * lddx;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int c = (it * 64 + lane) * VEC;
      float o[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = gv[it][e] * r - (xv[it][e] * mean) * r3;
      if constexpr (HAS_DRES) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[e] = o[e] + dv[HAS_DRES ? it : 0][e];
      }
      if (c < cols) store_n_nt<TX, VEC>(dxr + c, o);
    }
  }

  // Fold the waves' dW partials: fixed binary tree through LDS.
#pragma unroll
  for (int half = kBwdWaves / 2; half >= 1; half >>= 1) {
    if (wave >= half && wave < 2 * half) {
      float* dst = smem + (int64_t)(wave - half) * cols;
#pragma unroll
      for (int it = 0; it < ITERS; ++it) {
        const int c = (it * 64 + lane) * VEC;
        if (c < cols) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) dst[c + e] = acc[it][e];
        }
      }
    }
    __syncthreads();
    if (wave < half) {
      const float* src = smem + (int64_t)wave * cols;
#pragma unroll
      for (int it = 0; it < ITERS; ++it) {
        const int c = (it * 64 + lane) * VEC;
        if (c < cols) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[it][e] += src[c + e];
        }
      }
    }
    __syncthreads();
  }
  if (wave == 0) {
    float* pr = partial + (int64_t)blockIdx.x * cols;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int c = (it * 64 + lane) * VEC;
      if (c < cols) store_n<float, VEC>(pr + c, acc[it]);
    }
  }
}

// --------------------------------------------------------- generic backward
// Block b handles rows b, b+G, ...; thread t owns columns t, t+256, ... of
// partial row b (so no two threads touch the same partial element).
template <typename TX, typename TW, bool HAS_RRMS>
__global__ __launch_bounds__(kGenericThreads) void rms_bwd_generic(
    const TX* __restrict__ x, int64_t ldx, const TW* __restrict__ w, const TX* __restrict__ dy,
    int64_t lddy, const TX* __restrict__ dres, int64_t ldd, const float* __restrict__ rrms,
    float eps, TX* __restrict__ dx, int64_t lddx, float* __restrict__ partial, int64_t rows,
    int64_t cols) {
  __shared__ float red[4];
  float* pr = partial + (int64_t)blockIdx.x * cols;
  for (int64_t c = threadIdx.x; c < cols; c += kGenericThreads) pr[c] = 0.f;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const TX* xr = x + row * ldx;
    const TX* gr = dy + row * lddy;
    float ss = 0.f, dot = 0.f;
    for (int64_t c = threadIdx.x; c < cols; c += kGenericThreads) {
      const float xv = to_f32(xr[c]);
      ss += xv * xv;
      dot += (to_f32(gr[c]) * to_f32(w[c])) * xv;
    }
    float r;
    if constexpr (HAS_RRMS) {
      r = rrms[row];
    } else {
      ss = block_sum_256(ss, red);
      r = 1.0f / sqrtf(ss / (float)cols + eps);
    }
    dot = block_sum_256(dot, red);
    const float mean = dot / (float)cols;
    const float r3 = (r * r) * r;
    TX* dxr = dx + row * lddx;
    for (int64_t c = threadIdx.x; c < cols; c += kGenericThreads) {
      const float xv = to_f32(xr[c]);
      const float gv = to_f32(gr[c]);
      float o = (gv * to_f32(w[c])) * r - (xv * mean) * r3;
      if (dres != nullptr) o = o + to_f32(dres[row * ldd + c]);
      dxr[c] = from_f32<TX>(o);
      pr[c] += gv * (xv * r);
    }
  }
}

// Sums G partial rows in a fixed order.
// Wave form (cols % 4 == 0, G <= 256): one wave per 4-column vector, lane l
// summing partial rows l, l + 64, ... (16-byte loads, all in flight
// together), then a fixed-order wave reduction. No LDS and no barrier: the
// reduction is one L2 round trip.
constexpr int kRedWaveRows = 4;  // partial rows per lane (G <= 64 * kRedWaveRows)

template <typename TW>
__global__ __launch_bounds__(256) void rms_dw_reduce_wave(const float* __restrict__ partial, int G,
                                                           int64_t cols, TW* __restrict__ dw) {
  const int lane = threadIdx.x & 63;
  const int64_t c = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4;
  if (c >= cols) return;
  float v[kRedWaveRows][4];
#pragma unroll
  for (int i = 0; i < kRedWaveRows; ++i) {
    const int g = lane + 64 * i;
    if (g < G) {
      load_n<float, 4>(partial + (int64_t)g * cols + c, v[i]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[i][e] = 0.f;
    }
  }
  float o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float t = (v[0][e] + v[1][e]) + (v[2][e] + v[3][e]);
    o[e] = wave_sum(t);
  }
  if (lane == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) dw[c + e] = from_f32<TW>(o[e]);
  }
}

// Scalar form (any cols): 32 columns x 8 row slices per block.
template <typename TW>
__global__ __launch_bounds__(256) void rms_dw_reduce(const float* __restrict__ partial, int G,
                                                      int64_t cols, TW* __restrict__ dw) {
  __shared__ float sm[8][33];
  const int cl = threadIdx.x & 31;
  const int sl = threadIdx.x >> 5;
  const int64_t c = (int64_t)blockIdx.x * 32 + cl;
  float s = 0.f;
  if (c < cols)
    for (int g = sl; g < G; g += 8) s += partial[(int64_t)g * cols + c];
  sm[sl][cl] = s;
  __syncthreads();
  if (sl == 0 && c < cols) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) t += sm[i][cl];
    dw[c] = from_f32<TW>(t);
  }
}

// Register-path capacity: ITERS chunks of 16 bytes per lane. The backward
// holds three row-sized arrays per lane, so it stops at 32 values per array.
template <typename TX>
int pick_iters(int64_t cols, bool backward) {
  const int64_t per = 64 * vec16<TX>();
  const int max_it = backward ? 32 / vec16<TX>() : 8;
  for (int it : {1, 2, 4, 8})
    if (it <= max_it && cols <= per * it) return it;
  return 0;
}

// A row operand: base pointer and row stride in elements (ptr may be null:
// an absent optional operand).
struct RowOp {
  const void* ptr;
  int64_t ld;
};

template <typename TX, typename TW>
bool fast_path_ok(bool backward, const void* w, int64_t cols, std::initializer_list<RowOp> ops) {
  constexpr int VEC = vec16<TX>();
  if (cols % VEC != 0 || pick_iters<TX>(cols, backward) == 0) return false;
  if (!aligned16(w)) return false;
  for (const RowOp& o : ops)
    if (o.ptr != nullptr && (!aligned16(o.ptr) || (o.ld * (int64_t)sizeof(TX)) % 16 != 0))
      return false;
  return true;
}

// res / sum: the residual form (both given) or the plain norm (both null).
template <typename TX, typename TW>
int launch_fwd(const void* x, int64_t ldx, const void* res, int64_t ldr, void* sum, int64_t lds,
               const void* w, void* y, int64_t ldy, float* rrms, int64_t rows, int64_t cols,
               float eps, hipStream_t st) {
  if (rows == 0) return ML_OK;
  const TX* xp = static_cast<const TX*>(x);
  const TX* rp = static_cast<const TX*>(res);
  TX* sp = static_cast<TX*>(sum);
  const TW* wp = static_cast<const TW*>(w);
  TX* yp = static_cast<TX*>(y);
  if (fast_path_ok<TX, TW>(false, w, cols, {{x, ldx}, {y, ldy}, {res, ldr}, {sum, lds}})) {
    const dim3 grid((unsigned)((rows + kFwdWaves - 1) / kFwdWaves));
    const int it = pick_iters<TX>(cols, false);
#define ML_FWD(I, A)                                                                         \
  rms_fwd_reg<TX, TW, I, A><<<grid, 64 * kFwdWaves, 0, st>>>(xp, ldx, rp, ldr, sp, lds, wp, yp, \
                                                             ldy, rrms, rows, (int)cols, eps)
#define ML_FWD_A(I)  \
  if (rp) {          \
    ML_FWD(I, true); \
  } else {           \
    ML_FWD(I, false); \
  }
    switch (it) {
      case 1: ML_FWD_A(1); break;
      case 2: ML_FWD_A(2); break;
      case 4: ML_FWD_A(4); break;
      default: ML_FWD_A(8); break;
    }
#undef ML_FWD_A
#undef ML_FWD
  } else {
    ML_CHECK(rows <= 0x7fffffffLL, "rmsnorm: too many rows for the generic path (%lld)",
             (long long)rows);
    rms_fwd_generic<TX, TW><<<dim3((unsigned)rows), kGenericThreads, 0, st>>>(
        xp, ldx, rp, ldr, sp, lds, wp, yp, ldy, rrms, rows, cols, eps);
  }
  ML_LAUNCH_CHECK();
  return ML_OK;
}

int64_t bwd_blocks_fast(int64_t rows) {
  const int64_t b = (rows + kBwdWaves - 1) / kBwdWaves;
  return b < kMaxBwdBlocks ? b : kMaxBwdBlocks;
}
int64_t bwd_blocks_generic(int64_t rows) { return rows < kMaxBwdBlocks ? rows : kMaxBwdBlocks; }

// dres: the residual form's second gradient of the sum (null: plain norm).
template <typename TX, typename TW>
int launch_bwd(const void* x, int64_t ldx, const void* w, const void* dy, int64_t lddy,
               const void* dres, int64_t ldd, const float* rrms, float eps, void* dx,
               int64_t lddx, void* dw, void* ws, size_t ws_bytes, int64_t rows, int64_t cols,
               hipStream_t st) {
  const TX* xp = static_cast<const TX*>(x);
  const TW* wp = static_cast<const TW*>(w);
  const TX* gp = static_cast<const TX*>(dy);
  const TX* dp = static_cast<const TX*>(dres);
  TX* dxp = static_cast<TX*>(dx);
  TW* dwp = static_cast<TW*>(dw);
  float* part = static_cast<float*>(ws);
  const int64_t lds_bytes = (int64_t)(kBwdWaves / 2) * cols * (int64_t)sizeof(float);
  const bool fast =
      fast_path_ok<TX, TW>(true, w, cols, {{x, ldx}, {dx, lddx}, {dy, lddy}, {dres, ldd}}) &&
      lds_bytes <= 64 * 1024;
  const int64_t G = rows == 0 ? 0 : (fast ? bwd_blocks_fast(rows) : bwd_blocks_generic(rows));
  ML_CHECK(ws_bytes >= (size_t)(G * cols * (int64_t)sizeof(float)),
           "rmsnorm backward: workspace too small (%zu < %lld bytes)", ws_bytes,
           (long long)(G * cols * (int64_t)sizeof(float)));
  if (G > 0) {
    if (fast) {
      const int it = pick_iters<TX>(cols, true);
#define ML_BWD(I, R, D)                                                                           \
  rms_bwd_reg<TX, TW, I, R, D><<<dim3((unsigned)G), 64 * kBwdWaves, (size_t)lds_bytes, st>>>( \
      xp, ldx, wp, gp, lddy, dp, ldd, rrms, eps, dxp, lddx, part, rows, (int)cols)
#define ML_BWD_R(I)          \
  if (rrms && dp) {          \
    ML_BWD(I, true, true);   \
  } else if (rrms) {         \
    ML_BWD(I, true, false);  \
  } else if (dp) {           \
    ML_BWD(I, false, true);  \
  } else {                   \
    ML_BWD(I, false, false); \
  }
      switch (it) {
        case 1: ML_BWD_R(1); break;
        case 2: ML_BWD_R(2); break;
        case 4: ML_BWD_R(4); break;
        default:
          if constexpr (vec16<TX>() * 8 <= 32) {
            ML_BWD_R(8);
          }
          break;
      }
#undef ML_BWD_R
#undef ML_BWD
    } else {
      if (rrms)
        rms_bwd_generic<TX, TW, true><<<dim3((unsigned)G), kGenericThreads, 0, st>>>(
            xp, ldx, wp, gp, lddy, dp, ldd, rrms, eps, dxp, lddx, part, rows, cols);
      else
        rms_bwd_generic<TX, TW, false><<<dim3((unsigned)G), kGenericThreads, 0, st>>>(
            xp, ldx, wp, gp, lddy, dp, ldd, rrms, eps, dxp, lddx, part, rows, cols);
    }
    ML_LAUNCH_CHECK();
  }
  if (cols > 0) {
    static_assert(kMaxBwdBlocks <= 64 * kRedWaveRows, "wave reduction covers every partial row");
    if (cols % 4 == 0)
      rms_dw_reduce_wave<TW><<<dim3((unsigned)((cols / 4 + 3) / 4)), 256, 0, st>>>(part, (int)G,
                                                                                  cols, dwp);
    else
      rms_dw_reduce<TW><<<dim3((unsigned)((cols + 31) / 32)), 256, 0, st>>>(part, (int)G, cols,
                                                                             dwp);
    ML_LAUNCH_CHECK();
  }
  return ML_OK;
}

// Calls f(TX{}, TW{}) for the supported (x, w) dtype pairs: w either matches
// x or is fp32.
template <typename F>
int dispatch_xw(int x_dtype, int w_dtype, F&& f) {
  return dispatch_dtype(x_dtype, [&](auto tx) -> int {
    using TX = decltype(tx);
    if (w_dtype == ML_F32) return f(tx, float{});
    return dispatch_dtype(w_dtype, [&](auto tw) -> int {
      using TW = decltype(tw);
      if constexpr (std::is_same<TX, TW>::value) {
        return f(tx, tw);
      } else {
        set_error("rmsnorm: weight dtype %d must match x dtype %d or be fp32", w_dtype, x_dtype);
        return ML_ERR_INVALID;
      }
    });
  });
}

}  // namespace
}  // namespace mla

using namespace mla;

extern "C" int ml_rmsnorm_fwd(const void* x, int64_t ldx, const void* w, void* y, int64_t ldy,
                              float* rrms, int64_t rows, int64_t cols, float eps, int x_dtype,
                              int w_dtype, void* stream) {
  ML_CHECK(rows >= 0 && cols > 0, "rmsnorm: bad shape rows=%lld cols=%lld", (long long)rows,
           (long long)cols);
  ML_CHECK(rows == 0 || (x && w && y), "rmsnorm: null pointer");
  ML_CHECK(ldx >= cols && ldy >= cols, "rmsnorm: row stride smaller than cols");
  return dispatch_xw(x_dtype, w_dtype, [&](auto tx, auto tw) -> int {
    return launch_fwd<decltype(tx), decltype(tw)>(x, ldx, nullptr, 0, nullptr, 0, w, y, ldy, rrms,
                                                  rows, cols, eps, (hipStream_t)stream);
  });
}

extern "C" int ml_rmsnorm_add_fwd(const void* x, int64_t ldx, const void* residual, int64_t ldr,
                                  const void* w, void* sum, int64_t lds, void* y, int64_t ldy,
                                  float* rrms, int64_t rows, int64_t cols, float eps, int x_dtype,
                                  int w_dtype, void* stream) {
  ML_CHECK(rows >= 0 && cols > 0, "rmsnorm add: bad shape rows=%lld cols=%lld", (long long)rows,
           (long long)cols);
  ML_CHECK(rows == 0 || (x && residual && w && sum && y), "rmsnorm add: null pointer");
  ML_CHECK(ldx >= cols && ldr >= cols && lds >= cols && ldy >= cols,
           "rmsnorm add: row stride smaller than cols");
  return dispatch_xw(x_dtype, w_dtype, [&](auto tx, auto tw) -> int {
    return launch_fwd<decltype(tx), decltype(tw)>(x, ldx, residual, ldr, sum, lds, w, y, ldy,
                                                  rrms, rows, cols, eps, (hipStream_t)stream);
  });
}

extern "C" size_t ml_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  const int64_t g = bwd_blocks_generic(rows);  // >= the fast path's block count
  return (size_t)(g * cols * (int64_t)sizeof(float));
}

static int rmsnorm_bwd_checked(const void* x, int64_t ldx, const void* w, const void* dy,
                               int64_t lddy, const void* dres, int64_t ldd, const float* rrms,
                               float eps, void* dx, int64_t lddx, void* dw, void* workspace,
                               size_t workspace_bytes, int64_t rows, int64_t cols, int x_dtype,
                               int w_dtype, void* stream) {
  ML_CHECK(rows >= 0 && cols > 0, "rmsnorm backward: bad shape rows=%lld cols=%lld",
           (long long)rows, (long long)cols);
  ML_CHECK(w && dw, "rmsnorm backward: null weight / dw pointer");
  ML_CHECK(rows == 0 || (x && dy && dx && workspace), "rmsnorm backward: null pointer");
  ML_CHECK(ldx >= cols && lddy >= cols && lddx >= cols && (dres == nullptr || ldd >= cols),
           "rmsnorm backward: row stride smaller than cols");
  return dispatch_xw(x_dtype, w_dtype, [&](auto tx, auto tw) -> int {
    return launch_bwd<decltype(tx), decltype(tw)>(x, ldx, w, dy, lddy, dres, ldd, rrms, eps, dx,
                                                  lddx, dw, workspace, workspace_bytes, rows, cols,
                                                  (hipStream_t)stream);
  });
}

extern "C" int ml_rmsnorm_bwd(const void* x, int64_t ldx, const void* w, const void* dy,
                              int64_t lddy, const float* rrms, float eps, void* dx, int64_t lddx,
                              void* dw, void* workspace, size_t workspace_bytes, int64_t rows,
                              int64_t cols, int x_dtype, int w_dtype, void* stream) {
  return rmsnorm_bwd_checked(x, ldx, w, dy, lddy, nullptr, 0, rrms, eps, dx, lddx, dw, workspace,
                             workspace_bytes, rows, cols, x_dtype, w_dtype, stream);
}

// ------------------------------------------------ allocation-free backward --
// ml_rmsnorm_bwd_noalloc keeps the dW partial rows (min(rows, 256) x cols
// fp32) in this file-scope device array instead of a caller workspace. Each
// GPU holds its own copy for the life of the process. The array's name is a
// host-side stand-in: host code uses only the per-device address that
// hipGetSymbolAddress returns (looked up once per device, on the first call
// made with that device current). Every backward block writes its whole
// partial row before the reduction reads it, so the array needs no clearing;
// calls that overlap on one GPU share it and race.
namespace {
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
constexpr int kScratchDevices = 64;
void* g_scratch[kScratchDevices] = {};
hipError_t g_scratch_status[kScratchDevices] = {};
std::once_flag g_scratch_once[kScratchDevices];
}  // namespace

static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

// The current device's address of `scratch`; the stream must belong to
// that device.
static int scratch_address(hipStream_t st, void** out) {
  int dev = 0;
  ML_HIP_CHECK(hipGetDevice(&dev));
  ML_CHECK(dev >= 0 && dev < kScratchDevices, "rmsnorm backward (no-alloc): device %d out of range",
           dev);
  if (st != nullptr) {
    hipDevice_t sdev = 0;
    ML_HIP_CHECK(hipStreamGetDevice(st, &sdev));
    ML_CHECK(sdev == dev,
             "rmsnorm backward (no-alloc): the stream belongs to device %d, the current device is %d",
             (int)sdev, dev);
  }
  std::call_once(g_scratch_once[dev], [dev]() {
    void* p = nullptr;
    g_scratch_status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch[dev] = p;
  });
  if (g_scratch_status[dev] != hipSuccess || g_scratch[dev] == nullptr) {
    set_error("rmsnorm backward (no-alloc): hipGetSymbolAddress failed on device %d: %s", dev,
              hipGetErrorString(g_scratch_status[dev]));
    return ML_ERR_HIP;
  }
  *out = g_scratch[dev];
  return ML_OK;
}

extern "C" int ml_rmsnorm_bwd_noalloc(const void* x, int64_t ldx, const void* w, const void* dy,
                                      int64_t lddy, const float* rrms, float eps, void* dx,
                                      int64_t lddx, void* dw, int64_t rows, int64_t cols,
                                      int x_dtype, int w_dtype, void* stream) {
  ML_CHECK(rows >= 0 && cols > 0, "rmsnorm backward: bad shape rows=%lld cols=%lld",
           (long long)rows, (long long)cols);
  const size_t need = ml_rmsnorm_bwd_workspace_bytes(rows, cols);
  ML_CHECK(need <= kNoAllocScratchBytes,
           "rmsnorm backward (no-alloc): min(rows, 256) x cols x 4 = %zu bytes of dW partials "
           "exceed its %zu-byte scratch (cols <= %zu at 256 or more rows)",
           need, kNoAllocScratchBytes, kNoAllocScratchBytes / (256 * sizeof(float)));
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_address((hipStream_t)stream, &ws);
    if (rc != ML_OK) return rc;
  }
  return rmsnorm_bwd_checked(x, ldx, w, dy, lddy, nullptr, 0, rrms, eps, dx, lddx, dw, ws,
                             kNoAllocScratchBytes, rows, cols, x_dtype, w_dtype, stream);
}

extern "C" int ml_rmsnorm_add_bwd(const void* sum, int64_t lds, const void* w, const void* dy,
                                  int64_t lddy, const void* dsum, int64_t ldd, const float* rrms,
                                  float eps, void* dx, int64_t lddx, void* dw, void* workspace,
                                  size_t workspace_bytes, int64_t rows, int64_t cols, int x_dtype,
                                  int w_dtype, void* stream) {
  ML_CHECK(rows == 0 || dsum, "rmsnorm add backward: null sum gradient");
  return rmsnorm_bwd_checked(sum, lds, w, dy, lddy, dsum, ldd, rrms, eps, dx, lddx, dw, workspace,
                             workspace_bytes, rows, cols, x_dtype, w_dtype, stream);
}

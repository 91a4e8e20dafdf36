// Fused linear cross-entropy for gfx950
// (ops/fused_linear_cross_entropy.py:39-185 of the reference).
//
// Forward: ONE bf16 MFMA GEMM over the whole vocabulary, z = h W^T (+ b).
//   The logits never leave registers: each wave reduces its 128-column slice
//   of the tile to per-row (max, sum exp(z - max)) partials and the lane that
//   holds (row, label) writes the label logit. A row-parallel pass merges the
//   partials into lse (the online-softmax merge of the reference's chunk
//   loop, :39-55) and the masked per-token loss; a fixed-order single-block
//   pass forms the mean over valid tokens (clamped at 1, :149).
// Backward, per vocabulary chunk of `chunk` columns (the reference's
//   chunk_size, :57-80):
//   1. recompute the logits tile and write dlogits in bf16 from the epilogue:
//      d = (exp(z - lse) - [col == label]) * mask * (grad / n_valid)
//   2. dH += D W_c   (fp32 accumulation across chunks; MN-major B operand)
//   3. dW_c = D^T H  (written once per chunk, straight to bf16)
//   Memory beyond inputs/outputs: one [tokens, chunk] bf16 buffer plus an
//   fp32 [tokens, hidden] dH accumulator; the [tokens, vocab] logits never
//   exist. dH / dW are skipped when not requested (frozen lm_head).
#include <math.h>

#include "gemm_core.h"

namespace mla {
namespace flce {
namespace {

using namespace gemm;

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kColBlock = big::WN;  // columns per (max, sum) partial: one wave's sub-tile

__device__ __forceinline__ float exp_f(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

// Reductions over the 16 lanes of a group (the lanes that hold one row of a
// 16 x 16 accumulator tile).
__device__ __forceinline__ float grp16_max(float v) {
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 16));
  return v;
}
__device__ __forceinline__ float grp16_sum(float v) {
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) v += __shfl_xor(v, off, 16);
  return v;
}

template <typename TB>
__device__ __forceinline__ float bias_at(const TB* b, int64_t n) {
  return b ? to_f32(b[n]) : 0.f;
}

// ------------------------------------------------------------ forward epi --
// Each wave reduces its 128 logit columns to a (max, sum exp(z - max))
// partial per row; the lane holding (row, label) writes the label logit.
template <typename TB>
struct EpiLse {
  const TB* bias;
  const int64_t* labels;
  float* pmax;  // [M][nblk]
  float* psum;  // [M][nblk]
  float* zy;    // [M]
  int M, V, nblk;

  __device__ __forceinline__ void operator()(f32x4_t (&acc)[big::TM][big::TN], int m0, int n0,
                                             int lane, char*, int) const {
    // a wave whose 128 columns all lie past the vocabulary (second half of
    // the last tile) owns no partial slot
    if (n0 >= V) return;
    const int c = lane & 15;
    float bj[big::TN];
    bool okj[big::TN];
#pragma unroll
    for (int j = 0; j < big::TN; ++j) {
      const int n = n0 + 16 * j + c;
      okj[j] = n < V;
      bj[j] = okj[j] ? bias_at(bias, n) : 0.f;
    }
    const int nb = n0 / kColBlock;
#pragma unroll
    for (int i = 0; i < big::TM; ++i) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + 16 * i + 4 * (lane >> 4) + v;
        float z[big::TN];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < big::TN; ++j) {
          z[j] = okj[j] ? acc[i][j][v] + bj[j] : -INFINITY;
          mx = fmaxf(mx, z[j]);
        }
        if (m < M) {
          const int64_t lab = labels[m];
#pragma unroll
          for (int j = 0; j < big::TN; ++j)
            if (okj[j] && lab == (int64_t)(n0 + 16 * j + c)) zy[m] = z[j];
        }
        mx = grp16_max(mx);
        float s = 0.f;
        if (mx != -INFINITY) {
#pragma unroll
          for (int j = 0; j < big::TN; ++j) s += exp_f(z[j] - mx);
        }
        s = grp16_sum(s);
        if (c == 0 && m < M) {
          pmax[(int64_t)m * nblk + nb] = mx;
          psum[(int64_t)m * nblk + nb] = s;
        }
      }
    }
  }
};

// One wave per row: merge the row's partials into lse and its loss term.
__global__ __launch_bounds__(256) void lse_reduce_kernel(
    const float* __restrict__ pmax, const float* __restrict__ psum, int nblk,
    const float* __restrict__ zy, const int64_t* __restrict__ labels, int64_t ignore, int M,
    int64_t V, float* __restrict__ lse, float* __restrict__ loss_row, float* __restrict__ valid_row) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const float* pm = pmax + (int64_t)row * nblk;
  const float* ps = psum + (int64_t)row * nblk;
  float mx = -INFINITY;
  for (int b = lane; b < nblk; b += 64)
    if (ps[b] > 0.f) mx = fmaxf(mx, pm[b]);
  mx = wave_max(mx);
  float s = 0.f;
  for (int b = lane; b < nblk; b += 64)
    if (ps[b] > 0.f) s += ps[b] * expf(pm[b] - mx);
  s = wave_sum(s);
  if (lane == 0) {
    const float L = mx + logf(s);
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
// d = (exp(z - lse) - [col == label]) * mask * (grad / n_valid), to bf16.
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
                                             int lane, char*, int) const {
    const int c = lane & 15;
    const float scale = grad[0] / fmaxf(n_valid[0], 1.0f);
    float bj[big::TN];
    bool okj[big::TN];
#pragma unroll
    for (int j = 0; j < big::TN; ++j) {
      const int n = n0 + 16 * j + c;
      okj[j] = n < C;
      bj[j] = okj[j] ? bias_at(bias, n) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < big::TM; ++i) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + 16 * i + 4 * (lane >> 4) + v;
        if (m >= M) continue;
        const int64_t lab = labels[m];
        const float sc = lab != ignore ? scale : 0.f;
        const float L = lse[m];
        bf16* drow = D + (int64_t)m * ldd;
#pragma unroll
        for (int j = 0; j < big::TN; ++j) {
          if (!okj[j]) continue;
          const int n = n0 + 16 * j + c;
          float p = exp_f((acc[i][j][v] + bj[j]) - L);
          if (c0 + n == lab) p -= 1.0f;
          drow[n] = from_f32<bf16>(p * sc);
        }
      }
    }
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

__global__ void empty_loss_kernel(float* loss, float* n_valid) {
  loss[0] = 0.f;
  n_valid[0] = 0.f;
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
  int rc = make_problem<BigCfg>(pb, M, V, 1, &seg, kKMajor, kKMajor, 0);
  if (rc) return rc;
  EpiLse<TB> epi{bias, labels, w.pmax, w.psum, w.zy, M, V, nblk};
  gemm_kernel<BigCfg, kKMajor, kKMajor, EpiLse<TB>><<<dim3(grid_blocks(pb)), kThreads, 0, st>>>(pb, epi);
  ML_LAUNCH_CHECK();
  lse_reduce_kernel<<<dim3((M + 3) / 4), 256, 0, st>>>(w.pmax, w.psum, nblk, w.zy, labels, ignore,
                                                       M, V, lse, w.loss_row, w.valid_row);
  ML_LAUNCH_CHECK();
  loss_mean_kernel<<<1, 1024, 0, st>>>(w.loss_row, w.valid_row, M, loss, n_valid);
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
          <<<dim3(grid_blocks(pb)), kThreads, 0, st>>>(pb, epi);
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

}  // namespace
}  // namespace flce
}  // namespace mla

using namespace mla;

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

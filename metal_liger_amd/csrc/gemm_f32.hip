// fp32 GEMM on the matrix cores (v_mfma_f32_32x32x2_f32, full fp32
// products and sums) for the fp32 forms of the LoRA and fused linear
// cross-entropy ops (the reference runs them in whatever float dtype the
// model has, ops/fused_lora.py:69-82, ops/fused_linear_cross_entropy.py:108):
//
//   C[M, N] = alpha * sum_seg op(A_s) op(B_s) + beta * C      (all fp32)
//
// Operand layouts as in the bf16 engine: K-major element (r, k) at
// p[r * ld + k], MN-major at p[k * ld + r]; K may be a list of up to 8
// segments with their own pointers (K-concatenated operands).
//
// Tiles: 128 x 128 per block of 4 waves (2 x 2), a wave owns 64 x 64 =
// 2 x 2 MFMA tiles of 32 x 32 (64 fp32 accumulators). k-tiles of 16,
// staged global -> registers -> LDS (two stages); LDS holds each operand as
// 16 k-planes of 128 values with a pitch of 132 floats, so both the stores
// (4 consecutive k of a K-major row, or 4 consecutive rows of an MN-major
// k-plane) and the fragment reads (32 consecutive rows of one plane per
// half-wave) are free of bank conflicts. Rows past M / N re-read the last
// row (never stored); k past a segment's end is zero-filled.
#include "common.h"

namespace mla {
namespace gemmf32 {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBN = 128, kBK = 16;
constexpr int kThreads = 256;
constexpr int kPitch = 132;                     // floats per k-plane
constexpr int kOpFloats = kBK * kPitch;         // one operand stage
constexpr int kMaxSeg = 8;
enum : int { kKMajor = 0, kMNMajor = 1 };

struct Seg {
  const float* a;
  const float* b;
  int64_t lda, ldb;
  int k_len;
};

struct Prob {
  int M, N, nseg;
  Seg seg[kMaxSeg];
  float* C;
  int64_t ldc;
  float alpha, beta;
};

// Global -> register load of one operand's k-tile: 2 float4 per thread.
// K-major: thread t covers row (t / 4) + 64 i, k 4 (t % 4) .. + 3.
// MN-major: thread t covers k-plane (t / 32) + 8 i, rows 4 (t % 32) .. + 3.
template <int L>
__device__ __forceinline__ void load_tile(f32x4_t (&v)[2], const float* p, int64_t ld, int row0,
                                          int rows, int k0, int klen) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if constexpr (L == kKMajor) {
      int r = row0 + (t >> 2) + 64 * i;
      r = r < rows ? r : rows - 1;
      const int k = k0 + 4 * (t & 3);
      if (k + 4 <= klen && (reinterpret_cast<uintptr_t>(p + (int64_t)r * ld + k) & 15) == 0) {
        v[i] = *reinterpret_cast<const f32x4_t*>(p + (int64_t)r * ld + k);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[i][e] = (k + e < klen) ? p[(int64_t)r * ld + k + e] : 0.f;
      }
    } else {
      const int k = k0 + (t >> 5) + 8 * i;
      int r = row0 + 4 * (t & 31);
      if (k >= klen) {
        v[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      } else if (r + 4 <= rows && (reinterpret_cast<uintptr_t>(p + (int64_t)k * ld + r) & 15) == 0) {
        v[i] = *reinterpret_cast<const f32x4_t*>(p + (int64_t)k * ld + r);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int rr = r + e < rows ? r + e : rows - 1;
          v[i][e] = p[(int64_t)k * ld + rr];
        }
      }
    }
  }
}

template <int L>
__device__ __forceinline__ void store_tile(const f32x4_t (&v)[2], float* lds) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if constexpr (L == kKMajor) {
      const int r = (t >> 2) + 64 * i;
      const int k = 4 * (t & 3);
#pragma unroll
      for (int e = 0; e < 4; ++e) lds[(k + e) * kPitch + r] = v[i][e];
    } else {
      const int k = (t >> 5) + 8 * i;
      const int r = 4 * (t & 31);
      *reinterpret_cast<f32x4_t*>(lds + k * kPitch + r) = v[i];
    }
  }
}

template <int LA, int LB>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(const Prob pb) {
  __shared__ __attribute__((aligned(16))) float lds[2][2 * kOpFloats];
  const int tiles_m = (pb.M + kBM - 1) / kBM;
  const int tm = blockIdx.x % tiles_m, tn = blockIdx.x / tiles_m;
  const int m0 = tm * kBM, n0 = tn * kBN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  int nk = 0;
  for (int s = 0; s < pb.nseg; ++s) nk += (pb.seg[s].k_len + kBK - 1) / kBK;
  if (nk > 0) {
    int seg = 0, k0 = 0;
    while (pb.seg[seg].k_len == 0) ++seg;
    f32x4_t ra[2], rb[2];
    auto load = [&]() {
      const Seg& sg = pb.seg[seg];
      load_tile<LA>(ra, sg.a, sg.lda, m0, pb.M, k0, sg.k_len);
      load_tile<LB>(rb, sg.b, sg.ldb, n0, pb.N, k0, sg.k_len);
    };
    auto advance = [&]() {
      k0 += kBK;
      if (k0 >= pb.seg[seg].k_len) {
        k0 = 0;
        do {
          ++seg;
        } while (seg < pb.nseg && pb.seg[seg].k_len == 0);
      }
    };
    load();
    store_tile<LA>(ra, lds[0]);
    store_tile<LB>(rb, lds[0] + kOpFloats);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const bool more = kt + 1 < nk;
      if (more) {
        advance();
        load();
      }
      const float* As = lds[kt & 1];
      const float* Bs = As + kOpFloats;
#pragma unroll
      for (int ks = 0; ks < kBK; ks += 2) {
        const int kp = (ks + (lane >> 5)) * kPitch + (lane & 31);
        float a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) a[i] = As[kp + wm + 32 * i];
#pragma unroll
        for (int j = 0; j < 2; ++j) b[j] = Bs[kp + wn + 32 * j];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
      }
      if (more) {
        store_tile<LA>(ra, lds[(kt + 1) & 1]);
        store_tile<LB>(rb, lds[(kt + 1) & 1] + kOpFloats);
      }
      __syncthreads();
    }
  }
  // element v of tile (i, j): row wm + 32 i + 8 (v / 4) + 4 (lane / 32) + v % 4,
  // column wn + 32 j + lane % 32
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn + 32 * j + (lane & 31);
      if (n >= pb.N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (m < pb.M) {
          float* c = pb.C + (int64_t)m * pb.ldc + n;
          float o = pb.alpha * acc[i][j][v];
          if (pb.beta != 0.f) o += pb.beta * *c;
          *c = o;
        }
      }
    }
}

}  // namespace
}  // namespace gemmf32
}  // namespace mla

using namespace mla;

extern "C" int ml_gemm_f32_segments(int64_t M, int64_t N, int nseg, const int64_t* k_lens,
                                    const void* const* a_ptrs, const int64_t* ldas,
                                    const void* const* b_ptrs, const int64_t* ldbs, int a_layout,
                                    int b_layout, float* C, int64_t ldc, float alpha, float beta,
                                    void* stream) {
  using namespace gemmf32;
  ML_CHECK(M > 0 && N > 0 && M < (1LL << 31) && N < (1LL << 31), "gemm f32: bad M=%lld N=%lld",
           (long long)M, (long long)N);
  ML_CHECK(nseg >= 1 && nseg <= kMaxSeg, "gemm f32: 1..%d segments supported (got %d)", kMaxSeg,
           nseg);
  ML_CHECK(k_lens && a_ptrs && ldas && b_ptrs && ldbs, "gemm f32: null segment arrays");
  ML_CHECK(a_layout == kKMajor || a_layout == kMNMajor, "gemm f32: bad A layout %d", a_layout);
  ML_CHECK(b_layout == kKMajor || b_layout == kMNMajor, "gemm f32: bad B layout %d", b_layout);
  ML_CHECK(C != nullptr && ldc >= N, "gemm f32: bad C (ldc %lld < N %lld)", (long long)ldc,
           (long long)N);
  Prob pb{};
  pb.M = (int)M;
  pb.N = (int)N;
  pb.nseg = nseg;
  pb.C = C;
  pb.ldc = ldc;
  pb.alpha = alpha;
  pb.beta = beta;
  for (int s = 0; s < nseg; ++s) {
    ML_CHECK(k_lens[s] >= 0 && k_lens[s] < (1LL << 31), "gemm f32: bad K segment %d", s);
    Seg& g = pb.seg[s];
    g.a = static_cast<const float*>(a_ptrs[s]);
    g.b = static_cast<const float*>(b_ptrs[s]);
    g.lda = ldas[s];
    g.ldb = ldbs[s];
    g.k_len = (int)k_lens[s];
    if (g.k_len == 0) continue;
    ML_CHECK(g.a && g.b, "gemm f32: null operand in segment %d", s);
    ML_CHECK(a_layout == kKMajor ? g.lda >= g.k_len : g.lda >= M,
             "gemm f32: A leading dimension %lld too small in segment %d", (long long)g.lda, s);
    ML_CHECK(b_layout == kKMajor ? g.ldb >= g.k_len : g.ldb >= N,
             "gemm f32: B leading dimension %lld too small in segment %d", (long long)g.ldb, s);
  }
  const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  ML_CHECK(tiles <= 0x7fffffffLL, "gemm f32: too many tiles");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)tiles);
#define ML_GF(LA, LB) gemm_f32_kernel<LA, LB><<<grid, kThreads, 0, st>>>(pb)
  if (a_layout == kKMajor && b_layout == kKMajor) ML_GF(kKMajor, kKMajor);
  else if (a_layout == kKMajor) ML_GF(kKMajor, kMNMajor);
  else if (b_layout == kKMajor) ML_GF(kMNMajor, kKMajor);
  else ML_GF(kMNMajor, kMNMajor);
#undef ML_GF
  ML_LAUNCH_CHECK();
  return ML_OK;
}

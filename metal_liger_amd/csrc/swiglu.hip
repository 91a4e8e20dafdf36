// SwiGLU forward / backward for gfx950 (ops/fused_swiglu.py:26-50).
//
// Pure streaming kernels: 16-byte loads/stores, UNROLL independent 16-byte
// chunks per thread in flight, non-temporal stores, grid of 32-48 blocks per
// CU striding over the tensor (the best of a sweep over unroll 1-8, grid
// 4-64 blocks/CU and load/store cache hints on MI355X: 7.1 TB/s for the
// forward's access pattern, the same as a plain copy). sigmoid(gate) is recomputed in the backward
// (the reference saved it as an extra fp32 tensor, ops/fused_swiglu.py:34;
// recomputing it costs no HBM traffic). All math in fp32, products evaluated
// in the reference's order with one rounding each.
#include "swiglu_math.h"

#pragma clang fp contract(off)

namespace mla {
namespace {

constexpr int kThreads = 256;

// One grid-stride step over UNROLL 16-byte chunks. FULL: every chunk is in
// range, so the loads carry no guard (a guarded load sits in its own branch
// and the compiler waits for it before leaving the branch, serialising the
// chunks).
template <typename T, int UNROLL, bool FULL>
__device__ __forceinline__ void swiglu_fwd_step(const T* __restrict__ g, const T* __restrict__ u,
                                                T* __restrict__ o, int64_t base, int64_t nvec) {
  constexpr int VEC = vec16<T>();
  float gv[UNROLL][VEC], uv[UNROLL][VEC];
#pragma unroll
  for (int k = 0; k < UNROLL; ++k) {
    const int64_t i = base + (int64_t)k * kThreads;
    if (FULL || i < nvec) {
      load_n_nt<T, VEC>(g + i * VEC, gv[k]);
      load_n_nt<T, VEC>(u + i * VEC, uv[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < UNROLL; ++k) {
    const int64_t i = base + (int64_t)k * kThreads;
    if (FULL || i < nvec) {
      float ov[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) ov[e] = swiglu_fwd_elem(gv[k][e], uv[k][e]);
      store_n_nt<T, VEC>(o + i * VEC, ov);
    }
  }
}

template <typename T, int UNROLL>
__global__ __launch_bounds__(kThreads) void swiglu_fwd_vec(const T* __restrict__ g,
                                                            const T* __restrict__ u,
                                                            T* __restrict__ o, int64_t nvec) {
  const int64_t stride = (int64_t)gridDim.x * kThreads * UNROLL;
  int64_t base = (int64_t)blockIdx.x * kThreads * UNROLL + threadIdx.x;
  for (; base + (int64_t)(UNROLL - 1) * kThreads < nvec; base += stride)
    swiglu_fwd_step<T, UNROLL, true>(g, u, o, base, nvec);
  if (base < nvec) swiglu_fwd_step<T, UNROLL, false>(g, u, o, base, nvec);
}

template <typename T, int UNROLL, bool FULL>
// dy may alias dg (an in-place backward): it carries no __restrict__, and
// every element is loaded before its result is stored.
__device__ __forceinline__ void swiglu_bwd_step(const T* __restrict__ g, const T* __restrict__ u,
                                                const T* dy, T* dg, T* __restrict__ du,
                                                int64_t base, int64_t nvec) {
  constexpr int VEC = vec16<T>();
  float gv[UNROLL][VEC], uv[UNROLL][VEC], yv[UNROLL][VEC];
#pragma unroll
  for (int k = 0; k < UNROLL; ++k) {
    const int64_t i = base + (int64_t)k * kThreads;
    if (FULL || i < nvec) {
      load_n_nt<T, VEC>(g + i * VEC, gv[k]);
      load_n_nt<T, VEC>(u + i * VEC, uv[k]);
      load_n_nt<T, VEC>(dy + i * VEC, yv[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < UNROLL; ++k) {
    const int64_t i = base + (int64_t)k * kThreads;
    if (FULL || i < nvec) {
      float dgv[VEC], duv[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) swiglu_bwd_elem(gv[k][e], uv[k][e], yv[k][e], dgv[e], duv[e]);
      store_n_nt<T, VEC>(dg + i * VEC, dgv);
      store_n_nt<T, VEC>(du + i * VEC, duv);
    }
  }
}

template <typename T, int UNROLL>
__global__ __launch_bounds__(kThreads) void swiglu_bwd_vec(
    const T* __restrict__ g, const T* __restrict__ u, const T* dy, T* dg, T* __restrict__ du,
    int64_t nvec) {
  const int64_t stride = (int64_t)gridDim.x * kThreads * UNROLL;
  int64_t base = (int64_t)blockIdx.x * kThreads * UNROLL + threadIdx.x;
  for (; base + (int64_t)(UNROLL - 1) * kThreads < nvec; base += stride)
    swiglu_bwd_step<T, UNROLL, true>(g, u, dy, dg, du, base, nvec);
  if (base < nvec) swiglu_bwd_step<T, UNROLL, false>(g, u, dy, dg, du, base, nvec);
}

// Scalar kernels for the unaligned case and the tail of the vector path.
template <typename T>
__global__ __launch_bounds__(kThreads) void swiglu_fwd_scalar(const T* __restrict__ g,
                                                               const T* __restrict__ u,
                                                               T* __restrict__ o, int64_t begin,
                                                               int64_t n) {
  for (int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const float gv = to_f32(g[i]);
    o[i] = from_f32<T>(swiglu_fwd_elem(gv, to_f32(u[i])));
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void swiglu_bwd_scalar(
    const T* __restrict__ g, const T* __restrict__ u, const T* dy, T* dg, T* __restrict__ du,
    int64_t begin, int64_t n) {
  for (int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const float gv = to_f32(g[i]);
    const float uv = to_f32(u[i]);
    const float yv = to_f32(dy[i]);
    float dgv, duv;
    swiglu_bwd_elem(gv, uv, yv, dgv, duv);
    du[i] = from_f32<T>(duv);
    dg[i] = from_f32<T>(dgv);
  }
}

// Launch shapes (measured on [8192, 6144] bf16, inputs beyond the MALL): the
// forward runs a grid-stride loop of 2 vectors per thread over 48 blocks per
// CU; the backward covers its work in one pass, 4 vectors of each of its 3
// inputs in flight per thread (81 us against 85 us for the forward's shape).
constexpr int kUnrollFwd = 2;
constexpr int kUnrollBwd = 4;
constexpr int kBlocksPerCuFwd = 48;
constexpr int kBlocksPerCuBwd = 1 << 12;

unsigned stream_grid(int64_t work_items, int per_block, int blocks_per_cu = 16) {
  const int64_t need = (work_items + per_block - 1) / per_block;
  const int64_t cap = (int64_t)num_cus() * blocks_per_cu;
  const int64_t g = need < cap ? need : cap;
  return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace
}  // namespace mla

using namespace mla;

extern "C" int ml_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n, int dtype,
                             void* stream) {
  ML_CHECK(n >= 0, "swiglu: negative size");
  if (n == 0) return ML_OK;
  ML_CHECK(gate && up && out, "swiglu: null pointer");
  hipStream_t st = (hipStream_t)stream;
  return dispatch_dtype(dtype, [&](auto tv) -> int {
    using T = decltype(tv);
    constexpr int VEC = vec16<T>();
    const T* g = static_cast<const T*>(gate);
    const T* u = static_cast<const T*>(up);
    T* o = static_cast<T*>(out);
    int64_t done = 0;
    if (aligned16(g) && aligned16(u) && aligned16(o)) {
      const int64_t nvec = n / VEC;
      if (nvec > 0) {
        swiglu_fwd_vec<T, kUnrollFwd>
            <<<stream_grid(nvec, kThreads * kUnrollFwd, kBlocksPerCuFwd), kThreads, 0, st>>>(g, u, o, nvec);
        ML_LAUNCH_CHECK();
      }
      done = nvec * VEC;
    }
    if (done < n) {
      swiglu_fwd_scalar<T><<<stream_grid(n - done, kThreads), kThreads, 0, st>>>(g, u, o, done, n);
      ML_LAUNCH_CHECK();
    }
    return ML_OK;
  });
}

extern "C" int ml_swiglu_bwd(const void* gate, const void* up, const void* dy, void* dgate,
                             void* dup, int64_t n, int dtype, void* stream) {
  ML_CHECK(n >= 0, "swiglu backward: negative size");
  if (n == 0) return ML_OK;
  ML_CHECK(gate && up && dy && dgate && dup, "swiglu backward: null pointer");
  hipStream_t st = (hipStream_t)stream;
  return dispatch_dtype(dtype, [&](auto tv) -> int {
    using T = decltype(tv);
    constexpr int VEC = vec16<T>();
    const T* g = static_cast<const T*>(gate);
    const T* u = static_cast<const T*>(up);
    const T* y = static_cast<const T*>(dy);
    T* dg = static_cast<T*>(dgate);
    T* du = static_cast<T*>(dup);
    int64_t done = 0;
    if (aligned16(g) && aligned16(u) && aligned16(y) && aligned16(dg) && aligned16(du)) {
      const int64_t nvec = n / VEC;
      if (nvec > 0) {
        swiglu_bwd_vec<T, kUnrollBwd>
            <<<stream_grid(nvec, kThreads * kUnrollBwd, kBlocksPerCuBwd), kThreads, 0, st>>>(g, u, y, dg, du, nvec);
        ML_LAUNCH_CHECK();
      }
      done = nvec * VEC;
    }
    if (done < n) {
      swiglu_bwd_scalar<T>
          <<<stream_grid(n - done, kThreads), kThreads, 0, st>>>(g, u, y, dg, du, done, n);
      ML_LAUNCH_CHECK();
    }
    return ML_OK;
  });
}

// Plain bf16 GEMM entry points over the MFMA core:
//   C = alpha * op(A) op(B) + beta * C     (fp32 accumulation, C bf16 or fp32)
// with K optionally split into segments (K-concatenated operands).
#include "gemm_core.h"

namespace mla {
namespace gemm {
namespace {

int run(int64_t M, int64_t N, int nseg, const Segment* segs, int la, int lb, void* C, int64_t ldc,
        int c_dtype, float alpha, float beta, void* stream) {
  ML_CHECK(M > 0 && N > 0 && M < (1LL << 31) && N < (1LL << 31), "gemm: bad M=%lld N=%lld",
           (long long)M, (long long)N);
  ML_CHECK(la == kKMajor || la == kMNMajor, "gemm: bad A layout %d", la);
  ML_CHECK(lb == kKMajor || lb == kMNMajor, "gemm: bad B layout %d", lb);
  ML_CHECK(C != nullptr && ldc >= N, "gemm: bad C (ldc %lld < N %lld)", (long long)ldc,
           (long long)N);
  // the bf16 store epilogue writes rows of 8 columns as 16-byte vectors
  ML_CHECK(c_dtype != ML_BF16 || (ldc % 8 == 0 && aligned16(C)),
           "gemm: a bf16 C needs ldc a multiple of 8 and a 16-byte aligned base (ldc %lld)",
           (long long)ldc);
  Problem pb;
  int rc = make_problem<BigCfg>(pb, (int)M, (int)N, nseg, segs, la, lb, 0);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  // r4 is the faster engine when A is K-major, the big engine otherwise
  if (la == kKMajor) {
    if (c_dtype == ML_F32) return launch_store<float, R4Cfg>(pb, la, lb, C, ldc, alpha, beta, st);
    if (c_dtype == ML_BF16) return launch_store<bf16, R4Cfg>(pb, la, lb, C, ldc, alpha, beta, st);
  } else {
    if (c_dtype == ML_F32) return launch_store<float>(pb, la, lb, C, ldc, alpha, beta, st);
    if (c_dtype == ML_BF16) return launch_store<bf16>(pb, la, lb, C, ldc, alpha, beta, st);
  }
  set_error("gemm: C dtype %d not supported (fp32 or bf16)", c_dtype);
  return ML_ERR_INVALID;
}

// Split-K / tile-shape variant (cfg 0: 256x256, 1: 256x32, 2: 64x256).
template <class C, typename TC>
int run_splitk_cfg(const Problem& pb, int la, int lb, float* ws, TC* out, int64_t ldo, float alpha,
                   float beta, hipStream_t st) {
  if (la == kKMajor && lb == kKMajor) return launch_splitk<C, kKMajor, kKMajor, TC>(pb, ws, out, ldo, alpha, beta, st);
  if (la == kKMajor && lb == kMNMajor) return launch_splitk<C, kKMajor, kMNMajor, TC>(pb, ws, out, ldo, alpha, beta, st);
  if (la == kMNMajor && lb == kKMajor) return launch_splitk<C, kMNMajor, kKMajor, TC>(pb, ws, out, ldo, alpha, beta, st);
  return launch_splitk<C, kMNMajor, kMNMajor, TC>(pb, ws, out, ldo, alpha, beta, st);
}

template <class C>
int run_splitk(int64_t M, int64_t N, const Segment& seg, int la, int lb, int ksplit, void* C_,
               int64_t ldc, int c_dtype, float alpha, float beta, void* ws, size_t ws_bytes,
               hipStream_t st) {
  Problem pb;
  int rc = make_problem<C>(pb, (int)M, (int)N, 1, &seg, la, lb, 0, ksplit);
  if (rc) return rc;
  ML_CHECK(ws && ws_bytes >= splitk_ws_bytes(pb), "gemm: split-K workspace too small (%zu < %zu)",
           ws_bytes, splitk_ws_bytes(pb));
  float* w = static_cast<float*>(ws);
  if (c_dtype == ML_F32)
    return run_splitk_cfg<C, float>(pb, la, lb, w, static_cast<float*>(C_), ldc, alpha, beta, st);
  if (c_dtype == ML_BF16)
    return run_splitk_cfg<C, bf16>(pb, la, lb, w, static_cast<bf16*>(C_), ldc, alpha, beta, st);
  set_error("gemm: C dtype %d not supported (fp32 or bf16)", c_dtype);
  return ML_ERR_INVALID;
}

}  // namespace
}  // namespace gemm
}  // namespace mla

using namespace mla;

extern "C" int ml_gemm_bf16(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                            int a_layout, const void* B, int64_t ldb, int b_layout, void* C,
                            int64_t ldc, int c_dtype, float alpha, float beta, void* stream) {
  ML_CHECK(K >= 0 && K < (1LL << 31), "gemm: bad K=%lld", (long long)K);
  gemm::Segment s{{static_cast<const bf16*>(A), lda}, {static_cast<const bf16*>(B), ldb}, (int)K};
  return gemm::run(M, N, 1, &s, a_layout, b_layout, C, ldc, c_dtype, alpha, beta, stream);
}

extern "C" int ml_gemm_bf16_segments(int64_t M, int64_t N, int nseg, const int64_t* k_lens,
                                     const void* const* a_ptrs, const int64_t* ldas,
                                     const void* const* b_ptrs, const int64_t* ldbs, int a_layout,
                                     int b_layout, void* C, int64_t ldc, int c_dtype, float alpha,
                                     float beta, void* stream) {
  ML_CHECK(nseg >= 1 && nseg <= gemm::kMaxSeg, "gemm: 1..%d segments supported (got %d)",
           gemm::kMaxSeg, nseg);
  ML_CHECK(k_lens && a_ptrs && ldas && b_ptrs && ldbs, "gemm: null segment arrays");
  gemm::Segment segs[gemm::kMaxSeg];
  for (int s = 0; s < nseg; ++s) {
    ML_CHECK(k_lens[s] >= 0 && k_lens[s] < (1LL << 31), "gemm: bad K segment %d", s);
    segs[s] = gemm::Segment{{static_cast<const bf16*>(a_ptrs[s]), ldas[s]},
                            {static_cast<const bf16*>(b_ptrs[s]), ldbs[s]}, (int)k_lens[s]};
  }
  return gemm::run(M, N, nseg, segs, a_layout, b_layout, C, ldc, c_dtype, alpha, beta, stream);
}

extern "C" int ml_gemm_bf16_segments_group(int count, const int64_t* M, const int64_t* N,
                                           const int* nseg, const int64_t* k_lens,
                                           const void* const* a_ptrs, const int64_t* ldas,
                                           const void* const* b_ptrs, const int64_t* ldbs,
                                           int b_layout, void* const* C, const int64_t* ldc,
                                           int c_dtype, float alpha, float beta, void* stream) {
  ML_CHECK(count >= 1 && count <= gemm::kMaxGroup, "gemm group: 1..%d products (got %d)",
           gemm::kMaxGroup, count);
  ML_CHECK(M && N && nseg && k_lens && a_ptrs && ldas && b_ptrs && ldbs && C && ldc,
           "gemm group: null argument arrays");
  ML_CHECK(b_layout == gemm::kKMajor || b_layout == gemm::kMNMajor, "gemm group: bad B layout");
  gemm::Problem pbs[gemm::kMaxGroup];
  int base = 0;
  for (int g = 0; g < count; ++g) {
    ML_CHECK(M[g] > 0 && N[g] > 0 && M[g] < (1LL << 31) && N[g] < (1LL << 31),
             "gemm group: bad M=%lld N=%lld (product %d)", (long long)M[g], (long long)N[g], g);
    ML_CHECK(C[g] != nullptr && ldc[g] >= N[g], "gemm group: bad C (product %d)", g);
    ML_CHECK(c_dtype != ML_BF16 || (ldc[g] % 8 == 0 && aligned16(C[g])),
             "gemm group: a bf16 C needs ldc a multiple of 8 and a 16-byte aligned base "
             "(product %d, ldc %lld)", g, (long long)ldc[g]);
    ML_CHECK(nseg[g] >= 1 && nseg[g] <= gemm::kMaxSeg, "gemm group: 1..%d segments (product %d)",
             gemm::kMaxSeg, g);
    gemm::Segment segs[gemm::kMaxSeg];
    for (int s = 0; s < nseg[g]; ++s) {
      const int q = base + s;
      ML_CHECK(k_lens[q] >= 0 && k_lens[q] < (1LL << 31), "gemm group: bad K segment %d", q);
      segs[s] = gemm::Segment{{static_cast<const bf16*>(a_ptrs[q]), ldas[q]},
                              {static_cast<const bf16*>(b_ptrs[q]), ldbs[q]}, (int)k_lens[q]};
    }
    const int rc = gemm::make_problem<gemm::R4Cfg>(pbs[g], (int)M[g], (int)N[g], nseg[g], segs,
                                                   gemm::kKMajor, b_layout, 0);
    if (rc) return rc;
    base += nseg[g];
  }
  hipStream_t st = (hipStream_t)stream;
  if (c_dtype == ML_BF16)
    return gemm::launch_store_group<bf16>(pbs, count, b_layout, C, ldc, alpha, beta, st);
  if (c_dtype == ML_F32)
    return gemm::launch_store_group<float>(pbs, count, b_layout, C, ldc, alpha, beta, st);
  set_error("gemm group: C dtype %d not supported (fp32 or bf16)", c_dtype);
  return ML_ERR_INVALID;
}

extern "C" size_t ml_gemm_splitk_workspace_bytes(int64_t M, int64_t N, int64_t K, int ksplit) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const int64_t total = (K + gemm::kBK - 1) / gemm::kBK;
  const int64_t ks = ksplit < 1 ? 1 : ksplit;
  const int64_t kps = (total + ks - 1) / ks;
  const int64_t splits = (total + kps - 1) / kps;
  return (size_t)(splits * M * N) * sizeof(float);
}

extern "C" int ml_gemm_bf16_splitk(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                                   int a_layout, const void* B, int64_t ldb, int b_layout, void* C,
                                   int64_t ldc, int c_dtype, float alpha, float beta, int tile_cfg,
                                   int ksplit, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  ML_CHECK(M > 0 && N > 0 && M < (1LL << 31) && N < (1LL << 31), "gemm: bad M=%lld N=%lld",
           (long long)M, (long long)N);
  ML_CHECK(K > 0 && K < (1LL << 31), "gemm: bad K=%lld", (long long)K);
  ML_CHECK(a_layout == gemm::kKMajor || a_layout == gemm::kMNMajor, "gemm: bad A layout");
  ML_CHECK(b_layout == gemm::kKMajor || b_layout == gemm::kMNMajor, "gemm: bad B layout");
  ML_CHECK(C != nullptr && ldc >= N, "gemm: bad C");
  ML_CHECK(ksplit >= 1, "gemm: ksplit must be >= 1");
  gemm::Segment s{{static_cast<const bf16*>(A), lda}, {static_cast<const bf16*>(B), ldb}, (int)K};
  hipStream_t st = (hipStream_t)stream;
  switch (tile_cfg) {
    case 0: return gemm::run_splitk<gemm::BigCfg>(M, N, s, a_layout, b_layout, ksplit, C, ldc, c_dtype, alpha, beta, workspace, workspace_bytes, st);
    case 1: return gemm::run_splitk<gemm::TallCfg>(M, N, s, a_layout, b_layout, ksplit, C, ldc, c_dtype, alpha, beta, workspace, workspace_bytes, st);
    case 2: return gemm::run_splitk<gemm::WideCfg>(M, N, s, a_layout, b_layout, ksplit, C, ldc, c_dtype, alpha, beta, workspace, workspace_bytes, st);
    default: set_error("gemm: tile_cfg must be 0 (256x256), 1 (256x32) or 2 (64x256)"); return ML_ERR_INVALID;
  }
}

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
  Problem pb;
  int rc = make_problem(pb, (int)M, (int)N, nseg, segs, la, lb, 0);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (c_dtype == ML_F32) return launch_store<float>(pb, la, lb, C, ldc, alpha, beta, st);
  if (c_dtype == ML_BF16) return launch_store<bf16>(pb, la, lb, C, ldc, alpha, beta, st);
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

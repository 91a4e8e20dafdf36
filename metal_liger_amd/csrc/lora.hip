// Fused LoRA QKV / MLP backward for gfx950 (ops/fused_lora.py:121-171, :209-266).
//
// Per adapter with base W [out, in], A [r, in], B [out, r], scale s, the
// reference computes (dY the output grad, X the saved input):
//   dA = s (dY B)^T X          dB = s dY^T (X A^T)        dX += dY W + s (dY B) A
// Here, with every product on the bf16 MFMA engine (fp32 accumulation):
//   P   = s dY B               [tokens, r]   256x32 tiles, split-K over out
//   dA  = P^T X                [r, in]       64x256 tiles, split-K over tokens
//   dB  = s dY^T XA            [out, r]      256x32 tiles, split-K over tokens
//                                            (XA = X A^T saved by the forward)
//   dX  = [dY_1 | .. | dY_n | P_1..n] [W_1; ..; W_n; A_1..n]
//         ONE 256x256-tile GEMM over the K-concatenation of every adapter's
//         dY with its W plus the stacked rank-r terms (K = sum(out) + n r).
// The MLP backward first forms dH = dY_D W_D + P_D A_D with the SwiGLU
// backward fused into that GEMM's epilogue (gate / up read there, d_gate /
// d_up written in bf16; sigmoid recomputed), then treats (d_gate, d_up) as
// the output grads of the gate / up adapters. Split-K partials are summed in
// a fixed order, so every gradient is bit-reproducible.
#include <algorithm>

#include "gemm_core.h"

namespace mla {
namespace lora {
namespace {

using namespace gemm;

constexpr int kTargetItems = 512;  // work items per skinny launch (~2 per CU)

int pick_ksplit(int tiles, int k_len) {
  const int ktiles = (k_len + kBK - 1) / kBK;
  int ks = (kTargetItems + tiles - 1) / (tiles > 0 ? tiles : 1);
  ks = ks < 1 ? 1 : ks;
  return ks < ktiles ? ks : ktiles;
}

template <class C>
int tiles_of(int M, int N) {
  return ((M + C::BM - 1) / C::BM) * ((N + C::BN - 1) / C::BN);
}

// Split-K skinny product with its own partial workspace bound check.
template <class C, int LA, int LB, typename TC>
int skinny(int M, int N, const Segment& seg, TC* out, int64_t ldo, float alpha, float* ws,
           size_t ws_bytes, hipStream_t st) {
  Problem pb;
  int rc = make_problem<C>(pb, M, N, 1, &seg, LA, LB, 0, pick_ksplit(tiles_of<C>(M, N), seg.k_len));
  if (rc) return rc;
  ML_CHECK(splitk_ws_bytes(pb) <= ws_bytes, "lora: split-K workspace too small (%zu < %zu)",
           ws_bytes, splitk_ws_bytes(pb));
  return launch_splitk<C, LA, LB, TC>(pb, ws, out, ldo, alpha, 0.f, st);
}

template <class C>
size_t skinny_ws(int M, int N, int k_len) {
  const int ks = pick_ksplit(tiles_of<C>(M, N), k_len);
  const int ktiles = (k_len + kBK - 1) / kBK;
  const int kps = (ktiles + ks - 1) / ks;
  const int splits = (ktiles + kps - 1) / kps;
  return (size_t)splits * M * N * sizeof(float);
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

}  // namespace
}  // namespace lora
}  // namespace mla

using namespace mla;
using namespace mla::gemm;

// ------------------------------------------------------------------- QKV --

static size_t qkv_partial_bytes(int64_t N, int64_t in_f, const int64_t* out_f, int nadp,
                                int64_t r) {
  size_t m = lora::skinny_ws<WideCfg>((int)(nadp * r), (int)in_f, (int)N);
  for (int i = 0; i < nadp; ++i) {
    m = std::max(m, lora::skinny_ws<TallCfg>((int)N, (int)r, (int)out_f[i]));
    m = std::max(m, lora::skinny_ws<TallCfg>((int)out_f[i], (int)r, (int)N));
  }
  return m;
}

extern "C" size_t ml_lora_qkv_bwd_workspace_bytes(int64_t n_tokens, int64_t in_features,
                                                  const int64_t* out_features, int64_t rank) {
  if (n_tokens <= 0 || in_features <= 0 || rank <= 0 || !out_features) return 0;
  return lora::align256((size_t)(n_tokens * 3 * rank) * 2) +
         qkv_partial_bytes(n_tokens, in_features, out_features, 3, rank);
}

extern "C" int ml_lora_qkv_bwd(const void* X, int64_t n_tokens, int64_t in_features,
                               const void* const* dY, const int64_t* out_features,
                               const void* const* W, const void* A_stack, const void* const* B,
                               const float* scale, const void* XA, int64_t rank, void* dX,
                               float* dA, float* const* dB, void* workspace,
                               size_t workspace_bytes, void* stream) {
  const int nadp = 3;
  ML_CHECK(n_tokens > 0 && in_features > 0 && rank > 0, "lora qkv: bad sizes");
  ML_CHECK(n_tokens < (1LL << 31) && in_features < (1LL << 31), "lora qkv: sizes too large");
  ML_CHECK(in_features % 8 == 0 && rank % 8 == 0, "lora qkv: in_features and rank must be multiples of 8");
  ML_CHECK(X && dY && out_features && W && A_stack && B && scale && XA && dX && dA && dB,
           "lora qkv: null pointer");
  for (int i = 0; i < nadp; ++i) {
    ML_CHECK(dY[i] && W[i] && B[i] && dB[i], "lora qkv: null pointer for adapter %d", i);
    ML_CHECK(out_features[i] > 0 && out_features[i] % 8 == 0 && out_features[i] < (1LL << 31),
             "lora qkv: out_features[%d] must be a positive multiple of 8", i);
  }
  const size_t need = ml_lora_qkv_bwd_workspace_bytes(n_tokens, in_features, out_features, rank);
  ML_CHECK(workspace && workspace_bytes >= need, "lora qkv: workspace too small (%zu < %zu)",
           workspace_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  const int N = (int)n_tokens, IN = (int)in_features, R = (int)rank, R3 = 3 * (int)rank;
  char* ws = static_cast<char*>(workspace);
  bf16* P = reinterpret_cast<bf16*>(ws);  // [N, 3r], column block i = s_i dY_i B_i
  float* part = reinterpret_cast<float*>(ws + lora::align256((size_t)N * R3 * 2));
  const size_t part_bytes = workspace_bytes - lora::align256((size_t)N * R3 * 2);
  const bf16* x = static_cast<const bf16*>(X);
  const bf16* xa = static_cast<const bf16*>(XA);
  int rc;
  for (int i = 0; i < nadp; ++i) {
    const int OUT = (int)out_features[i];
    const bf16* dy = static_cast<const bf16*>(dY[i]);
    // P_i = s_i dY_i B_i: A = dY_i [N, out] K-major, B = B_i [out, r] (k = out, n = r) MN-major
    Segment sp{{dy, OUT}, {static_cast<const bf16*>(B[i]), R}, OUT};
    rc = lora::skinny<TallCfg, kKMajor, kMNMajor, bf16>(N, R, sp, P + i * R, R3, scale[i], part,
                                                         part_bytes, st);
    if (rc) return rc;
    // dB_i = s_i dY_i^T XA_i: A = dY_i^T (MN-major, ld out), B = XA_i (MN-major, ld 3r)
    Segment sb{{dy, OUT}, {xa + i * R, R3}, N};
    rc = lora::skinny<TallCfg, kMNMajor, kMNMajor, float>(OUT, R, sb, dB[i], R, scale[i], part,
                                                           part_bytes, st);
    if (rc) return rc;
  }
  // dA_stack = P^T X: A = P^T (MN-major, ld 3r), B = X (MN-major, ld in)
  Segment sa{{P, R3}, {x, IN}, N};
  rc = lora::skinny<WideCfg, kMNMajor, kMNMajor, float>(R3, IN, sa, dA, IN, 1.0f, part, part_bytes,
                                                         st);
  if (rc) return rc;
  // dX = [dQ | dK | dV | P] [Wq; Wk; Wv; A_stack]
  Segment segs[4];
  for (int i = 0; i < nadp; ++i)
    segs[i] = Segment{{static_cast<const bf16*>(dY[i]), out_features[i]},
                      {static_cast<const bf16*>(W[i]), IN}, (int)out_features[i]};
  segs[3] = Segment{{P, R3}, {static_cast<const bf16*>(A_stack), IN}, R3};
  Problem pb;
  rc = make_problem<BigCfg>(pb, N, IN, 4, segs, kKMajor, kMNMajor, 0);
  if (rc) return rc;
  return launch_store<bf16>(pb, kKMajor, kMNMajor, dX, IN, 1.0f, 0.0f, st);
}

// ------------------------------------------------------------------- MLP --

static size_t mlp_partial_bytes(int64_t N, int64_t H, int64_t I, int64_t r) {
  size_t m = lora::skinny_ws<TallCfg>((int)N, (int)r, (int)H);          // P_D
  m = std::max(m, lora::skinny_ws<WideCfg>((int)r, (int)I, (int)N));   // dA_D
  m = std::max(m, lora::skinny_ws<TallCfg>((int)H, (int)r, (int)N));   // dB_D
  m = std::max(m, lora::skinny_ws<TallCfg>((int)N, (int)r, (int)I));   // P_G, P_U
  m = std::max(m, lora::skinny_ws<WideCfg>((int)(2 * r), (int)H, (int)N));  // dA_GU
  m = std::max(m, lora::skinny_ws<TallCfg>((int)I, (int)r, (int)N));   // dB_G, dB_U
  return m;
}

extern "C" size_t ml_lora_mlp_bwd_workspace_bytes(int64_t n_tokens, int64_t hidden,
                                                  int64_t intermediate, int64_t rank) {
  if (n_tokens <= 0 || hidden <= 0 || intermediate <= 0 || rank <= 0) return 0;
  return 2 * lora::align256((size_t)(n_tokens * intermediate) * 2) +
         lora::align256((size_t)(n_tokens * rank) * 2) +
         lora::align256((size_t)(n_tokens * 2 * rank) * 2) +
         mlp_partial_bytes(n_tokens, hidden, intermediate, rank);
}

extern "C" int ml_lora_mlp_bwd(const void* X, int64_t n_tokens, int64_t hidden,
                               int64_t intermediate, const void* gate, const void* up,
                               const void* h, const void* dY, const void* WG, const void* WU,
                               const void* WD, const void* A_GU, const void* A_D, const void* BG,
                               const void* BU, const void* BD, const float* scale,
                               const void* XA_GU, const void* hA_D, int64_t rank, void* dX,
                               float* dA_GU, float* dA_D, float* dB_G, float* dB_U, float* dB_D,
                               void* workspace, size_t workspace_bytes, void* stream) {
  ML_CHECK(n_tokens > 0 && hidden > 0 && intermediate > 0 && rank > 0, "lora mlp: bad sizes");
  ML_CHECK(n_tokens < (1LL << 31) && hidden < (1LL << 31) && intermediate < (1LL << 31),
           "lora mlp: sizes too large");
  ML_CHECK(hidden % 8 == 0 && intermediate % 8 == 0 && rank % 8 == 0,
           "lora mlp: hidden, intermediate and rank must be multiples of 8");
  ML_CHECK(X && gate && up && h && dY && WG && WU && WD && A_GU && A_D && BG && BU && BD && scale &&
               XA_GU && hA_D && dX && dA_GU && dA_D && dB_G && dB_U && dB_D,
           "lora mlp: null pointer");
  const size_t need = ml_lora_mlp_bwd_workspace_bytes(n_tokens, hidden, intermediate, rank);
  ML_CHECK(workspace && workspace_bytes >= need, "lora mlp: workspace too small (%zu < %zu)",
           workspace_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  const int N = (int)n_tokens, H = (int)hidden, I = (int)intermediate, R = (int)rank, R2 = 2 * R;
  char* ws = static_cast<char*>(workspace);
  bf16* dgate = reinterpret_cast<bf16*>(ws);
  ws += lora::align256((size_t)N * I * 2);
  bf16* dup = reinterpret_cast<bf16*>(ws);
  ws += lora::align256((size_t)N * I * 2);
  bf16* PD = reinterpret_cast<bf16*>(ws);  // [N, r]  = s_D dY B_D
  ws += lora::align256((size_t)N * R * 2);
  bf16* PGU = reinterpret_cast<bf16*>(ws);  // [N, 2r] = [s_G d_gate B_G | s_U d_up B_U]
  ws += lora::align256((size_t)N * R2 * 2);
  float* part = reinterpret_cast<float*>(ws);
  const size_t part_bytes = workspace_bytes - (size_t)(ws - static_cast<char*>(workspace));
  const bf16* x = static_cast<const bf16*>(X);
  const bf16* dy = static_cast<const bf16*>(dY);
  int rc;

  // down projection: P_D, dA_D = P_D^T h, dB_D = s_D dY^T hA_D
  Segment s1{{dy, H}, {static_cast<const bf16*>(BD), R}, H};
  rc = lora::skinny<TallCfg, kKMajor, kMNMajor, bf16>(N, R, s1, PD, R, scale[2], part, part_bytes, st);
  if (rc) return rc;
  Segment s2{{PD, R}, {static_cast<const bf16*>(h), I}, N};
  rc = lora::skinny<WideCfg, kMNMajor, kMNMajor, float>(R, I, s2, dA_D, I, 1.0f, part, part_bytes, st);
  if (rc) return rc;
  Segment s3{{dy, H}, {static_cast<const bf16*>(hA_D), R}, N};
  rc = lora::skinny<TallCfg, kMNMajor, kMNMajor, float>(H, R, s3, dB_D, R, scale[2], part,
                                                         part_bytes, st);
  if (rc) return rc;
  // dH = dY W_D + P_D A_D, a bf16 product as in the reference
  // (ops/fused_lora.py:230-233), written into d_gate's buffer; then the
  // SwiGLU backward (:235-244) streams dH, gate, up into d_gate (in place:
  // each element is read before it is written) and d_up. Two passes beat
  // the backward fused into the GEMM's epilogue here: with every CU in the
  // epilogue at once, the 512 KB of gate / up / d_gate / d_up per tile left
  // the matrix cores idle (324 us against 200 + 74 us).
  {
    Segment segs[2] = {Segment{{dy, H}, {static_cast<const bf16*>(WD), I}, H},
                       Segment{{PD, R}, {static_cast<const bf16*>(A_D), I}, R}};
    Problem pb;
    rc = make_problem<BigCfg>(pb, N, I, 2, segs, kKMajor, kMNMajor, 0);
    if (rc) return rc;
    rc = launch_store<bf16>(pb, kKMajor, kMNMajor, dgate, I, 1.f, 0.f, st);
    if (rc) return rc;
    rc = ml_swiglu_bwd(gate, up, dgate, dgate, dup, (int64_t)N * I, ML_BF16, st);
    if (rc) return rc;
  }
  // gate / up adapters
  const bf16* dgu[2] = {dgate, dup};
  const void* Bs[2] = {BG, BU};
  float* dBs[2] = {dB_G, dB_U};
  const bf16* xa = static_cast<const bf16*>(XA_GU);
  for (int i = 0; i < 2; ++i) {
    Segment sp{{dgu[i], I}, {static_cast<const bf16*>(Bs[i]), R}, I};
    rc = lora::skinny<TallCfg, kKMajor, kMNMajor, bf16>(N, R, sp, PGU + i * R, R2, scale[i], part,
                                                         part_bytes, st);
    if (rc) return rc;
    Segment sb{{dgu[i], I}, {xa + i * R, R2}, N};
    rc = lora::skinny<TallCfg, kMNMajor, kMNMajor, float>(I, R, sb, dBs[i], R, scale[i], part,
                                                           part_bytes, st);
    if (rc) return rc;
  }
  Segment sa{{PGU, R2}, {x, H}, N};
  rc = lora::skinny<WideCfg, kMNMajor, kMNMajor, float>(R2, H, sa, dA_GU, H, 1.0f, part,
                                                         part_bytes, st);
  if (rc) return rc;
  // dX = [d_gate | d_up | P_GU] [W_G; W_U; A_GU]
  Segment segs[3] = {Segment{{dgate, I}, {static_cast<const bf16*>(WG), H}, I},
                     Segment{{dup, I}, {static_cast<const bf16*>(WU), H}, I},
                     Segment{{PGU, R2}, {static_cast<const bf16*>(A_GU), H}, R2}};
  Problem pb;
  rc = make_problem<BigCfg>(pb, N, H, 3, segs, kKMajor, kMNMajor, 0);
  if (rc) return rc;
  return launch_store<bf16>(pb, kKMajor, kMNMajor, dX, H, 1.0f, 0.0f, st);
}

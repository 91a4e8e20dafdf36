// Fused LoRA QKV / MLP backward for gfx950 (ops/fused_lora.py:121-171, :209-266).
//
// Per adapter with base W [out, in], A [r, in], B [out, r], scale s, the
// reference computes (dY the output grad, X the saved input):
//   dA = s (dY B)^T X          dB = s dY^T (X A^T)        dX += dY W + s (dY B) A
// Here, with every product on bf16 MFMAs (fp32 accumulation):
//   P, dB = s dY B, s dY^T XA  ONE pass over dY (dy_pass_kernel, rank 16;
//                              XA = X A^T saved by the forward); other ranks
//                              use two split-K skinny products
//   dA  = P^T X                [r, in]       64x256 tiles, split-K over tokens
//   dX  = [dY_1 | .. | dY_n | P_1..n] [W_1; ..; W_n; A_1..n]
//         ONE 256x256-tile GEMM over the K-concatenation of every adapter's
//         dY with its W plus the stacked rank-r terms (K = sum(out) + n r).
// The MLP backward first forms dH = dY_D W_D + P_D A_D (bf16), runs the
// SwiGLU backward over it in place (sigmoid recomputed), then treats
// (d_gate, d_up) as the output grads of the gate / up adapters; at rank 16
// one pass (mlp_mid_kernel) does the SwiGLU backward, the gate / up dY-pass
// work and P_D^T h. Partials are
// summed in a fixed order, so every gradient is bit-reproducible.
#include <algorithm>

#include "gemm_core.h"
#include "swiglu_math.h"

namespace mla {
namespace lora {
namespace {

using namespace gemm;

constexpr int kTargetItems = 512;  // work items per skinny launch (~2 per CU)

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

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

// ------------------------------------------------------------- dY pass --
// One pass over an adapter's output grad dY [N, O] (bf16) gives both rank-r
// products that read it (rank padded to 16):
//   P  = s dY B       [N, 16]    (a reduction over O)
//   dB = s dY^T XA    [O, 16]    (a reduction over N; XA = X A^T)
// A workgroup of 4 waves owns a 256 x 256 tile of dY (rows m0 .., columns
// c0 ..) and streams it through LDS in chunks of 32 rows, loaded global ->
// LDS three chunks ahead, each chunk laid out like the GEMM engine's
// MN-major k-tile (32 rows of 512 B; the 32-byte unit u of row r at
// u ^ h(r)), with the chunk's 32 XA rows (1 KB) beside it. Per chunk:
//   P:  A = the chunk's rows (ds_read_b128 of 8 columns), B = B[c][0..15]
//       in registers (loaded once); wave w takes columns 64 w .. 64 w + 63
//       (two k-steps of 32), the four waves' partial sums meet in LDS and
//       the tile's fp32 partial goes to Ppart[ctile][row][16];
//   dB: A = the chunk transposed (two ds_read_b64_tr_b16 per fragment),
//       B = the chunk's XA rows; wave w accumulates columns 64 w .. 64 w + 63
//       (four 16 x 16 tiles) over the tile's rows, written at the end to
//       dBpart[rtile][col][16].
// The partials are summed in a fixed order by dy_reduce_kernel, which also
// applies s (bit-reproducible results). Columns past O load the last
// valid 8 columns again and meet B = 0 / are not stored; rows past N load
// as zeros.
constexpr int kDyRows = 256, kDyCols = 256, kDyChunk = 32, kDyStages = 4, kDyRank = 16;
constexpr int kDyChunkBytes = kDyChunk * kDyCols * 2;  // 16 KB
constexpr int kDyXaBytes = kDyChunk * kDyRank * 2;     // 1 KB
constexpr int kDyStageBytes = kDyChunkBytes + kDyXaBytes;
constexpr int kDyMaxAdapters = 3;
// 5 loads per wave per chunk (4 x 1 KB of dY, 256 B of XA); with three
// chunks in flight, chunk t has landed once at most 10 remain.
constexpr int kDyWaitAhead = big::wait_vm(10);

struct DyAdapter {
  const bf16* dy;  // [N, O], row stride ldy
  const bf16* b;   // [O, 16] (B padded to rank 16), row stride ldb
  const bf16* xa;  // [N, 16] slice of X A^T, row stride ldxa
  float* ppart;    // [ctiles][N][16]
  float* dbpart;   // [rtiles][O][16]
  int64_t ldy, ldb, ldxa;
  int O, ctiles, first;  // first: this adapter's first workgroup
};

struct DyArgs {
  DyAdapter ad[kDyMaxAdapters];
  int nadp, N;
};

inline int dy_ctiles(int O) { return (O + kDyCols - 1) / kDyCols; }
inline int dy_rtiles(int N) { return (N + kDyRows - 1) / kDyRows; }
inline size_t dy_ppart_bytes(int N, int O) { return (size_t)dy_ctiles(O) * N * kDyRank * 4; }
inline size_t dy_dbpart_bytes(int N, int O) { return (size_t)dy_rtiles(N) * O * kDyRank * 4; }

__global__ __launch_bounds__(256) void dy_pass_kernel(const DyArgs args) {
  __shared__ __attribute__((aligned(16))) char lds[kDyStages * kDyStageBytes];
  __shared__ __attribute__((aligned(16))) float pred[4][kDyChunk * kDyRank];
  const int bid = blockIdx.x;
  const int ai = (args.nadp > 2 && bid >= args.ad[2].first) ? 2
                 : (args.nadp > 1 && bid >= args.ad[1].first) ? 1 : 0;
  const DyAdapter& A = ai == 0 ? args.ad[0] : ai == 1 ? args.ad[1] : args.ad[2];
  const int local = bid - A.first;
  const int ct = local % A.ctiles, rt = local / A.ctiles;
  const int m0 = rt * kDyRows, c0 = ct * kDyCols;
  const int N = args.N, O = A.O;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rows = N - m0 < kDyRows ? N - m0 : kDyRows;
  const int nchunks = (rows + kDyChunk - 1) / kDyChunk;

  // B fragments of this wave's two k-steps: lane (n = lane % 16, k group
  // lane / 16) holds B[c][n] for c = c0 + 64 w + 32 ks + 8 (lane / 16) + j.
  bf16x8_t bfr[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int cb = c0 + 64 * wave + 32 * ks + 8 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = cb + j;
      bfr[ks][j] = c < O ? A.b[(int64_t)c * A.ldb + (lane & 15)] : static_cast<bf16>(0.f);
    }
  }
  __builtin_amdgcn_s_waitcnt(big::kWaitVm0);  // before the LDS loads start counting

  // Per-lane load offsets: dY group g = wave + 4 i covers chunk rows 2 g,
  // 2 g + 1; lane l fetches the 8 columns its LDS slot holds.
  uint32_t dyoff[4];
  int dyrow[4];
  {
    const int p = lane & 31;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 2 * (wave + 4 * i) + (lane >> 5);
      const int h = (r & 3) | (((r >> 3) & 1) << 2);
      int e = 8 * (2 * ((p >> 1) ^ h) + (p & 1));
      e = c0 + e <= O - 8 ? e : O - 8 - c0;
      dyoff[i] = (uint32_t)(((int64_t)r * A.ldy + c0 + e) * 2);
      dyrow[i] = r;
    }
  }
  // XA: wave w loads rows 8 w .. 8 w + 7 of the chunk, lane l one dword.
  const int xarow = 8 * wave + (lane >> 3);
  const uint32_t xaoff = (uint32_t)(((int64_t)xarow * A.ldxa + 2 * (lane & 7)) * 2);

  auto chunk_loads = [&](int t, char* st) __attribute__((always_inline)) {
    const int rbase = m0 + kDyChunk * t;
    const rsrc_t ry = make_rsrc(reinterpret_cast<const char*>(A.dy + (int64_t)rbase * A.ldy));
    const rsrc_t rx = make_rsrc(reinterpret_cast<const char*>(A.xa + (int64_t)rbase * A.ldxa));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = t < nchunks && rbase + dyrow[i] < N;
      buf_load_lds(ry, ok ? dyoff[i] : big::kOob, st + (wave + 4 * i) * 1024);
    }
    const bool okx = t < nchunks && rbase + xarow < N;
    buf_load_lds_dword(rx, okx ? xaoff : big::kOob, st + kDyChunkBytes + wave * 256);
  };

  FragAddr<kMNMajor, 4> fa;
  frag_addr_setup<kMNMajor, 4>(fa, 64 * wave, lane);
  f32x4_t accb[4];
#pragma unroll
  for (int f = 0; f < 4; ++f) accb[f] = f32x4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int j = 0; j < kDyStages - 1; ++j) chunk_loads(j, lds + j * kDyStageBytes);

  for (int t = 0; t < nchunks; ++t) {
    char* cur = lds + (t % kDyStages) * kDyStageBytes;
    __builtin_amdgcn_s_waitcnt(kDyWaitAhead);
    __syncthreads();  // chunk t published; stage (t - 1) % 4 and pred free
    chunk_loads(t + kDyStages - 1, lds + ((t + kDyStages - 1) % kDyStages) * kDyStageBytes);

    // P: rows 16 mt + lane % 16, columns 64 w + 32 ks + 8 (lane / 16) ..
    f32x4_t accp[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int r = 16 * mt + (lane & 15);
      const int h = (r & 3) | (((r >> 3) & 1) << 2);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int c = 64 * wave + 32 * ks + 8 * (lane >> 4);
        const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(
            cur + r * 512 + (((c >> 4) ^ h) << 5) + (c & 15) * 2);
        accp[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bfr[ks], accp[mt], 0, 0, 0);
      }
    }
    // dB: B operand = XA rows 8 (lane / 16) + j of column lane % 16
    bf16x8_t xf;
    {
      const bf16* xl = reinterpret_cast<const bf16*>(cur + kDyChunkBytes);
#pragma unroll
      for (int j = 0; j < 8; ++j) xf[j] = xl[(8 * (lane >> 4) + j) * kDyRank + (lane & 15)];
    }
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      bf16x8_t af;
      read_big_frag<kMNMajor, 4>(af, cur, fa, f, 0);
      read_big_frag<kMNMajor, 4>(af, cur, fa, f, 1);
      accb[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, xf, accb[f], 0, 0, 0);
    }
    // the four waves' P partials meet in LDS; element v of tile mt is row
    // 16 mt + 4 (lane / 16) + v, column lane % 16
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        pred[wave][(16 * mt + 4 * (lane >> 4) + v) * kDyRank + (lane & 15)] = accp[mt][v];
    __syncthreads();
#pragma unroll
    for (int e = tid; e < kDyChunk * kDyRank; e += 256) {
      const int row = m0 + kDyChunk * t + e / kDyRank;
      if (row < N)
        A.ppart[((int64_t)ct * N + row) * kDyRank + (e % kDyRank)] =
            (pred[0][e] + pred[1][e]) + (pred[2][e] + pred[3][e]);
    }
  }
  // dB partial: element v of tile f is column c0 + 64 w + 16 f + 4 (lane / 16) + v
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int col = c0 + 64 * wave + 16 * f + 4 * (lane >> 4) + v;
      if (col < O) A.dbpart[((int64_t)rt * O + col) * kDyRank + (lane & 15)] = accb[f][v];
    }
  __builtin_amdgcn_s_waitcnt(big::kWaitVm0);  // loads past the last chunk have landed
  __syncthreads();
}

// The fixed-order partial sums of a dY pass, every adapter's P (bf16) and dB
// (fp32) in one launch: blockIdx.y picks the job. Same arithmetic as
// reduce_partials_kernel (splits summed in order, then scaled); N = 16.
struct DyReduceJob {
  const float* part;
  int splits, rows;
  void* out;  // bf16 (P) or fp32 (dB), row stride ld
  int64_t ld;
  float scale;
  int out_f32;
};
struct DyReduceArgs {
  DyReduceJob job[2 * kDyMaxAdapters];
};

__global__ __launch_bounds__(256) void dy_reduce_kernel(const DyReduceArgs args) {
  const DyReduceJob& j = args.job[blockIdx.y];
  const int64_t total = (int64_t)j.rows * kDyRank;
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < total / 4;
       q += (int64_t)gridDim.x * 256) {
    const int64_t e = q * 4;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    int k = 0;
    for (; k + 4 <= j.splits; k += 4) {
      float v[4][4];
#pragma unroll
      for (int u = 0; u < 4; ++u) load_n<float, 4>(j.part + (int64_t)(k + u) * total + e, v[u]);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] += v[u][c];
    }
    for (; k < j.splits; ++k) {
      float v[4];
      load_n<float, 4>(j.part + (int64_t)k * total + e, v);
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] += v[c];
    }
    const int64_t m = e / kDyRank, n = e % kDyRank;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float r = j.scale * acc[c];
      if (j.out_f32)
        static_cast<float*>(j.out)[m * j.ld + n + c] = r;
      else
        static_cast<bf16*>(j.out)[m * j.ld + n + c] = from_f32<bf16>(r);
    }
  }
}

// Host side of the dY pass for up to three adapters of one layer. ws holds
// every adapter's partials; P_i (bf16, row stride ldp) and dB_i (fp32 [O_i,
// ldb_out]) receive s_i times the sums.
struct DyJob {
  const bf16* dy;
  int64_t ldy;
  int O;
  const bf16* b;
  int64_t ldb;
  const bf16* xa;
  int64_t ldxa;
  float scale;
  bf16* p;
  int64_t ldp;
  float* db;
  int64_t lddb;
};

inline size_t dy_pass_ws_bytes(int N, const int* O, int n) {
  size_t b = 0;
  for (int i = 0; i < n; ++i)
    b += align256(dy_ppart_bytes(N, O[i])) + align256(dy_dbpart_bytes(N, O[i]));
  return b;
}

inline int dy_pass(int N, const DyJob* jobs, int n, char* ws, size_t ws_bytes, hipStream_t st) {
  ML_CHECK(n >= 1 && n <= kDyMaxAdapters, "lora dY pass: 1..3 adapters");
  int O[kDyMaxAdapters];
  for (int i = 0; i < n; ++i) O[i] = jobs[i].O;
  ML_CHECK(dy_pass_ws_bytes(N, O, n) <= ws_bytes, "lora dY pass: workspace too small");
  DyArgs args{};
  args.nadp = n;
  args.N = N;
  int blocks = 0;
  char* w = ws;
  for (int i = 0; i < n; ++i) {
    const DyJob& j = jobs[i];
    ML_CHECK(j.O >= 8 && j.O % 8 == 0 && j.ldy % 8 == 0 && j.ldxa % 8 == 0,
             "lora dY pass: out features and strides must be multiples of 8");
    DyAdapter& a = args.ad[i];
    a.dy = j.dy;
    a.b = j.b;
    a.xa = j.xa;
    a.ldy = j.ldy;
    a.ldb = j.ldb;
    a.ldxa = j.ldxa;
    a.O = j.O;
    a.ctiles = dy_ctiles(j.O);
    a.first = blocks;
    a.ppart = reinterpret_cast<float*>(w);
    w += align256(dy_ppart_bytes(N, j.O));
    a.dbpart = reinterpret_cast<float*>(w);
    w += align256(dy_dbpart_bytes(N, j.O));
    blocks += a.ctiles * dy_rtiles(N);
  }
  dy_pass_kernel<<<dim3((unsigned)blocks), 256, 0, st>>>(args);
  ML_LAUNCH_CHECK();
  DyReduceArgs red{};
  for (int i = 0; i < n; ++i) {
    const DyJob& j = jobs[i];
    const DyAdapter& a = args.ad[i];
    red.job[2 * i] = DyReduceJob{a.ppart, a.ctiles, N, j.p, j.ldp, j.scale, 0};
    red.job[2 * i + 1] = DyReduceJob{a.dbpart, dy_rtiles(N), j.O, j.db, j.lddb, j.scale, 1};
  }
  dy_reduce_kernel<<<dim3(128, (unsigned)(2 * n)), 256, 0, st>>>(red);
  ML_LAUNCH_CHECK();
  return ML_OK;
}


// ------------------------------------------------------------- P^T X pass --
// dA = P^T X [RT, IN] for RT = 16, 32 or 48 stacked rank-16 adapters (X the
// saved input or h, P the rank-r products): one pass over X. A workgroup of
// 4 waves owns a 256 x 256 tile of X and streams it through LDS in chunks of
// 32 rows (global -> LDS, three chunks ahead; the same swizzled MN-major
// layout as the dY pass) with the chunk's 32 rows of P beside it. Per chunk,
// wave w: B = X columns 64 w .. 64 w + 63 (transposing reads), A = P^T (P
// rows read from LDS), RT / 16 x 4 MFMA tiles of fp32 accumulators kept over
// the tile's rows and written as the row tile's partial part[rtile][RT][IN];
// reduce_partials_kernel sums the row tiles in a fixed order.
constexpr int kPxRows = 256, kPxCols = 256, kPxChunk = 32, kPxStages = 4;

inline int px_rtiles(int N) { return (N + kPxRows - 1) / kPxRows; }
inline size_t ptx_pass_ws_bytes(int N, int RT, int IN) {
  return (size_t)px_rtiles(N) * RT * IN * sizeof(float);
}

template <int RT>
__global__ __launch_bounds__(256) void ptx_pass_kernel(const bf16* __restrict__ P, int64_t ldp,
                                                       const bf16* __restrict__ X, int64_t ldx,
                                                       int N, int IN, float* __restrict__ part) {
  constexpr int MT = RT / 16;
  constexpr int kXBytes = kPxChunk * kPxCols * 2;  // 16 KB
  constexpr int kPBytes = kPxChunk * RT * 2;        // 1 KB per 16 columns of P
  constexpr int kStage = kXBytes + kPBytes;
  constexpr int kPLoads = MT;  // 256-byte P loads per wave per chunk
  static_assert(kPBytes == 4 * kPLoads * 256, "P chunk in whole 256-byte loads");
  // 4 + kPLoads loads per wave per chunk; chunk t has landed once the two
  // chunks after it remain in flight
  constexpr int kWaitAhead = big::wait_vm(2 * (4 + kPLoads));
  __shared__ __attribute__((aligned(16))) char lds[kPxStages * kStage];
  const int ctiles = (IN + kPxCols - 1) / kPxCols;
  const int ct = blockIdx.x % ctiles, rt = blockIdx.x / ctiles;
  const int m0 = rt * kPxRows, c0 = ct * kPxCols;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rows = N - m0 < kPxRows ? N - m0 : kPxRows;
  const int nchunks = (rows + kPxChunk - 1) / kPxChunk;

  // X: group g = wave + 4 i covers chunk rows 2 g, 2 g + 1 (columns clamped
  // to the last valid 8); P: lane l of load j takes dword (4 j + w) 64 + l
  // of the chunk's rows (RT / 2 dwords per row).
  uint32_t xoff[4];
  int xrow[4];
  {
    const int p = lane & 31;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 2 * (wave + 4 * i) + (lane >> 5);
      const int h = (r & 3) | (((r >> 3) & 1) << 2);
      int e = 8 * (2 * ((p >> 1) ^ h) + (p & 1));
      e = c0 + e <= IN - 8 ? e : IN - 8 - c0;
      xoff[i] = (uint32_t)(((int64_t)r * ldx + c0 + e) * 2);
      xrow[i] = r;
    }
  }
  uint32_t poff[kPLoads];
  int prow[kPLoads];
#pragma unroll
  for (int j = 0; j < kPLoads; ++j) {
    const int d = (4 * j + wave) * 64 + lane;
    prow[j] = d / (RT / 2);
    poff[j] = (uint32_t)(((int64_t)prow[j] * ldp + 2 * (d % (RT / 2))) * 2);
  }
  auto chunk_loads = [&](int t, char* st) __attribute__((always_inline)) {
    const int rbase = m0 + kPxChunk * t;
    const rsrc_t rx = make_rsrc(reinterpret_cast<const char*>(X + (int64_t)rbase * ldx));
    const rsrc_t rp = make_rsrc(reinterpret_cast<const char*>(P + (int64_t)rbase * ldp));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = t < nchunks && rbase + xrow[i] < N;
      buf_load_lds(rx, ok ? xoff[i] : big::kOob, st + (wave + 4 * i) * 1024);
    }
#pragma unroll
    for (int j = 0; j < kPLoads; ++j) {
      const bool ok = t < nchunks && rbase + prow[j] < N;
      buf_load_lds_dword(rp, ok ? poff[j] : big::kOob, st + kXBytes + (4 * j + wave) * 256);
    }
  };

  FragAddr<kMNMajor, 4> fb;
  frag_addr_setup<kMNMajor, 4>(fb, 64 * wave, lane);
  f32x4_t acc[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int f = 0; f < 4; ++f) acc[mt][f] = f32x4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int j = 0; j < kPxStages - 1; ++j) chunk_loads(j, lds + j * kStage);
  for (int t = 0; t < nchunks; ++t) {
    const char* cur = lds + (t % kPxStages) * kStage;
    __builtin_amdgcn_s_waitcnt(kWaitAhead);
    __syncthreads();  // chunk t published; stage (t - 1) % 4 free
    chunk_loads(t + kPxStages - 1, lds + ((t + kPxStages - 1) % kPxStages) * kStage);
    bf16x8_t bx[4];
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      read_big_frag<kMNMajor, 4>(bx[f], cur, fb, f, 0);
      read_big_frag<kMNMajor, 4>(bx[f], cur, fb, f, 1);
    }
    // A = P^T: lane (m = r index 16 mt + lane % 16, k = chunk rows 8 (lane / 16) + j)
    const bf16* pl = reinterpret_cast<const bf16*>(cur + kXBytes);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      bf16x8_t a;
#pragma unroll
      for (int j = 0; j < 8; ++j) a[j] = pl[(8 * (lane >> 4) + j) * RT + 16 * mt + (lane & 15)];
#pragma unroll
      for (int f = 0; f < 4; ++f)
        acc[mt][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bx[f], acc[mt][f], 0, 0, 0);
    }
  }
  // element v of tile (mt, f): row 16 mt + 4 (lane / 16) + v, column
  // c0 + 64 w + 16 f + lane % 16
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int col = c0 + 64 * wave + 16 * f + (lane & 15);
        if (col < IN)
          part[((int64_t)rt * RT + 16 * mt + 4 * (lane >> 4) + v) * IN + col] = acc[mt][f][v];
      }
  __builtin_amdgcn_s_waitcnt(big::kWaitVm0);  // loads past the last chunk have landed
  __syncthreads();
}

// dA [RT, IN] (fp32, row stride ldda) = P^T X.
inline int ptx_pass(int N, const bf16* P, int64_t ldp, int RT, const bf16* X, int64_t ldx, int IN,
                    float* dA, int64_t ldda, char* ws, size_t ws_bytes, hipStream_t st) {
  ML_CHECK(RT == 16 || RT == 32 || RT == 48, "lora P^T X pass: 16, 32 or 48 rows (got %d)", RT);
  ML_CHECK(IN >= 8 && IN % 8 == 0 && ldx % 8 == 0 && ldp % 8 == 0,
           "lora P^T X pass: sizes and strides must be multiples of 8");
  ML_CHECK(ptx_pass_ws_bytes(N, RT, IN) <= ws_bytes, "lora P^T X pass: workspace too small");
  float* part = reinterpret_cast<float*>(ws);
  const unsigned blocks = (unsigned)(px_rtiles(N) * ((IN + kPxCols - 1) / kPxCols));
  if (RT == 16)
    ptx_pass_kernel<16><<<dim3(blocks), 256, 0, st>>>(P, ldp, X, ldx, N, IN, part);
  else if (RT == 32)
    ptx_pass_kernel<32><<<dim3(blocks), 256, 0, st>>>(P, ldp, X, ldx, N, IN, part);
  else
    ptx_pass_kernel<48><<<dim3(blocks), 256, 0, st>>>(P, ldp, X, ldx, N, IN, part);
  ML_LAUNCH_CHECK();
  reduce_partials_kernel<float><<<dim3(256), 256, 0, st>>>(part, px_rtiles(N), RT, IN, dA, ldda,
                                                           1.0f, 0.f);
  ML_LAUNCH_CHECK();
  return ML_OK;
}

// -------------------------------------------- MLP SwiGLU backward pass --
// The MLP backward's middle, rank 16, in one pass over dH [N, I]: the SwiGLU
// backward and the three rank-16 products that read its inputs or outputs,
//   d_gate, d_up = SwiGLU'(gate, up) dH   (stored; d_gate over dH in place)
//   P_G, dB_G    = s_G d_gate B_G, s_G d_gate^T XA_G     (as the dY pass)
//   P_U, dB_U    = s_U d_up B_U,   s_U d_up^T XA_U
//   dA_D         = P_D^T h                               (as the P^T X pass)
// instead of a SwiGLU backward, a dY pass over d_gate / d_up and a P^T X
// pass over h (which read d_gate / d_up back from HBM and take 5 launches).
// A workgroup of 4 waves owns a 256 x 256 tile and walks it in chunks of 32
// rows. Per chunk each thread loads one 16-byte vector of dH, gate, up and h
// from each of 4 rows (rows t / 32 + 8 i, columns 8 (t % 32) ..) - the next
// chunk's loads are in flight while the current chunk's MFMAs run - forms
// d_gate / d_up with the SwiGLU kernels' element math, stores them, and
// writes d_gate, d_up and h into LDS in the dY pass's MN-major layout (the
// 32-byte unit u of row r at u ^ h(r)), beside the chunk's XA and P_D rows.
// The MFMA work, the partial layouts and the fixed-order reduction are the
// dY pass's and the P^T X pass's, so the results equal theirs bit for bit.
// Rows past N and columns past I enter as zeros and are not stored.
constexpr int kMidD = 0;                                // d_gate chunk
constexpr int kMidU = kDyChunkBytes;                    // d_up chunk
constexpr int kMidH = 2 * kDyChunkBytes;                // h chunk; then the P meets
constexpr int kMidXa = 3 * kDyChunkBytes;               // XA_G [32][16], XA_U [32][16]
constexpr int kMidPd = kMidXa + 2 * kDyXaBytes;         // P_D [32][16]
constexpr int kMidBytes = kMidPd + kDyXaBytes;          // 51 KB: three workgroups per CU
constexpr int kMidMeetBytes = 4 * kDyChunk * kDyRank * 4;  // one adapter's P meet
static_assert(2 * kMidMeetBytes <= kDyChunkBytes, "both P meets fit in the h region");

struct MlpMidArgs {
  bf16* dh;  // [N, I]: dH in, d_gate out
  bf16* dup;  // [N, I]
  const bf16* gate;
  const bf16* up;
  const bf16* h;   // [N, I] each, dense (h: unused when the kernel recomputes it)
  const bf16* xa;  // [N, 32]: XA_G | XA_U, row stride ldxa
  const bf16* pd;  // [N, 16]: P_D, row stride ldpd
  const bf16* b[2];  // B_G, B_U [I, 16], row stride ldb
  float* ppart[2];   // [ctiles][N][16]
  float* dbpart[2];  // [rtiles][I][16]
  float* dapart;     // [rtiles][16][I]
  int64_t ldxa, ldpd, ldb;
  int N, I, ctiles;
};

__device__ __forceinline__ int mn_swz(int r) { return (r & 3) | (((r >> 3) & 1) << 2); }

// 16 bytes or zeros, as a vector select (a select between two structs would
// go through scratch memory)
__device__ __forceinline__ u32x4_t keep16(bool ok, u32x4_t v) {
  return ok ? v : u32x4_t{0u, 0u, 0u, 0u};
}

// RH: h = silu(gate) up is recomputed from the gate / up vectors (rounded to
// bf16 as the SwiGLU forward rounds it) instead of read.
template <bool RH>
__global__ __launch_bounds__(256) void mlp_mid_kernel(const MlpMidArgs args) {
  typedef Pack<bf16, 8> V8;
  __shared__ __attribute__((aligned(16))) char lds[kMidBytes];
  const int ct = blockIdx.x % args.ctiles, rt = blockIdx.x / args.ctiles;
  const int m0 = rt * kDyRows, c0 = ct * kDyCols;
  const int N = args.N, I = args.I;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rows = N - m0 < kDyRows ? N - m0 : kDyRows;
  const int nchunks = (rows + kDyChunk - 1) / kDyChunk;

  // B fragments of this wave's two k-steps, as in the dY pass: the tile's
  // B_G / B_U rows [256][16] are staged through the (still unused) h region
  // with 16-byte loads, rows past I as zeros.
  bf16x8_t bfr[2][2];
  {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // 16-byte vector v: adapter v / 512 (= q / 2), row (v / 2) % 256, half v % 2
      const int v = tid + 256 * q;
      const int row = (v >> 1) & 255, c = c0 + row;
      const bf16* src = args.b[q >> 1];
      const u32x4_t x = *reinterpret_cast<const u32x4_t*>(
          src + (int64_t)(c < I ? c : I - 1) * args.ldb + 8 * (v & 1));
      *reinterpret_cast<u32x4_t*>(lds + kMidH + 16 * v) = keep16(c < I, x);
    }
    __syncthreads();
    const bf16* bl = reinterpret_cast<const bf16*>(lds + kMidH);
#pragma unroll
    for (int ad = 0; ad < 2; ++ad)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int cb = 64 * wave + 32 * ks + 8 * (lane >> 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) bfr[ad][ks][j] = bl[(ad * 256 + cb + j) * kDyRank + (lane & 15)];
      }
  }

  // This thread's vectors: chunk rows (tid / 32) + 8 i, columns cc .. cc + 7
  // (a column group past I reads the last valid one and is zeroed).
  const int cg = tid & 31;
  const int cc = c0 + 8 * cg;
  const bool okc = cc < I;
  const int ccl = okc ? cc : I - 8;
  uint32_t ldsoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rq = (tid >> 5) + 8 * i;
    ldsoff[i] = (uint32_t)(rq * 512 + ((((cg >> 1) ^ mn_swz(rq)) << 5) | ((cg & 1) << 4)));
  }
  // The chunk's small rows: threads 0..127 one 16-byte quarter of an XA_GU
  // row (row tid / 4), threads 128..191 one half of a P_D row; the others
  // load P_D's first vector again and store nothing (every thread loads, so
  // that no load sits in a branch the compiler would wait for).
  const int srow = tid < 128 ? (tid >> 2) : tid < 192 ? ((tid - 128) >> 1) : 0;
  const bool sxa = tid < 128;
  const bf16* sbase = sxa ? args.xa : args.pd;
  const int64_t sld = sxa ? args.ldxa : args.ldpd;
  const int scol = sxa ? 8 * (tid & 3) : tid < 192 ? 8 * (tid & 1) : 0;
  const uint32_t sdst =
      sxa ? (uint32_t)(kMidXa + ((tid & 3) >> 1) * kDyXaBytes + srow * 32 + (tid & 1) * 16)
          : (uint32_t)(kMidPd + srow * 32 + (tid & 1) * 16);

  // The [N, I] operands share one layout: a chunk's vectors are addressed
  // as a uniform chunk base plus a 32-bit byte offset per row (the host
  // checks N I < 2^31), one VGPR each instead of a 64-bit address per load.
  auto nt16 = [](const bf16* base, int64_t chunk_bytes, uint32_t off) __attribute__((always_inline)) {
    return __builtin_nontemporal_load(
        reinterpret_cast<const u32x4_t*>(reinterpret_cast<const char*>(base) + chunk_bytes + off));
  };
  u32x4_t vd[4], vg[4], vu[4], vh[4], vs;
  auto load_chunk = [&](int t) __attribute__((always_inline)) {
    const int rb = m0 + kDyChunk * t;
    const int64_t cb = (int64_t)rb * I * 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rq = (tid >> 5) + 8 * i;
      const int rr = rb + rq < N ? rq : N - 1 - rb;  // rows past N re-read the last row
      const uint32_t off = (uint32_t)(rr * I + ccl) * 2u;
      vd[i] = nt16(args.dh, cb, off);
      vg[i] = nt16(args.gate, cb, off);
      vu[i] = nt16(args.up, cb, off);
      if constexpr (!RH) vh[i] = nt16(args.h, cb, off);
    }
    const int r = rb + srow;
    vs = *reinterpret_cast<const u32x4_t*>(sbase + (int64_t)(r < N ? r : N - 1) * sld + scol);
  };

  FragAddr<kMNMajor, 4> fa;
  frag_addr_setup<kMNMajor, 4>(fa, 64 * wave, lane);
  f32x4_t accb[2][4], acca[4];
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    accb[0][f] = accb[1][f] = acca[f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  load_chunk(0);
  for (int t = 0; t < nchunks; ++t) {
    const int rb = m0 + kDyChunk * t;
    __syncthreads();  // the previous chunk's LDS reads are done
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rb + (tid >> 5) + 8 * i;
      const bool ok = okc && r < N;
      const V8 g8 = __builtin_bit_cast(V8, vg[i]), u8 = __builtin_bit_cast(V8, vu[i]),
               y8 = __builtin_bit_cast(V8, vd[i]);
      V8 pg, pu, ph;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float dgf, duf, hf;
        if constexpr (RH) {
          swiglu_bwd_fwd_elem(to_f32(g8.v[e]), to_f32(u8.v[e]), to_f32(y8.v[e]), dgf, duf, hf);
          ph.v[e] = from_f32<bf16>(hf);
        } else {
          swiglu_bwd_elem(to_f32(g8.v[e]), to_f32(u8.v[e]), to_f32(y8.v[e]), dgf, duf);
        }
        pg.v[e] = from_f32<bf16>(dgf);
        pu.v[e] = from_f32<bf16>(duf);
      }
      if constexpr (RH) vh[i] = __builtin_bit_cast(u32x4_t, ph);
      const u32x4_t xg = __builtin_bit_cast(u32x4_t, pg), xu = __builtin_bit_cast(u32x4_t, pu);
      if (ok) {
        const int64_t cb = (int64_t)rb * I * 2;
        const uint32_t off = (uint32_t)(((tid >> 5) + 8 * i) * I + cc) * 2u;
        __builtin_nontemporal_store(
            xg, reinterpret_cast<u32x4_t*>(reinterpret_cast<char*>(args.dh) + cb + off));
        __builtin_nontemporal_store(
            xu, reinterpret_cast<u32x4_t*>(reinterpret_cast<char*>(args.dup) + cb + off));
      }
      *reinterpret_cast<u32x4_t*>(lds + kMidD + ldsoff[i]) = keep16(ok, xg);
      *reinterpret_cast<u32x4_t*>(lds + kMidU + ldsoff[i]) = keep16(ok, xu);
      *reinterpret_cast<u32x4_t*>(lds + kMidH + ldsoff[i]) = keep16(ok, vh[i]);
      // one vector at a time: interleaved, the four vectors' fp32 operands
      // would need 96 VGPRs
      __builtin_amdgcn_sched_barrier(0);
    }
    if (tid < 192) *reinterpret_cast<u32x4_t*>(lds + sdst) = keep16(rb + srow < N, vs);
    // the next chunk's loads go out only after this chunk's vectors are
    // consumed (hoisted above, both chunks' 64 VGPRs would be live at once)
    asm volatile("" ::: "memory");
    if (t + 1 < nchunks) load_chunk(t + 1);
    __syncthreads();  // chunk t published

    // dA_D: A = P_D^T (rows of the chunk's P_D), B = h, as the P^T X pass
    {
      const bf16* pl = reinterpret_cast<const bf16*>(lds + kMidPd);
      bf16x8_t a;
#pragma unroll
      for (int j = 0; j < 8; ++j) a[j] = pl[(8 * (lane >> 4) + j) * kDyRank + (lane & 15)];
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        bf16x8_t bx;
        read_big_frag<kMNMajor, 4>(bx, lds + kMidH, fa, f, 0);
        read_big_frag<kMNMajor, 4>(bx, lds + kMidH, fa, f, 1);
        acca[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bx, acca[f], 0, 0, 0);
      }
    }
    __syncthreads();  // every wave is done with the h region, which takes the P meets
#pragma unroll
    for (int ad = 0; ad < 2; ++ad) {
      const char* cur = lds + (ad == 0 ? kMidD : kMidU);
      // P, as the dY pass; the four waves' partials meet in LDS (element v
      // of tile mt: row 16 mt + 4 (lane / 16) + v, column lane % 16)
      float* pred = reinterpret_cast<float*>(lds + kMidH + ad * kMidMeetBytes);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int r = 16 * mt + (lane & 15);
        const int h = mn_swz(r);
        f32x4_t accp = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const int c = 64 * wave + 32 * ks + 8 * (lane >> 4);
          const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(
              cur + r * 512 + (((c >> 4) ^ h) << 5) + (c & 15) * 2);
          accp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bfr[ad][ks], accp, 0, 0, 0);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v)
          pred[wave * (kDyChunk * kDyRank) + (16 * mt + 4 * (lane >> 4) + v) * kDyRank +
               (lane & 15)] = accp[v];
      }
      // dB, as the dY pass
      bf16x8_t xf;
      const bf16* xl = reinterpret_cast<const bf16*>(lds + kMidXa + ad * kDyXaBytes);
#pragma unroll
      for (int j = 0; j < 8; ++j) xf[j] = xl[(8 * (lane >> 4) + j) * kDyRank + (lane & 15)];
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        bf16x8_t af;
        read_big_frag<kMNMajor, 4>(af, cur, fa, f, 0);
        read_big_frag<kMNMajor, 4>(af, cur, fa, f, 1);
        accb[ad][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, xf, accb[ad][f], 0, 0, 0);
      }
    }
    __syncthreads();  // the P meets are complete
#pragma unroll
    for (int ad = 0; ad < 2; ++ad) {
      const float* pred = reinterpret_cast<const float*>(lds + kMidH + ad * kMidMeetBytes);
      constexpr int W = kDyChunk * kDyRank;
#pragma unroll
      for (int e = tid; e < W; e += 256) {
        const int row = rb + e / kDyRank;
        if (row < N)
          args.ppart[ad][((int64_t)ct * N + row) * kDyRank + (e % kDyRank)] =
              (pred[e] + pred[W + e]) + (pred[2 * W + e] + pred[3 * W + e]);
      }
    }
  }
  // dB partials (element v of tile f: column c0 + 64 w + 16 f + 4 (lane / 16) + v)
  // and the dA partial (row 4 (lane / 16) + v, column c0 + 64 w + 16 f + lane % 16)
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int col = c0 + 64 * wave + 16 * f + 4 * (lane >> 4) + v;
      if (col < I) {
#pragma unroll
        for (int ad = 0; ad < 2; ++ad)
          args.dbpart[ad][((int64_t)rt * I + col) * kDyRank + (lane & 15)] = accb[ad][f][v];
      }
      const int cola = c0 + 64 * wave + 16 * f + (lane & 15);
      if (cola < I)
        args.dapart[((int64_t)rt * kDyRank + 4 * (lane >> 4) + v) * I + cola] = acca[f][v];
    }
}

// The fused pass's dA_D partials: one [16, I] fp32 block per row tile of the
// pass itself (its row tiles are the dY pass's, not the P^T X pass's).
inline size_t mlp_mid_dapart_bytes(int N, int I) {
  return (size_t)dy_rtiles(N) * kDyRank * I * sizeof(float);
}

inline size_t mlp_mid_ws_bytes(int N, int I) {
  const int O[2] = {I, I};
  return dy_pass_ws_bytes(N, O, 2) + align256(mlp_mid_dapart_bytes(N, I));
}

// Whether the fused pass takes these operands (16-byte aligned vectors).
inline bool mlp_mid_ok(int I, const void* const* ptrs, int n, int64_t ldxa, int64_t ldpd) {
  if (I < 8 || I % 8 != 0 || ldxa % 8 != 0 || ldpd % 8 != 0) return false;
  for (int i = 0; i < n; ++i)
    if (!aligned16(ptrs[i])) return false;
  return true;
}

// Host side: d_gate (over dH) and d_up; P_G, P_U (bf16, s times the sums,
// row stride ldp) and dB_G, dB_U (fp32 [I, lddb]); dA_D (fp32 [16, I], row
// stride I). h null: recomputed from gate and up.
inline int mlp_mid_pass(int N, int I, bf16* dh, bf16* dup, const bf16* gate, const bf16* up,
                        const bf16* h, const bf16* xa, int64_t ldxa, const bf16* pd,
                        int64_t ldpd, const bf16* bg, const bf16* bu, int64_t ldb, float sg,
                        float su, bf16* pg, bf16* pu, int64_t ldp, float* dbg, float* dbu,
                        int64_t lddb, float* da, char* ws, size_t ws_bytes, hipStream_t st) {
  ML_CHECK(mlp_mid_ws_bytes(N, I) <= ws_bytes, "lora mlp pass: workspace too small");
  MlpMidArgs a{};
  a.dh = dh;
  a.dup = dup;
  a.gate = gate;
  a.up = up;
  a.h = h;
  a.xa = xa;
  a.pd = pd;
  a.b[0] = bg;
  a.b[1] = bu;
  a.ldxa = ldxa;
  a.ldpd = ldpd;
  a.ldb = ldb;
  a.N = N;
  a.I = I;
  a.ctiles = dy_ctiles(I);
  char* w = ws;
  for (int ad = 0; ad < 2; ++ad) {
    a.ppart[ad] = reinterpret_cast<float*>(w);
    w += align256(dy_ppart_bytes(N, I));
    a.dbpart[ad] = reinterpret_cast<float*>(w);
    w += align256(dy_dbpart_bytes(N, I));
  }
  a.dapart = reinterpret_cast<float*>(w);
  const unsigned blocks = (unsigned)(a.ctiles * dy_rtiles(N));
  if (h)
    mlp_mid_kernel<false><<<dim3(blocks), 256, 0, st>>>(a);
  else
    mlp_mid_kernel<true><<<dim3(blocks), 256, 0, st>>>(a);
  ML_LAUNCH_CHECK();
  DyReduceArgs red{};
  red.job[0] = DyReduceJob{a.ppart[0], a.ctiles, N, pg, ldp, sg, 0};
  red.job[1] = DyReduceJob{a.dbpart[0], dy_rtiles(N), I, dbg, lddb, sg, 1};
  red.job[2] = DyReduceJob{a.ppart[1], a.ctiles, N, pu, ldp, su, 0};
  red.job[3] = DyReduceJob{a.dbpart[1], dy_rtiles(N), I, dbu, lddb, su, 1};
  // dA_D [16, I] dense: the same flat index in the partials and the output
  red.job[4] = DyReduceJob{a.dapart, dy_rtiles(N), I, da, kDyRank, 1.0f, 1};
  dy_reduce_kernel<<<dim3(128, 5), 256, 0, st>>>(red);
  ML_LAUNCH_CHECK();
  return ML_OK;
}

// ------------------------------------------------------------------ X A^T --
// XA [N, R] = X [N, K] A^T for the adapters' stacked A matrices (A [R, K],
// R <= 64): the LoRA forwards' rank-r products (F.linear(x, A) of
// ops/fused_lora.py:79-81). A workgroup of 4 waves owns 32 rows of X; wave w
// takes the w-th quarter of the k range in steps of 32, with the MFMA
// operands loaded straight from global memory in their register layout
// (lane l: 16 bytes of row l % 16 at k offset 8 (l / 16)), and the four
// waves' [32, 16 NT] fp32 sums meet in LDS in a fixed order before the bf16
// store. X is read once from HBM, A (<= 256 KB) from L2; no split-K partials
// and no second launch. Rows past N and columns past R are not stored;
// lanes whose k lies past K contribute zeros (K % 8 == 0).
constexpr int kXaRows = 32;

template <int NT>
__global__ __launch_bounds__(256) void xa_kernel(const bf16* __restrict__ X, int64_t ldx,
                                                 const bf16* __restrict__ A, int64_t lda, int N,
                                                 int K, int R, bf16* __restrict__ XA,
                                                 int64_t ldo) {
  constexpr int W = kXaRows * 16 * NT;  // one wave's sums
  __shared__ float red[4 * W];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m0 = blockIdx.x * kXaRows;
  const int ksteps = (K + 31) / 32;
  const int per = (ksteps + 3) / 4;
  const int kb = wave * per, ke = kb + per < ksteps ? kb + per : ksteps;
  const int lr = lane & 15, lk = 8 * (lane >> 4);
  // row starts (rows past N / R re-read the last row and are not stored)
  const bf16* x0 = X + (int64_t)(m0 + lr < N ? m0 + lr : N - 1) * ldx;
  const bf16* x1 = X + (int64_t)(m0 + 16 + lr < N ? m0 + 16 + lr : N - 1) * ldx;
  const bf16* ap[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) ap[j] = A + (int64_t)(16 * j + lr < R ? 16 * j + lr : R - 1) * lda;
  f32x4_t acc[2][NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[0][j] = acc[1][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const bf16x8_t zero = bf16x8_t{};
  // groups of 4 k-steps: every load of a group is in flight before its MFMAs
  // (steps past this wave's range load in-range data and are zeroed)
  for (int s0 = kb; s0 < ke; s0 += 4) {
    bf16x8_t a0[4], a1[4], b[4][NT];
    bool ok[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = 32 * (s0 + u);
      ok[u] = s0 + u < ke && k + lk < K;
      const int kc = ok[u] ? k + lk : 0;  // lanes past K read the row's first 8
      a0[u] = *reinterpret_cast<const bf16x8_t*>(x0 + kc);
      a1[u] = *reinterpret_cast<const bf16x8_t*>(x1 + kc);
#pragma unroll
      for (int j = 0; j < NT; ++j) b[u][j] = *reinterpret_cast<const bf16x8_t*>(ap[j] + kc);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const bf16x8_t p0 = ok[u] ? a0[u] : zero, p1 = ok[u] ? a1[u] : zero;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const bf16x8_t q = ok[u] ? b[u][j] : zero;
        acc[0][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p0, q, acc[0][j], 0, 0, 0);
        acc[1][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p1, q, acc[1][j], 0, 0, 0);
      }
    }
  }
  // element v of tile (t, j): row 16 t + 4 (lane / 16) + v, column 16 j + lane % 16
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        red[wave * W + (16 * t + 4 * (lane >> 4) + v) * (16 * NT) + 16 * j + lr] = acc[t][j][v];
  __syncthreads();
  for (int e = tid; e < W; e += 256) {
    const int row = m0 + e / (16 * NT), col = e % (16 * NT);
    if (row < N && col < R)
      XA[(int64_t)row * ldo + col] =
          from_f32<bf16>((red[e] + red[W + e]) + (red[2 * W + e] + red[3 * W + e]));
  }
}

}  // namespace
}  // namespace lora
}  // namespace mla

using namespace mla;
using namespace mla::gemm;

// ----------------------------------------------------------------- X A^T --

extern "C" int ml_lora_xa(const void* X, int64_t n_tokens, int64_t in_features, int64_t ldx,
                          const void* A, int64_t rank_total, void* XA, int64_t ldo,
                          void* stream) {
  ML_CHECK(n_tokens >= 0 && n_tokens < (1LL << 31), "lora xa: bad token count");
  ML_CHECK(in_features >= 8 && in_features % 8 == 0 && in_features < (1LL << 31),
           "lora xa: in_features must be a positive multiple of 8");
  ML_CHECK(rank_total >= 1 && rank_total <= 64, "lora xa: 1..64 stacked rank rows (got %lld)",
           (long long)rank_total);
  ML_CHECK(ldx >= in_features && ldx % 8 == 0 && ldo >= rank_total,
           "lora xa: bad leading dimensions");
  if (n_tokens == 0) return ML_OK;  // (an empty X may have no storage)
  ML_CHECK(X && A && XA, "lora xa: null pointer");
  ML_CHECK(aligned16(X) && aligned16(A), "lora xa: X and A must be 16-byte aligned");
  const int N = (int)n_tokens, K = (int)in_features, R = (int)rank_total;
  const dim3 grid((unsigned)((N + lora::kXaRows - 1) / lora::kXaRows));
  hipStream_t st = (hipStream_t)stream;
  const bf16* x = static_cast<const bf16*>(X);
  const bf16* a = static_cast<const bf16*>(A);
  bf16* o = static_cast<bf16*>(XA);
  switch ((R + 15) / 16) {
    case 1: lora::xa_kernel<1><<<grid, 256, 0, st>>>(x, ldx, a, K, N, K, R, o, ldo); break;
    case 2: lora::xa_kernel<2><<<grid, 256, 0, st>>>(x, ldx, a, K, N, K, R, o, ldo); break;
    case 3: lora::xa_kernel<3><<<grid, 256, 0, st>>>(x, ldx, a, K, N, K, R, o, ldo); break;
    default: lora::xa_kernel<4><<<grid, 256, 0, st>>>(x, ldx, a, K, N, K, R, o, ldo); break;
  }
  ML_LAUNCH_CHECK();
  return ML_OK;
}

// ------------------------------------------------------------------- QKV --

static size_t qkv_partial_bytes(int64_t N, int64_t in_f, const int64_t* out_f, int nadp,
                                int64_t r) {
  size_t m = lora::skinny_ws<WideCfg>((int)(nadp * r), (int)in_f, (int)N);
  if (r == lora::kDyRank) {
    int O[3];
    for (int i = 0; i < nadp; ++i) O[i] = (int)out_f[i];
    m = std::max(m, lora::ptx_pass_ws_bytes((int)N, (int)(nadp * r), (int)in_f));
    return std::max(m, lora::dy_pass_ws_bytes((int)N, O, nadp));
  }
  for (int i = 0; i < nadp; ++i) {
    m = std::max(m, lora::skinny_ws<TallCfg>((int)N, (int)r, (int)out_f[i]));
    m = std::max(m, lora::skinny_ws<TallCfg>((int)out_f[i], (int)r, (int)N));
  }
  return m;
}

// Backward of nadp (1..3) adapters that share the input X: P_i and dB_i by
// one pass over each dY_i (rank 16) or split-K skinny products, dA = P^T X,
// and dX = [dY_1 | ... | P] [W_1; ...; A_stack] as one K-concatenated GEMM.
static size_t adapters_bwd_ws_bytes(int64_t N, int64_t IN, const int64_t* out_f, int nadp,
                                    int64_t r) {
  return lora::align256((size_t)(N * nadp * r) * 2) + qkv_partial_bytes(N, IN, out_f, nadp, r);
}

static int adapters_bwd(const char* what, int nadp, const void* X, int64_t n_tokens,
                        int64_t in_features, const void* const* dY, const int64_t* out_features,
                        const void* const* W, const void* A_stack, const void* const* B,
                        const float* scale, const void* XA, int64_t rank, void* dX, float* dA,
                        float* const* dB, void* workspace, size_t workspace_bytes,
                        hipStream_t st) {
  ML_CHECK(n_tokens > 0 && in_features > 0 && rank > 0, "%s: bad sizes", what);
  ML_CHECK(n_tokens < (1LL << 31) && in_features < (1LL << 31), "%s: sizes too large", what);
  ML_CHECK(in_features % 8 == 0 && rank % 8 == 0,
           "%s: in_features and rank must be multiples of 8", what);
  ML_CHECK(X && dY && out_features && W && A_stack && B && scale && XA && dX && dA && dB,
           "%s: null pointer", what);
  for (int i = 0; i < nadp; ++i) {
    ML_CHECK(dY[i] && W[i] && B[i] && dB[i], "%s: null pointer for adapter %d", what, i);
    ML_CHECK(out_features[i] > 0 && out_features[i] % 8 == 0 && out_features[i] < (1LL << 31),
             "%s: out_features[%d] must be a positive multiple of 8", what, i);
  }
  const size_t need = adapters_bwd_ws_bytes(n_tokens, in_features, out_features, nadp, rank);
  ML_CHECK(aligned16(dX), "%s: dX must be 16-byte aligned (it is written as 16-byte rows)",
           what);
  ML_CHECK(workspace && workspace_bytes >= need, "%s: workspace too small (%zu < %zu)", what,
           workspace_bytes, need);
  const int N = (int)n_tokens, IN = (int)in_features, R = (int)rank, RS = nadp * (int)rank;
  char* ws = static_cast<char*>(workspace);
  bf16* P = reinterpret_cast<bf16*>(ws);  // [N, nadp r], column block i = s_i dY_i B_i
  float* part = reinterpret_cast<float*>(ws + lora::align256((size_t)N * RS * 2));
  const size_t part_bytes = workspace_bytes - lora::align256((size_t)N * RS * 2);
  const bf16* x = static_cast<const bf16*>(X);
  const bf16* xa = static_cast<const bf16*>(XA);
  int rc;
  if (R == lora::kDyRank) {
    // P_i and dB_i of every adapter: one pass over each dY_i
    lora::DyJob jobs[3];
    for (int i = 0; i < nadp; ++i)
      jobs[i] = lora::DyJob{static_cast<const bf16*>(dY[i]), out_features[i],
                            (int)out_features[i], static_cast<const bf16*>(B[i]), R, xa + i * R,
                            RS, scale[i], P + i * R, RS, dB[i], R};
    rc = lora::dy_pass(N, jobs, nadp, reinterpret_cast<char*>(part), part_bytes, st);
    if (rc) return rc;
  }
  for (int i = 0; i < nadp && R != lora::kDyRank; ++i) {
    const int OUT = (int)out_features[i];
    const bf16* dy = static_cast<const bf16*>(dY[i]);
    // P_i = s_i dY_i B_i: A = dY_i [N, out] K-major, B = B_i [out, r] (k = out, n = r) MN-major
    Segment sp{{dy, OUT}, {static_cast<const bf16*>(B[i]), R}, OUT};
    rc = lora::skinny<TallCfg, kKMajor, kMNMajor, bf16>(N, R, sp, P + i * R, RS, scale[i], part,
                                                         part_bytes, st);
    if (rc) return rc;
    // dB_i = s_i dY_i^T XA_i: A = dY_i^T (MN-major, ld out), B = XA_i (MN-major, ld nadp r)
    Segment sb{{dy, OUT}, {xa + i * R, RS}, N};
    rc = lora::skinny<TallCfg, kMNMajor, kMNMajor, float>(OUT, R, sb, dB[i], R, scale[i], part,
                                                           part_bytes, st);
    if (rc) return rc;
  }
  // dA_stack = P^T X: A = P^T (MN-major, ld nadp r), B = X (MN-major, ld in)
  if (R == lora::kDyRank) {
    rc = lora::ptx_pass(N, P, RS, RS, x, IN, IN, dA, IN, reinterpret_cast<char*>(part), part_bytes,
                        st);
  } else {
    Segment sa{{P, RS}, {x, IN}, N};
    rc = lora::skinny<WideCfg, kMNMajor, kMNMajor, float>(RS, IN, sa, dA, IN, 1.0f, part,
                                                           part_bytes, st);
  }
  if (rc) return rc;
  // dX = [dY_1 | ... | dY_nadp | P] [W_1; ...; W_nadp; A_stack]
  Segment segs[4];
  for (int i = 0; i < nadp; ++i)
    segs[i] = Segment{{static_cast<const bf16*>(dY[i]), out_features[i]},
                      {static_cast<const bf16*>(W[i]), IN}, (int)out_features[i]};
  segs[nadp] = Segment{{P, RS}, {static_cast<const bf16*>(A_stack), IN}, RS};
  Problem pb;
  rc = make_problem<BigCfg>(pb, N, IN, nadp + 1, segs, kKMajor, kMNMajor, 0);
  if (rc) return rc;
  return launch_store<bf16, R4Cfg>(pb, kKMajor, kMNMajor, dX, IN, 1.0f, 0.0f, st);
}

extern "C" size_t ml_lora_qkv_bwd_workspace_bytes(int64_t n_tokens, int64_t in_features,
                                                  const int64_t* out_features, int64_t rank) {
  if (n_tokens <= 0 || in_features <= 0 || rank <= 0 || !out_features) return 0;
  return adapters_bwd_ws_bytes(n_tokens, in_features, out_features, 3, rank);
}

extern "C" int ml_lora_qkv_bwd(const void* X, int64_t n_tokens, int64_t in_features,
                               const void* const* dY, const int64_t* out_features,
                               const void* const* W, const void* A_stack, const void* const* B,
                               const float* scale, const void* XA, int64_t rank, void* dX,
                               float* dA, float* const* dB, void* workspace,
                               size_t workspace_bytes, void* stream) {
  return adapters_bwd("lora qkv", 3, X, n_tokens, in_features, dY, out_features, W, A_stack, B,
                      scale, XA, rank, dX, dA, dB, workspace, workspace_bytes,
                      (hipStream_t)stream);
}

// ------------------------------------------------------ single projection --

extern "C" size_t ml_lora_linear_bwd_workspace_bytes(int64_t n_tokens, int64_t in_features,
                                                     int64_t out_features, int64_t rank) {
  if (n_tokens <= 0 || in_features <= 0 || rank <= 0 || out_features <= 0) return 0;
  return adapters_bwd_ws_bytes(n_tokens, in_features, &out_features, 1, rank);
}

extern "C" int ml_lora_linear_bwd(const void* X, int64_t n_tokens, int64_t in_features,
                                  const void* dY, int64_t out_features, const void* W,
                                  const void* A, const void* B, float scale, const void* XA,
                                  int64_t rank, void* dX, float* dA, float* dB, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  const void* dys[1] = {dY};
  const void* ws_[1] = {W};
  const void* bs[1] = {B};
  float* dbs[1] = {dB};
  return adapters_bwd("lora linear", 1, X, n_tokens, in_features, dys, &out_features, ws_, A, bs,
                      &scale, XA, rank, dX, dA, dbs, workspace, workspace_bytes,
                      (hipStream_t)stream);
}

// ------------------------------------------------------------------- MLP --

static size_t mlp_partial_bytes(int64_t N, int64_t H, int64_t I, int64_t r) {
  size_t m = lora::skinny_ws<TallCfg>((int)N, (int)r, (int)H);          // P_D
  m = std::max(m, lora::skinny_ws<WideCfg>((int)r, (int)I, (int)N));   // dA_D
  m = std::max(m, lora::skinny_ws<TallCfg>((int)H, (int)r, (int)N));   // dB_D
  m = std::max(m, lora::skinny_ws<TallCfg>((int)N, (int)r, (int)I));   // P_G, P_U
  m = std::max(m, lora::skinny_ws<WideCfg>((int)(2 * r), (int)H, (int)N));  // dA_GU
  m = std::max(m, lora::skinny_ws<TallCfg>((int)I, (int)r, (int)N));   // dB_G, dB_U
  if (r == lora::kDyRank) {
    const int OD[1] = {(int)H}, OGU[2] = {(int)I, (int)I};
    m = std::max(m, lora::dy_pass_ws_bytes((int)N, OD, 1));
    m = std::max(m, lora::dy_pass_ws_bytes((int)N, OGU, 2));
    m = std::max(m, lora::ptx_pass_ws_bytes((int)N, (int)r, (int)I));
    m = std::max(m, lora::ptx_pass_ws_bytes((int)N, (int)(2 * r), (int)H));
    m = std::max(m, lora::mlp_mid_ws_bytes((int)N, (int)I));
  }
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
  ML_CHECK(X && gate && up && dY && WG && WU && WD && A_GU && A_D && BG && BU && BD && scale &&
               XA_GU && hA_D && dX && dA_GU && dA_D && dB_G && dB_U && dB_D,
           "lora mlp: null pointer");
  ML_CHECK(aligned16(dX), "lora mlp: dX must be 16-byte aligned (it is written as 16-byte rows)");
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
  const bf16* xa = static_cast<const bf16*>(XA_GU);
  int rc;
  // rank 16 with 16-byte aligned operands: the SwiGLU backward, the gate /
  // up adapters' P and dB, and dA_D in one pass (lora::mlp_mid_pass)
  const void* mid_ptrs[9] = {gate, up, dgate, dup, xa, PD, BG, BU, h};
  const bool fused_mid = R == lora::kDyRank && (int64_t)N * I < (1LL << 31) &&
                         lora::mlp_mid_ok(I, mid_ptrs, h ? 9 : 8, R2, R);

  // down projection: P_D, dA_D = P_D^T h, dB_D = s_D dY^T hA_D
  if (R == lora::kDyRank) {  // P_D and dB_D in one pass over dY
    const lora::DyJob jd{dy, H, H, static_cast<const bf16*>(BD), R,
                         static_cast<const bf16*>(hA_D), R, scale[2], PD, R, dB_D, R};
    rc = lora::dy_pass(N, &jd, 1, reinterpret_cast<char*>(part), part_bytes, st);
    if (rc) return rc;
  } else {
    Segment s1{{dy, H}, {static_cast<const bf16*>(BD), R}, H};
    rc = lora::skinny<TallCfg, kKMajor, kMNMajor, bf16>(N, R, s1, PD, R, scale[2], part,
                                                         part_bytes, st);
    if (rc) return rc;
    Segment s3{{dy, H}, {static_cast<const bf16*>(hA_D), R}, N};
    rc = lora::skinny<TallCfg, kMNMajor, kMNMajor, float>(H, R, s3, dB_D, R, scale[2], part,
                                                           part_bytes, st);
    if (rc) return rc;
  }
  if (!fused_mid && !h) {
    // h = silu(gate) up, as the SwiGLU forward forms it, into d_gate's buffer
    // (free until dH is written there below)
    rc = ml_swiglu_fwd(gate, up, dgate, (int64_t)N * I, ML_BF16, st);
    if (rc) return rc;
    h = dgate;
  }
  if (fused_mid) {
    rc = ML_OK;  // dA_D comes from the fused pass below
  } else if (R == lora::kDyRank) {
    rc = lora::ptx_pass(N, PD, R, R, static_cast<const bf16*>(h), I, I, dA_D, I,
                        reinterpret_cast<char*>(part), part_bytes, st);
  } else {
    Segment s2{{PD, R}, {static_cast<const bf16*>(h), I}, N};
    rc = lora::skinny<WideCfg, kMNMajor, kMNMajor, float>(R, I, s2, dA_D, I, 1.0f, part,
                                                           part_bytes, st);
  }
  if (rc) return rc;
  // dH = dY W_D + P_D A_D, a bf16 product as in the reference
  // (ops/fused_lora.py:230-233), written into d_gate's buffer; then the
  // SwiGLU backward (:235-244) streams dH, gate, up into d_gate (in place:
  // each element is read before it is written) and d_up - at rank 16 inside
  // the fused pass that also forms the gate / up adapters' P, dB and dA_D.
  // A separate pass beats the backward fused into the GEMM's epilogue here:
  // with every CU in the epilogue at once, the 512 KB of gate / up / d_gate
  // / d_up per tile left the matrix cores idle (324 us against 200 + 74 us).
  {
    Segment segs[2] = {Segment{{dy, H}, {static_cast<const bf16*>(WD), I}, H},
                       Segment{{PD, R}, {static_cast<const bf16*>(A_D), I}, R}};
    Problem pb;
    rc = make_problem<BigCfg>(pb, N, I, 2, segs, kKMajor, kMNMajor, 0);
    if (rc) return rc;
    rc = launch_store<bf16, R4Cfg>(pb, kKMajor, kMNMajor, dgate, I, 1.f, 0.f, st);
    if (rc) return rc;
  }
  if (fused_mid) {
    rc = lora::mlp_mid_pass(N, I, dgate, dup, static_cast<const bf16*>(gate),
                            static_cast<const bf16*>(up), static_cast<const bf16*>(h), xa, R2, PD,
                            R, static_cast<const bf16*>(BG), static_cast<const bf16*>(BU), R,
                            scale[0], scale[1], PGU, PGU + R, R2, dB_G, dB_U, R, dA_D,
                            reinterpret_cast<char*>(part), part_bytes, st);
    if (rc) return rc;
  } else {
    rc = ml_swiglu_bwd(gate, up, dgate, dgate, dup, (int64_t)N * I, ML_BF16, st);
    if (rc) return rc;
  }
  // gate / up adapters
  const bf16* dgu[2] = {dgate, dup};
  const void* Bs[2] = {BG, BU};
  float* dBs[2] = {dB_G, dB_U};
  if (fused_mid) {
    // P_G, P_U, dB_G, dB_U came from the fused pass
  } else if (R == lora::kDyRank) {  // P_G, P_U, dB_G, dB_U: one pass over each of d_gate, d_up
    lora::DyJob jobs[2];
    for (int i = 0; i < 2; ++i)
      jobs[i] = lora::DyJob{dgu[i], I, I, static_cast<const bf16*>(Bs[i]), R, xa + i * R, R2,
                            scale[i], PGU + i * R, R2, dBs[i], R};
    rc = lora::dy_pass(N, jobs, 2, reinterpret_cast<char*>(part), part_bytes, st);
    if (rc) return rc;
  }
  for (int i = 0; i < 2 && R != lora::kDyRank; ++i) {
    Segment sp{{dgu[i], I}, {static_cast<const bf16*>(Bs[i]), R}, I};
    rc = lora::skinny<TallCfg, kKMajor, kMNMajor, bf16>(N, R, sp, PGU + i * R, R2, scale[i], part,
                                                         part_bytes, st);
    if (rc) return rc;
    Segment sb{{dgu[i], I}, {xa + i * R, R2}, N};
    rc = lora::skinny<TallCfg, kMNMajor, kMNMajor, float>(I, R, sb, dBs[i], R, scale[i], part,
                                                           part_bytes, st);
    if (rc) return rc;
  }
  if (R == lora::kDyRank) {
    rc = lora::ptx_pass(N, PGU, R2, R2, x, H, H, dA_GU, H, reinterpret_cast<char*>(part),
                        part_bytes, st);
  } else {
    Segment sa{{PGU, R2}, {x, H}, N};
    rc = lora::skinny<WideCfg, kMNMajor, kMNMajor, float>(R2, H, sa, dA_GU, H, 1.0f, part,
                                                           part_bytes, st);
  }
  if (rc) return rc;
  // dX = [d_gate | d_up | P_GU] [W_G; W_U; A_GU]
  Segment segs[3] = {Segment{{dgate, I}, {static_cast<const bf16*>(WG), H}, I},
                     Segment{{dup, I}, {static_cast<const bf16*>(WU), H}, I},
                     Segment{{PGU, R2}, {static_cast<const bf16*>(A_GU), H}, R2}};
  Problem pb;
  rc = make_problem<BigCfg>(pb, N, H, 3, segs, kKMajor, kMNMajor, 0);
  if (rc) return rc;
  return launch_store<bf16, R4Cfg>(pb, kKMajor, kMNMajor, dX, H, 1.0f, 0.0f, st);
}

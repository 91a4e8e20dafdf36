// bf16 MFMA GEMM core for gfx950 (CDNA4): C[M,N] = sum_k A[m,k] * B[k,n],
// fp32 accumulation, pluggable epilogue.
//
// Tiling
//   block tile 256 x 256 x 64, 256 threads = 4 wave64s in a 2 x 2 grid, each
//   wave owns a 128 x 128 sub-tile = 4 x 4 v_mfma_f32_32x32x16_bf16 tiles
//   (256 fp32 accumulators per lane, held in AGPRs).
// Operand layouts (per operand, "rows" = M for A, N for B)
//   K-major : element (r, k) at p[r * ld + k]   (A row-major, F.linear weight)
//   MN-major: element (r, k) at p[k * ld + r]   (A^T stored, B row-major)
//   Both are staged into LDS as [rows][64 k] bf16, 128 bytes per row, with
//   the 16-byte chunks of a row XOR-swizzled so that ds_read_b128 fragment
//   reads (32 consecutive rows, same k chunk) and the stores are free of
//   bank conflicts for both 8- and 16-lane bank groups. MN-major tiles are
//   transposed in registers (8 x 8 bf16 blocks, v_perm_b32) on their way
//   into LDS, so the MFMA inner loop is the same for every layout.
// Pipeline
//   two LDS stages (2 x 64 KiB): the global loads of k-tile t+1 are in
//   flight while the MFMAs of k-tile t run; one barrier per k-tile.
// K segments
//   K may be a concatenation of up to kMaxSeg segments with their own A/B
//   pointers and leading dimensions (e.g. [dQ | dK | dV | lora] against
//   [Wq; Wk; Wv; A]); a segment's last k-tile is zero-filled past its end.
// Tile order
//   workgroups are dispatched round-robin over the 8 XCDs, so block b is
//   remapped to logical tile (b % 8) * ceil(T/8) + b / 8: each XCD walks a
//   contiguous range of logical tiles, ordered m-fastest within groups of
//   group_m m-tiles, so concurrently running tiles of one XCD share B (and
//   A within a group) in that XCD's L2.
#pragma once

#include "common.h"

namespace mla {
namespace gemm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kThreads = 256;
constexpr int kWM = 128, kWN = 128;
constexpr int kTM = kWM / 32, kTN = kWN / 32;
constexpr int kMaxSeg = 4;
constexpr int kRowBytes = kBK * 2;                 // 128
constexpr int kTileBytes = kBM * kRowBytes;        // 32 KiB (A and B tiles alike)
constexpr int kLdsBytes = 4 * kTileBytes;          // A + B, two stages: 128 KiB
constexpr int kXcds = 8;

enum : int { kKMajor = 0, kMNMajor = 1 };

struct Operand {
  const bf16* ptr;
  int64_t ld;
};

struct Segment {
  Operand a, b;
  int k_len;  // multiple of 8
};

struct Problem {
  int M, N;
  int nseg;
  Segment seg[kMaxSeg];
  int tiles_m, tiles_n;
  int group_m;
};

// 16-byte chunk c of LDS row r lives at chunk c ^ swz(r).
__device__ __forceinline__ int swz(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }

__device__ __forceinline__ int lds_off(int r, int c) { return r * kRowBytes + ((c ^ swz(r)) << 4); }

// ------------------------------------------------------------ tile loaders --
// Each thread moves 8 x 16 bytes of a 256-row x 64-k tile per k-step. The
// address of every load is a wave-uniform tile base (scalar registers) plus a
// 32-bit per-thread byte offset computed once per tile and K segment.
struct TileRegs {
  u32x4 v[8];
};

struct TileIter {
  const char* base;   // uniform: operand origin of this tile at k = 0 of the segment
  uint32_t off[8];    // per-thread byte offsets (k = 0)
  int64_t kstride;    // bytes per k step of 1 (K-major: 2, MN-major: 2 * ld)
};

// K-major: chunk q = tid + 256 i -> row q / 8, k-chunk q % 8 (a wave reads 8
// rows x 128 contiguous bytes per instruction). Rows past the operand end
// re-read its last row (those outputs are never stored).
__device__ __forceinline__ void setup_kmajor(TileIter& it, const Operand& op, int row0, int rows,
                                             int tid) {
  it.base = reinterpret_cast<const char*>(op.ptr + (int64_t)row0 * op.ld);
  it.kstride = 2;
  const int last = rows - 1 - row0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int q = tid + kThreads * i;
    int r = q >> 3;
    r = r < last ? r : last;
    it.off[i] = (uint32_t)(((int64_t)r * op.ld + ((q & 7) << 3)) * 2);
  }
}

// MN-major: thread owns the 8 (k) x 8 (r) block kb = tid % 8, rb = tid / 8 and
// loads its 8 k-rows of 16 bytes (8 consecutive r). rows % 8 == 0 is required.
__device__ __forceinline__ void setup_mnmajor(TileIter& it, const Operand& op, int row0, int rows,
                                              int tid) {
  it.base = reinterpret_cast<const char*>(op.ptr + row0);
  it.kstride = 2 * op.ld;
  const int kb = tid & 7;
  int r = (tid >> 3) << 3;
  r = r < rows - row0 - 8 ? r : rows - row0 - 8;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    it.off[j] = (uint32_t)((((int64_t)((kb << 3) + j)) * op.ld + r) * 2);
}

template <int LAYOUT>
__device__ __forceinline__ void setup_tile(TileIter& it, const Operand& op, int row0, int rows,
                                           int tid) {
  if constexpr (LAYOUT == kKMajor)
    setup_kmajor(it, op, row0, rows, tid);
  else
    setup_mnmajor(it, op, row0, rows, tid);
}

// Loads the k-tile starting at k0 of a segment of length klen; k past klen
// reads as zero.
template <int LAYOUT>
__device__ __forceinline__ void load_tile(TileRegs& t, const TileIter& it, int k0, int klen,
                                          int tid) {
  const char* b = it.base + (int64_t)k0 * it.kstride;
  const int kb8 = (tid & 7) << 3;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int kk = (LAYOUT == kKMajor) ? k0 + kb8 : k0 + kb8 + i;
    const bool kin = kk < klen;
    // k past the segment end re-reads the tile origin (row row0, k 0 of the
    // segment: always in bounds) and is replaced by zeros
    const u32x4 val = *reinterpret_cast<const u32x4*>(kin ? b + it.off[i] : it.base);
    t.v[i] = kin ? val : u32x4{0u, 0u, 0u, 0u};
  }
}

__device__ __forceinline__ void store_kmajor(const TileRegs& t, char* lds, int tid) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int q = tid + kThreads * i;
    *reinterpret_cast<u32x4*>(lds + lds_off(q >> 3, q & 7)) = t.v[i];
  }
}

// Transposes the 8 x 8 block (t.v[j] holds r = 0..7 at k = j) into 8 rows of
// 8 consecutive k and stores them at chunk kb of rows 8 rb .. 8 rb + 7.
__device__ __forceinline__ void store_mnmajor(const TileRegs& t, char* lds, int tid) {
  const int kb = tid & 7;
  const int rb = tid >> 3;
#pragma unroll
  for (int rr = 0; rr < 8; ++rr) {
    const unsigned sel = (rr & 1) ? 0x07060302u : 0x05040100u;
    u32x4 o;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp)
      o[pp] = __builtin_amdgcn_perm(t.v[2 * pp + 1][rr >> 1], t.v[2 * pp][rr >> 1], sel);
    *reinterpret_cast<u32x4*>(lds + lds_off((rb << 3) + rr, kb)) = o;
  }
}

template <int LAYOUT>
__device__ __forceinline__ void store_tile(const TileRegs& t, char* lds, int tid) {
  if constexpr (LAYOUT == kKMajor)
    store_kmajor(t, lds, tid);
  else
    store_mnmajor(t, lds, tid);
}

// ----------------------------------------------------------------- compute --
__device__ __forceinline__ void mma_tile(f32x16_t (&acc)[kTM][kTN], const char* As, const char* Bs,
                                         int wm, int wn, int lane) {
  const int lr = lane & 31;
  const int hk = lane >> 5;
#pragma unroll
  for (int s = 0; s < kBK / 16; ++s) {
    const int c = 2 * s + hk;
    bf16x8_t af[kTM], bfr[kTN];
#pragma unroll
    for (int i = 0; i < kTM; ++i)
      af[i] = *reinterpret_cast<const bf16x8_t*>(As + lds_off(wm + 32 * i + lr, c));
#pragma unroll
    for (int j = 0; j < kTN; ++j)
      bfr[j] = *reinterpret_cast<const bf16x8_t*>(Bs + lds_off(wn + 32 * j + lr, c));
#pragma unroll
    for (int i = 0; i < kTM; ++i)
#pragma unroll
      for (int j = 0; j < kTN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
  }
}

// Logical tile of this workgroup (XCD-aware, grouped); false if none.
__device__ __forceinline__ bool tile_coords(const Problem& pb, int& tm, int& tn) {
  const int T = pb.tiles_m * pb.tiles_n;
  const int T8 = (T + kXcds - 1) / kXcds;
  const int bid = blockIdx.x;
  const int logical = (bid % kXcds) * T8 + bid / kXcds;
  if (logical >= T) return false;
  const int gsize = pb.group_m * pb.tiles_n;
  const int g = logical / gsize;
  const int first_m = g * pb.group_m;
  const int gm = min(pb.tiles_m - first_m, pb.group_m);
  const int within = logical - g * gsize;
  tm = first_m + within % gm;
  tn = within / gm;
  return true;
}

inline int grid_blocks(const Problem& pb) {
  const int T = pb.tiles_m * pb.tiles_n;
  return ((T + kXcds - 1) / kXcds) * kXcds;
}

// Geometry of one lane's accumulators: element v of MFMA tile (i, j) sits at
// row m0 + 32 i + acc_row(v, lane), column n0 + 32 j + (lane & 31).
__device__ __forceinline__ int acc_row(int v, int lane) {
  return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
}

// Main loop: accumulates the tile (tm, tn) into acc. smem is the kernel's
// __shared__ array (stage s of A at s * kTileBytes, of B at (2 + s) * kTileBytes).
template <int LA, int LB>
__device__ __forceinline__ void mainloop(const Problem& pb, int tm, int tn, char* smem,
                                         f32x16_t (&acc)[kTM][kTN]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * kWM;
  const int wn = (wave & 1) * kWN;
  const int m0 = tm * kBM;
  const int n0 = tn * kBN;
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  int nk = 0;
  for (int s = 0; s < pb.nseg; ++s) nk += (pb.seg[s].k_len + kBK - 1) / kBK;
  if (nk == 0) return;

  TileIter ia, ib;
  TileRegs ra, rb;
  int seg = 0, k0 = 0, klen = pb.seg[0].k_len;
  setup_tile<LA>(ia, pb.seg[0].a, m0, pb.M, tid);
  setup_tile<LB>(ib, pb.seg[0].b, n0, pb.N, tid);
  load_tile<LA>(ra, ia, 0, klen, tid);
  load_tile<LB>(rb, ib, 0, klen, tid);
  store_tile<LA>(ra, smem, tid);
  store_tile<LB>(rb, smem + 2 * kTileBytes, tid);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      k0 += kBK;
      if (k0 >= klen) {
        ++seg;
        k0 = 0;
        klen = pb.seg[seg].k_len;
        setup_tile<LA>(ia, pb.seg[seg].a, m0, pb.M, tid);
        setup_tile<LB>(ib, pb.seg[seg].b, n0, pb.N, tid);
      }
      load_tile<LA>(ra, ia, k0, klen, tid);
      load_tile<LB>(rb, ib, k0, klen, tid);
    }
    mma_tile(acc, smem + cur * kTileBytes, smem + (2 + cur) * kTileBytes, wm, wn, lane);
    if (more) {
      store_tile<LA>(ra, smem + (cur ^ 1) * kTileBytes, tid);
      store_tile<LB>(rb, smem + (2 + (cur ^ 1)) * kTileBytes, tid);
    }
    __syncthreads();
  }
}

// The GEMM kernel: mainloop + epilogue functor
//   epi(acc, m_base, n_base, lane, smem) with m_base / n_base the origin of
//   this wave's 128 x 128 sub-tile. smem may be reused by the epilogue.
template <int LA, int LB, class Epi>
__global__ __launch_bounds__(kThreads) void gemm_kernel(const Problem pb, const Epi epi) {
  __shared__ __attribute__((aligned(16))) char smem[kLdsBytes];
  int tm, tn;
  if (!tile_coords(pb, tm, tn)) return;
  f32x16_t acc[kTM][kTN];
  mainloop<LA, LB>(pb, tm, tn, smem, acc);
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  epi(acc, tm * kBM + (wave >> 1) * kWM, tn * kBN + (wave & 1) * kWN, tid & 63, smem);
}

// C = alpha * acc + beta * C (C of type TC, row-major with ldc).
template <typename TC>
struct EpiStore {
  TC* C;
  int64_t ldc;
  int M, N;
  float alpha, beta;

  __device__ __forceinline__ void operator()(f32x16_t (&acc)[kTM][kTN], int m0, int n0, int lane,
                                             char*) const {
    const int col = lane & 31;
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      const int n = n0 + 32 * j + col;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < kTM; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int m = m0 + 32 * i + acc_row(v, lane);
          if (m < M) {
            TC* p = C + (int64_t)m * ldc + n;
            float r = alpha * acc[i][j][v];
            if (beta != 0.f) r += beta * to_f32(*p);
            *p = from_f32<TC>(r);
          }
        }
      }
    }
  }
};

// ---------------------------------------------------------------- host side --

// Validates one operand of a segment. rows_dim: M (A) or N (B).
inline int check_operand(const Operand& op, int layout, int rows_dim, int k_len, const char* what) {
  ML_CHECK(op.ptr != nullptr, "gemm: null %s", what);
  ML_CHECK(aligned16(op.ptr), "gemm: %s must be 16-byte aligned", what);
  ML_CHECK(op.ld % 8 == 0, "gemm: leading dimension of %s must be a multiple of 8 (got %lld)", what,
           (long long)op.ld);
  if (layout == kKMajor) {
    ML_CHECK(op.ld >= k_len, "gemm: %s leading dimension %lld < K segment %d", what,
             (long long)op.ld, k_len);
  } else {
    ML_CHECK(rows_dim % 8 == 0, "gemm: MN-major %s needs its M/N size %% 8 == 0 (got %d)", what,
             rows_dim);
    ML_CHECK(op.ld >= rows_dim, "gemm: %s leading dimension %lld < %d", what, (long long)op.ld,
             rows_dim);
  }
  return ML_OK;
}

inline int make_problem(Problem& pb, int M, int N, int nseg, const Segment* segs, int la, int lb,
                        int group_m) {
  ML_CHECK(M > 0 && N > 0, "gemm: empty output (M=%d, N=%d)", M, N);
  ML_CHECK(nseg >= 1 && nseg <= kMaxSeg, "gemm: 1..%d K segments supported (got %d)", kMaxSeg,
           nseg);
  pb = Problem{};
  pb.M = M;
  pb.N = N;
  pb.nseg = nseg;
  const bool any_kmajor = la == kKMajor || lb == kKMajor;
  for (int s = 0; s < nseg; ++s) {
    ML_CHECK(segs[s].k_len >= 0 && (!any_kmajor || segs[s].k_len % 8 == 0),
             "gemm: K segment %d length must be a non-negative multiple of 8 (got %d)", s,
             segs[s].k_len);
    pb.seg[s] = segs[s];
    if (segs[s].k_len > 0) {
      int rc = check_operand(segs[s].a, la, M, segs[s].k_len, "A");
      if (rc) return rc;
      rc = check_operand(segs[s].b, lb, N, segs[s].k_len, "B");
      if (rc) return rc;
    }
  }
  // drop empty segments
  int w = 0;
  for (int s = 0; s < pb.nseg; ++s)
    if (pb.seg[s].k_len > 0) pb.seg[w++] = pb.seg[s];
  pb.nseg = w;
  pb.tiles_m = (M + kBM - 1) / kBM;
  pb.tiles_n = (N + kBN - 1) / kBN;
  pb.group_m = group_m > 0 ? min(group_m, pb.tiles_m) : pb.tiles_m;
  return ML_OK;
}

template <typename TC>
inline int launch_store(const Problem& pb, int la, int lb, void* C, int64_t ldc, float alpha, float beta,
                 hipStream_t st) {
  EpiStore<TC> epi{static_cast<TC*>(C), ldc, pb.M, pb.N, alpha, beta};
  const dim3 grid(grid_blocks(pb));
#define ML_G(LA, LB) gemm_kernel<LA, LB, EpiStore<TC>><<<grid, kThreads, 0, st>>>(pb, epi)
  if (la == kKMajor && lb == kKMajor) ML_G(kKMajor, kKMajor);
  else if (la == kKMajor && lb == kMNMajor) ML_G(kKMajor, kMNMajor);
  else if (la == kMNMajor && lb == kKMajor) ML_G(kMNMajor, kKMajor);
  else ML_G(kMNMajor, kMNMajor);
#undef ML_G
  ML_LAUNCH_CHECK();
  return ML_OK;
}

}  // namespace gemm
}  // namespace mla

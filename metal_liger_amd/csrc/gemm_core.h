// bf16 MFMA GEMM core for gfx950 (CDNA4): C[M,N] = sum_k A[m,k] * B[k,n],
// fp32 accumulation, pluggable epilogue.
//
// Tiling (compile-time tile shape Cfg<BM, BN, WAVES_M>)
//   256 threads = 4 wave64s in a WAVES_M x (4 / WAVES_M) grid; a wave owns a
//   (BM / WAVES_M) x (BN / WAVES_N) sub-tile made of 32 x 32 tiles of
//   v_mfma_f32_32x32x16_bf16 (accumulators in AGPRs). BK = 64.
//   The big-GEMM shape is 256 x 256 (2 x 2 waves of 128 x 128); narrow shapes
//   (256 x 32, 64 x 256) serve the rank-r LoRA products without wasting MFMA
//   work on padding.
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
//   two LDS stages: the global loads of k-tile t+1 are in flight while the
//   MFMAs of k-tile t run; one barrier per k-tile. Global addresses are a
//   uniform tile base (scalar registers) plus 32-bit per-thread offsets.
// K segments
//   K may be a concatenation of up to kMaxSeg segments with their own A/B
//   pointers and leading dimensions (e.g. [dQ | dK | dV | lora] against
//   [Wq; Wk; Wv; A]); a segment's last k-tile is zero-filled past its end.
// Split-K
//   with ksplit > 1 (single segment), split s accumulates k-tiles
//   [s * kps, (s + 1) * kps) and the epilogue receives s; EpiPartial writes
//   fp32 partial tiles that reduce_partials_kernel sums in fixed order.
// Tile order
//   workgroups are dispatched round-robin over the 8 XCDs, so block b is
//   remapped to logical work item (b % 8) * ceil(W/8) + b / 8: each XCD walks
//   a contiguous range, ordered m-fastest within groups of group_m m-tiles,
//   so concurrently running tiles of one XCD share operands in its L2.
#pragma once

#include <utility>

#include "common.h"

namespace mla {
namespace gemm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;
constexpr int kThreads = 256;
constexpr int kMaxSeg = 8;
constexpr int kRowBytes = kBK * 2;  // 128
constexpr int kXcds = 8;

// Default m-tiles per tile-order group (group_m = 0): with 32 blocks
// resident per XCD, groups of 8 give each XCD an 8 x 4 patch of tiles.
#ifndef ML_GEMM_GROUP_M
#define ML_GEMM_GROUP_M 8
#endif

template <int BM_, int BN_, int WAVES_M_>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_;
  static constexpr int WAVES_M = WAVES_M_, WAVES_N = 4 / WAVES_M_;
  static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  static constexpr int TM = WM / 32, TN = WN / 32;
  static constexpr int A_BYTES = BM * kRowBytes, B_BYTES = BN * kRowBytes;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int LDS_BYTES = 2 * STAGE_BYTES;
  static_assert(WAVES_M * WAVES_N == 4, "4 waves per block");
  static_assert(TM >= 1 && TN >= 1 && WM % 32 == 0 && WN % 32 == 0, "wave tile of 32x32 MFMAs");
  static_assert(BM <= 256 && BN <= 256, "at most one 16-byte chunk set per thread");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
};

using BigCfg = Cfg<256, 256, 2>;   // 2 x 2 waves of 128 x 128
using TallCfg = Cfg<256, 32, 4>;   // 4 x 1 waves of 64 x 32  (rank-r wide outputs)
using WideCfg = Cfg<64, 256, 1>;   // 1 x 4 waves of 64 x 64  (few-row outputs)

// Names for the big tile
constexpr int kBM = BigCfg::BM, kBN = BigCfg::BN;
constexpr int kWM = BigCfg::WM, kWN = BigCfg::WN;
constexpr int kTM = BigCfg::TM, kTN = BigCfg::TN;

enum : int { kKMajor = 0, kMNMajor = 1 };

struct Operand {
  const bf16* ptr;
  int64_t ld;
};

struct Segment {
  Operand a, b;
  int k_len;
};

struct Problem {
  int M, N;
  int nseg;
  Segment seg[kMaxSeg];
  int tiles_m, tiles_n;
  int group_m;
  int ksplit;  // >= 1; > 1 only with one segment
  int kps;     // k-tiles per split
};

// 16-byte chunk c of LDS row r lives at chunk c ^ swz(r).
__device__ __forceinline__ int swz(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }

__device__ __forceinline__ int lds_off(int r, int c) { return r * kRowBytes + ((c ^ swz(r)) << 4); }

// ------------------------------------------------------------ tile loaders --
// A ROWS x 64 tile: K-major moves ROWS / 32 chunks of 16 bytes per thread
// (chunk q = tid + 256 i -> row q / 8, k-chunk q % 8; a wave reads 8 rows x
// 128 contiguous bytes per instruction); MN-major moves one 8 (k) x 8 (r)
// block per thread (kb = tid % 8, rb = tid / 8) for the first ROWS threads.
struct TileRegs {
  u32x4 v[8];
};

struct TileIter {
  const char* base;   // uniform: operand origin of this tile at k = 0 of the segment
  uint32_t off[8];    // per-thread byte offsets (k = 0)
  int64_t kstride;    // bytes per unit of k
};

template <int ROWS>
constexpr int kmajor_chunks() { return ROWS / 32; }

// Rows past the operand end re-read its last row (those outputs are never stored).
template <int ROWS>
__device__ __forceinline__ void setup_kmajor(TileIter& it, const Operand& op, int row0, int rows,
                                             int tid) {
  it.base = reinterpret_cast<const char*>(op.ptr + (int64_t)row0 * op.ld);
  it.kstride = 2;
  const int last = rows - 1 - row0;
#pragma unroll
  for (int i = 0; i < kmajor_chunks<ROWS>(); ++i) {
    const int q = tid + kThreads * i;
    int r = q >> 3;
    r = r < last ? r : last;
    it.off[i] = (uint32_t)(((int64_t)r * op.ld + ((q & 7) << 3)) * 2);
  }
}

// rows % 8 == 0 is required (16-byte loads of 8 consecutive r).
template <int ROWS>
__device__ __forceinline__ void setup_mnmajor(TileIter& it, const Operand& op, int row0, int rows,
                                              int tid) {
  it.base = reinterpret_cast<const char*>(op.ptr + row0);
  it.kstride = 2 * op.ld;
  const int kb = tid & 7;
  int r = (tid >> 3) << 3;
  r = r < ROWS ? r : 0;  // threads past the tile's rows do not load
  r = r < rows - row0 - 8 ? r : rows - row0 - 8;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    it.off[j] = (uint32_t)((((int64_t)((kb << 3) + j)) * op.ld + r) * 2);
}

template <int LAYOUT, int ROWS>
__device__ __forceinline__ void setup_tile(TileIter& it, const Operand& op, int row0, int rows,
                                           int tid) {
  if constexpr (LAYOUT == kKMajor)
    setup_kmajor<ROWS>(it, op, row0, rows, tid);
  else
    setup_mnmajor<ROWS>(it, op, row0, rows, tid);
}

// Loads the k-tile starting at k0 (< klen) of a segment of length klen.
// Interior tiles (k0 + 64 <= klen, a uniform test) load unpredicated from a
// uniform base plus 32-bit per-thread offsets. In a segment's last, partial
// tile the lanes whose k lies past klen read the tile origin instead (always
// in bounds); store_tile zeroes their data. Nothing consumes the loaded
// registers before the LDS store, so the load latency overlaps the MFMAs.
template <int LAYOUT, int ROWS>
__device__ __forceinline__ void load_tile(TileRegs& t, const TileIter& it, int k0, int klen,
                                          int tid) {
  // MN-major tiles narrower than the block: only the first ROWS / 8 x 8
  // threads hold a block (store_mnmajor skips the others too).
  if (LAYOUT == kMNMajor && ROWS < kThreads && ((tid >> 3) << 3) >= ROWS) return;
  const char* b = it.base + (int64_t)k0 * it.kstride;
  constexpr int NL = (LAYOUT == kKMajor) ? kmajor_chunks<ROWS>() : 8;
  if (k0 + kBK <= klen) {
#pragma unroll
    for (int i = 0; i < NL; ++i) t.v[i] = *reinterpret_cast<const u32x4*>(b + it.off[i]);
  } else {
    const int kb8 = (tid & 7) << 3;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int kk = (LAYOUT == kKMajor) ? k0 + kb8 : k0 + kb8 + i;
      t.v[i] = *reinterpret_cast<const u32x4*>(b + (kk < klen ? it.off[i] : 0u));
    }
  }
}

// Zeroes the chunks of a partial tile whose k lies past klen (uniform test).
template <int LAYOUT, int ROWS>
__device__ __forceinline__ void zero_tail(TileRegs& t, int k0, int klen, int tid) {
  if (k0 + kBK <= klen) return;
  const int kb8 = (tid & 7) << 3;
  constexpr int NL = (LAYOUT == kKMajor) ? kmajor_chunks<ROWS>() : 8;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int kk = (LAYOUT == kKMajor) ? k0 + kb8 : k0 + kb8 + i;
    if (kk >= klen) t.v[i] = u32x4{0u, 0u, 0u, 0u};
  }
}

template <int ROWS>
__device__ __forceinline__ void store_kmajor(const TileRegs& t, char* lds, int tid) {
#pragma unroll
  for (int i = 0; i < kmajor_chunks<ROWS>(); ++i) {
    const int q = tid + kThreads * i;
    *reinterpret_cast<u32x4*>(lds + lds_off(q >> 3, q & 7)) = t.v[i];
  }
}

// Transposes the 8 x 8 block (t.v[j] holds r = 0..7 at k = j) into 8 rows of
// 8 consecutive k and stores them at chunk kb of rows 8 rb .. 8 rb + 7.
template <int ROWS>
__device__ __forceinline__ void store_mnmajor(const TileRegs& t, char* lds, int tid) {
  const int kb = tid & 7;
  const int rb = tid >> 3;
  if ((rb << 3) >= ROWS) return;
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

template <int LAYOUT, int ROWS>
__device__ __forceinline__ void store_tile(TileRegs& t, char* lds, int tid, int k0, int klen) {
  zero_tail<LAYOUT, ROWS>(t, k0, klen, tid);
  if constexpr (LAYOUT == kKMajor)
    store_kmajor<ROWS>(t, lds, tid);
  else
    store_mnmajor<ROWS>(t, lds, tid);
}

// Software-pipelined staging: a tile held in registers is written to LDS in
// four parts, one per MFMA k-step, and each register is reloaded with the
// following tile as soon as its part is written (K-major: the chunks just
// stored; MN-major: all eight after the last part, since every row of the
// 8 x 8 transpose reads all eight registers).
template <int LAYOUT, int ROWS>
constexpr int store_count(int part) {
  if constexpr (LAYOUT == kKMajor) {
    int n = 0;
    for (int i = 0; i < kmajor_chunks<ROWS>(); ++i) n += (i * 4 / kmajor_chunks<ROWS>() == part);
    return n;
  } else {
    return 2;
  }
}

template <int LAYOUT, int ROWS>
constexpr int reload_count(int part) {
  if constexpr (LAYOUT == kKMajor)
    return store_count<LAYOUT, ROWS>(part);
  else
    return part == 3 ? 8 : 0;
}

// ----------------------------------------------------------------- compute --
// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;
constexpr int kSchedDsWrite = 0x200;
constexpr int kSchedVmemRead = 0x020;

// Fragments of one 16-wide k-step for a wave: TM A fragments, TN B fragments.
template <class C>
struct Frags {
  bf16x8_t a[C::TM], b[C::TN];
};

template <class C>
__device__ __forceinline__ void load_frags(Frags<C>& f, const char* As, const char* Bs, int wm,
                                           int wn, int lane, int s) {
  const int lr = lane & 31;
  const int c = 2 * s + (lane >> 5);
  // B first: the first TN MFMAs of a step use every B fragment and A[0].
#pragma unroll
  for (int j = 0; j < C::TN; ++j)
    f.b[j] = *reinterpret_cast<const bf16x8_t*>(Bs + lds_off(wn + 32 * j + lr, c));
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
    f.a[i] = *reinterpret_cast<const bf16x8_t*>(As + lds_off(wm + 32 * i + lr, c));
}

template <class C>
__device__ __forceinline__ void mfma_step(f32x16_t (&acc)[C::TM][C::TN], const Frags<C>& f) {
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
}

// Interleaves the next k-step's LDS reads with this k-step's MFMAs: the
// compiler otherwise serialises each fragment read against the MFMAs that
// consume it and exposes the LDS latency every few MFMAs.
template <class C>
__device__ __forceinline__ void sched_reads_between_mfmas() {
  constexpr int kReads = C::TM + C::TN;
  constexpr int kMfma = C::TM * C::TN;
  constexpr int kPer = kMfma / kReads > 0 ? kMfma / kReads : 1;
#pragma unroll
  for (int q = 0; q < kReads; ++q) {
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, kPer, 0);
  }
  if constexpr (kMfma > kPer * kReads)
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, kMfma - kPer * kReads, 0);
}

// One 64-wide k-tile from LDS stage (As, Bs): 4 k-steps with the fragments
// of step s + 1 read while the MFMAs of step s run.
// sched_barrier(0) fences each block so that the scheduler can only
// interleave step s + 1's reads with step s's MFMAs, which keeps both
// fragment sets live in distinct registers.
template <class C>
__device__ __forceinline__ void mma_tile(f32x16_t (&acc)[C::TM][C::TN], const char* As,
                                         const char* Bs, int wm, int wn, int lane) {
  Frags<C> f0, f1;
  load_frags<C>(f0, As, Bs, wm, wn, lane, 0);
  __builtin_amdgcn_sched_barrier(0);
  load_frags<C>(f1, As, Bs, wm, wn, lane, 1);
  mfma_step<C>(acc, f0);
  sched_reads_between_mfmas<C>();
  __builtin_amdgcn_sched_barrier(0);
  load_frags<C>(f0, As, Bs, wm, wn, lane, 2);
  mfma_step<C>(acc, f1);
  sched_reads_between_mfmas<C>();
  __builtin_amdgcn_sched_barrier(0);
  load_frags<C>(f1, As, Bs, wm, wn, lane, 3);
  mfma_step<C>(acc, f0);
  sched_reads_between_mfmas<C>();
  __builtin_amdgcn_sched_barrier(0);
  mfma_step<C>(acc, f1);
  __builtin_amdgcn_sched_barrier(0);
}

// Compile-time loop: f(std::integral_constant<int, q>) for q = 0 .. N-1.
template <class F, int... Q>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Q...>) {
  (f(std::integral_constant<int, Q>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Single operations of a k-step, addressed by compile-time index.
// Fragment read q: B[q] for q < TN, then A[q - TN].
template <class C, int Q>
__device__ __forceinline__ void read_frag(Frags<C>& f, const char* As, const char* Bs, int wm,
                                          int wn, int lane, int s) {
  const int lr = lane & 31;
  const int c = 2 * s + (lane >> 5);
  if constexpr (Q < C::TN)
    f.b[Q] = *reinterpret_cast<const bf16x8_t*>(Bs + lds_off(wn + 32 * Q + lr, c));
  else
    f.a[Q - C::TN] = *reinterpret_cast<const bf16x8_t*>(As + lds_off(wm + 32 * (Q - C::TN) + lr, c));
}

// First K-major chunk written in part P of a tile of NL chunks per thread.
constexpr int part_first(int nl, int part) { return (part * nl + 3) / 4; }

// The I-th LDS store of part P (K-major: chunk part_first + I; MN-major:
// row 2P + I of the 8 x 8 block).
template <int LAYOUT, int ROWS, int P, int I>
__device__ __forceinline__ void store_one(const TileRegs& t, char* lds, int tid) {
  if constexpr (LAYOUT == kKMajor) {
    constexpr int i = part_first(kmajor_chunks<ROWS>(), P) + I;
    const int q = tid + kThreads * i;
    *reinterpret_cast<u32x4*>(lds + lds_off(q >> 3, q & 7)) = t.v[i];
  } else {
    const int kb = tid & 7;
    const int rb = tid >> 3;
    if (ROWS < kThreads && (rb << 3) >= ROWS) return;
    constexpr int rr = 2 * P + I;
    constexpr unsigned sel = (rr & 1) ? 0x07060302u : 0x05040100u;
    u32x4 o;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp)
      o[pp] = __builtin_amdgcn_perm(t.v[2 * pp + 1][rr >> 1], t.v[2 * pp][rr >> 1], sel);
    *reinterpret_cast<u32x4*>(lds + lds_off((rb << 3) + rr, kb)) = o;
  }
}

// The I-th reload of part P (K-major: the chunk store_one<P, I> wrote;
// MN-major, part 3 only: register I). Lanes whose k lies past klen read the
// tile origin (in bounds); zero_tail clears them before the tile is stored.
template <int LAYOUT, int ROWS, int P, int I>
__device__ __forceinline__ void reload_one(TileRegs& t, const char* b, const TileIter& it, int k0,
                                           int klen, int tid) {
  if (LAYOUT == kMNMajor && ROWS < kThreads && ((tid >> 3) << 3) >= ROWS) return;
  const int kb8 = (tid & 7) << 3;
  if constexpr (LAYOUT == kKMajor) {
    constexpr int i = part_first(kmajor_chunks<ROWS>(), P) + I;
    t.v[i] = *reinterpret_cast<const u32x4*>(b + (k0 + kb8 < klen ? it.off[i] : 0u));
  } else {
    t.v[I] = *reinterpret_cast<const u32x4*>(b + (k0 + kb8 + I < klen ? it.off[I] : 0u));
  }
}

// One k-step of the pipelined tile, in a fixed issue order: MFMA slot q
// (q = 0 .. TM*TN-1) is preceded by the q-th fragment read of step S + 1,
// the q-th LDS store of part S of the staged tile and the q-th reload;
// sched_barrier(0) keeps the compiler from regrouping them.
template <class C, int LA, int LB, bool RELOAD, int S>
__device__ __forceinline__ void pipe_step(f32x16_t (&acc)[C::TM][C::TN], Frags<C>& fnext,
                                          const Frags<C>& fcur, const char* As, const char* Bs,
                                          int wm, int wn, int lane, TileRegs& ra, TileRegs& rb,
                                          char* nxt, const char* bA, const char* bB,
                                          const TileIter& ia, const TileIter& ib, int k0,
                                          int klen, int tid) {
  constexpr int kReads = S < 3 ? C::TM + C::TN : 0;
  constexpr int kWa = store_count<LA, C::BM>(S), kWb = store_count<LB, C::BN>(S);
  constexpr int kLa = RELOAD ? reload_count<LA, C::BM>(S) : 0;
  constexpr int kLb = RELOAD ? reload_count<LB, C::BN>(S) : 0;
  constexpr int kMfma = C::TM * C::TN;
  // Stores: A in slots [0, kWa), B in [kWa, kWa + kWb). A reload never
  // precedes the store that reads its register: K-major chunk i is stored
  // and reloaded in one slot (store first); an MN-major operand's reloads
  // start after its last store, since each transposed row reads all eight
  // registers.
  constexpr int kA0 = LA == kMNMajor ? kWa : 0;
  constexpr int kB0min = LB == kMNMajor ? kWa + kWb : kWa;
  constexpr int kB0 = kA0 + kLa > kB0min ? kA0 + kLa : kB0min;
  constexpr int kMax1 = kReads > kWa + kWb ? kReads : kWa + kWb;
  constexpr int kMax2 = kMax1 > kB0 + kLb ? kMax1 : kB0 + kLb;
  constexpr int kSlots = kMfma > kMax2 ? kMfma : kMax2;
  char* nxtB = nxt + C::A_BYTES;
  static_for<kSlots>([&](auto qc) {
    constexpr int q = decltype(qc)::value;
    if constexpr (q < kReads) read_frag<C, q>(fnext, As, Bs, wm, wn, lane, S + 1);
    if constexpr (q < kWa) store_one<LA, C::BM, S, q>(ra, nxt, tid);
    else if constexpr (q < kWa + kWb) store_one<LB, C::BN, S, q - kWa>(rb, nxtB, tid);
    if constexpr (q >= kA0 && q < kA0 + kLa)
      reload_one<LA, C::BM, S, q - kA0>(ra, bA, ia, k0, klen, tid);
    if constexpr (q >= kB0 && q < kB0 + kLb)
      reload_one<LB, C::BN, S, q - kB0>(rb, bB, ib, k0, klen, tid);
    if constexpr (q < kMfma) {
      constexpr int i = q / C::TN, j = q % C::TN;
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fcur.a[i], fcur.b[j], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  });
}

// A k-tile from LDS stage (As, Bs) while the registers (ra, rb) holding the
// next tile are written to stage nxt and, with RELOAD, refilled with the
// k-tile at k0 of the iterators (ia, ib).
template <class C, int LA, int LB, bool RELOAD>
__device__ __forceinline__ void mma_tile_pipelined(f32x16_t (&acc)[C::TM][C::TN], const char* As,
                                                   const char* Bs, int wm, int wn, int lane,
                                                   TileRegs& ra, TileRegs& rb, char* nxt,
                                                   const TileIter& ia, const TileIter& ib, int k0,
                                                   int klen, int tid) {
  Frags<C> f0, f1;
  load_frags<C>(f0, As, Bs, wm, wn, lane, 0);
  __builtin_amdgcn_sched_barrier(0);
  const char* bA = ia.base + (int64_t)k0 * ia.kstride;
  const char* bB = ib.base + (int64_t)k0 * ib.kstride;
  pipe_step<C, LA, LB, RELOAD, 0>(acc, f1, f0, As, Bs, wm, wn, lane, ra, rb, nxt, bA, bB, ia, ib,
                                  k0, klen, tid);
  pipe_step<C, LA, LB, RELOAD, 1>(acc, f0, f1, As, Bs, wm, wn, lane, ra, rb, nxt, bA, bB, ia, ib,
                                  k0, klen, tid);
  pipe_step<C, LA, LB, RELOAD, 2>(acc, f1, f0, As, Bs, wm, wn, lane, ra, rb, nxt, bA, bB, ia, ib,
                                  k0, klen, tid);
  pipe_step<C, LA, LB, RELOAD, 3>(acc, f0, f1, As, Bs, wm, wn, lane, ra, rb, nxt, bA, bB, ia, ib,
                                  k0, klen, tid);
}

// Work item of this workgroup (XCD-aware, grouped); false if none.
__device__ __forceinline__ bool tile_coords(const Problem& pb, int& tm, int& tn, int& split) {
  const int W = pb.tiles_m * pb.tiles_n * pb.ksplit;
  const int W8 = (W + kXcds - 1) / kXcds;
  const int bid = blockIdx.x;
  const int logical = (bid % kXcds) * W8 + bid / kXcds;
  if (logical >= W) return false;
  split = logical % pb.ksplit;
  const int t = logical / pb.ksplit;
  const int gsize = pb.group_m * pb.tiles_n;
  const int g = t / gsize;
  const int first_m = g * pb.group_m;
  const int gm = min(pb.tiles_m - first_m, pb.group_m);
  const int within = t - g * gsize;
  tm = first_m + within % gm;
  tn = within / gm;
  return true;
}

inline int grid_blocks(const Problem& pb) {
  const int W = pb.tiles_m * pb.tiles_n * pb.ksplit;
  return ((W + kXcds - 1) / kXcds) * kXcds;
}

// Geometry of one lane's accumulators: element v of MFMA tile (i, j) sits at
// row m0 + 32 i + acc_row(v, lane), column n0 + 32 j + (lane & 31).
__device__ __forceinline__ int acc_row(int v, int lane) {
  return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
}

// Main loop: accumulates work item (tm, tn, split) into acc.
template <class C, int LA, int LB>
__device__ __forceinline__ void mainloop(const Problem& pb, int tm, int tn, int split,
                                         char* stage0, char* stage1,
                                         f32x16_t (&acc)[C::TM][C::TN]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave / C::WAVES_N) * C::WM;
  const int wn = (wave % C::WAVES_N) * C::WN;
  const int m0 = tm * C::BM;
  const int n0 = tn * C::BN;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  int nk, seg = 0, k0 = 0;
  if (pb.ksplit > 1) {
    // single segment: k-tiles [split * kps, min(total, (split + 1) * kps))
    const int total = (pb.seg[0].k_len + kBK - 1) / kBK;
    const int first = split * pb.kps;
    nk = total - first < pb.kps ? total - first : pb.kps;
    k0 = first * kBK;
  } else {
    nk = 0;
    for (int s = 0; s < pb.nseg; ++s) nk += (pb.seg[s].k_len + kBK - 1) / kBK;
  }
  if (nk <= 0) return;
  int klen = pb.seg[0].k_len;

  TileIter ia, ib;
  TileRegs ra, rb;
  setup_tile<LA, C::BM>(ia, pb.seg[0].a, m0, pb.M, tid);
  setup_tile<LB, C::BN>(ib, pb.seg[0].b, n0, pb.N, tid);
  load_tile<LA, C::BM>(ra, ia, k0, klen, tid);
  load_tile<LB, C::BN>(rb, ib, k0, klen, tid);
  store_tile<LA, C::BM>(ra, stage0, tid, k0, klen);
  store_tile<LB, C::BN>(rb, stage0 + C::A_BYTES, tid, k0, klen);
  __syncthreads();

  // Pipeline: while k-tile kt is multiplied from LDS stage kt % 2, the
  // registers holding k-tile kt + 1 are written to the other stage, part by
  // part, and refilled with k-tile kt + 2.
  auto advance = [&]() {
    k0 += kBK;
    if (k0 >= klen) {
      ++seg;
      k0 = 0;
      klen = pb.seg[seg].k_len;
      setup_tile<LA, C::BM>(ia, pb.seg[seg].a, m0, pb.M, tid);
      setup_tile<LB, C::BN>(ib, pb.seg[seg].b, n0, pb.N, tid);
    }
  };
  if (nk > 1) {
    advance();
    load_tile<LA, C::BM>(ra, ia, k0, klen, tid);
    load_tile<LB, C::BN>(rb, ib, k0, klen, tid);
  }
  int kt = 0;
  for (; kt + 2 < nk; ++kt) {
    char* st = (kt & 1) ? stage1 : stage0;
    char* nx = (kt & 1) ? stage0 : stage1;
    const int k0s = k0, klens = klen;  // the tile in registers
    advance();                         // the tile to load
    zero_tail<LA, C::BM>(ra, k0s, klens, tid);
    zero_tail<LB, C::BN>(rb, k0s, klens, tid);
    mma_tile_pipelined<C, LA, LB, true>(acc, st, st + C::A_BYTES, wm, wn, lane, ra, rb, nx, ia, ib,
                                        k0, klen, tid);
    __syncthreads();
  }
  if (kt + 1 < nk) {
    char* st = (kt & 1) ? stage1 : stage0;
    char* nx = (kt & 1) ? stage0 : stage1;
    zero_tail<LA, C::BM>(ra, k0, klen, tid);
    zero_tail<LB, C::BN>(rb, k0, klen, tid);
    mma_tile_pipelined<C, LA, LB, false>(acc, st, st + C::A_BYTES, wm, wn, lane, ra, rb, nx, ia,
                                         ib, k0, klen, tid);
    __syncthreads();
    ++kt;
  }
  char* st = (kt & 1) ? stage1 : stage0;
  mma_tile<C>(acc, st, st + C::A_BYTES, wm, wn, lane);
  __syncthreads();  // the epilogue may reuse the LDS
}

// ---------------------------------------------- direct-to-LDS main loop --
// For the 256 x 256 tile with a K-major A operand. The LDS-staged loop is
// bound by LDS traffic (stores through VGPRs plus fragment reads); here the
// K-major operands go from global memory straight into LDS with
// global_load_lds_dwordx4, which writes lane l's 16 bytes at LDS offset
// 16 l of the instruction's base. One instruction fills an 8-row group
// (1 KB) of the [rows][64 k] tile: lane l lands on row l / 8, physical
// chunk l % 8, so it fetches logical chunk (l % 8) ^ swz(row) - the swizzle
// is applied on the global side. Wave w fills groups w + 4 i. An MN-major B
// keeps the register path (transposed on its way into LDS). The two LDS
// stages are distinct __shared__ arrays and the loop is unrolled by two, so
// the compiler sees that reads of one stage do not alias the loads into the
// other and does not wait for them.
// The lane id through an opaque move: values derived from it inside a rarely
// taken branch (segment switch, partial tile) are computed there instead of
// being hoisted out of the main loop and held in registers across it.
__device__ __forceinline__ int opaque_lane() {
  int l = threadIdx.x;
  asm volatile("v_mov_b32 %0, %1" : "=v"(l) : "v"(l));
  return l & 63;
}

template <int ROWS>
struct DtlIter {
  const char* base;            // uniform: tile origin at k = 0 of the segment
  uint32_t off[ROWS / 32];     // group i: byte offset of this lane's row and chunk
};

template <int ROWS>
__device__ __forceinline__ void setup_dtl(DtlIter<ROWS>& it, const Operand& op, int row0, int rows,
                                          int wave) {
  const int lane = opaque_lane();
  it.base = reinterpret_cast<const char*>(op.ptr + (int64_t)row0 * op.ld);
  const int last = rows - 1 - row0;
#pragma unroll
  for (int i = 0; i < ROWS / 32; ++i) {
    const int r = 8 * (wave + 4 * i) + (lane >> 3);
    const int c = (lane & 7) ^ swz(r);
    const int rc = r < last ? r : last;
    it.off[i] = (uint32_t)(((int64_t)rc * op.ld + 8 * c) * 2);
  }
}

// Loads the k-tile at k0 (< klen) into the LDS tile `lds`. In a segment's
// last, partial tile the lanes whose chunk lies past klen load the tile
// origin instead (in bounds); dtl_zero_tail overwrites those chunks.
template <int ROWS>
__device__ __forceinline__ void dtl_load(const DtlIter<ROWS>& it, char* lds, int k0, int klen,
                                         int wave) {
  const char* b = it.base + (int64_t)k0 * 2;
  if (k0 + kBK <= klen) {
#pragma unroll
    for (int i = 0; i < ROWS / 32; ++i) {
      auto* dst = (__attribute__((address_space(3))) void*)(lds + (wave + 4 * i) * 1024);
      const void* src = b + it.off[i];  // (a named pointer: the host pass rejects the inline form)
      __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
    }
  } else {
    const int l = opaque_lane();
#pragma unroll
    for (int i = 0; i < ROWS / 32; ++i) {
      auto* dst = (__attribute__((address_space(3))) void*)(lds + (wave + 4 * i) * 1024);
      const int r = 8 * (wave + 4 * i) + (l >> 3);
      const uint32_t off = k0 + 8 * ((l & 7) ^ swz(r)) < klen ? it.off[i] : 0u;
      const void* src = b + off;
      __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
    }
  }
}

// For a partial k-tile: waits for this wave's direct loads, then zeroes the
// chunks its lanes loaded past klen (each lane owns the 16 bytes its load
// wrote). Call before the barrier that publishes the tile.
template <int ROWS>
__device__ __forceinline__ void dtl_zero_tail(char* lds, int k0, int klen, int wave) {
  if (k0 + kBK <= klen) return;
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  const int l = opaque_lane();
#pragma unroll
  for (int i = 0; i < ROWS / 32; ++i) {
    const int r = 8 * (wave + 4 * i) + (l >> 3);
    if (k0 + 8 * ((l & 7) ^ swz(r)) >= klen)
      *reinterpret_cast<u32x4*>(lds + (wave + 4 * i) * 1024 + 16 * l) = u32x4{0u, 0u, 0u, 0u};
  }
}

// One k-step: fragment reads of step S + 1, MFMAs of step S and, for a
// register-staged B, part S of its LDS store (SB) and reload (RB).
template <class C, int LB, bool SB, bool RB, int S>
__device__ __forceinline__ void dtl_step(f32x16_t (&acc)[C::TM][C::TN], Frags<C>& fnext,
                                         const Frags<C>& fcur, const char* As, const char* Bs,
                                         int wm, int wn, int lane, TileRegs& rb, char* nxtB,
                                         const char* bB, const TileIter& ib, int k0B, int klenB,
                                         int tid) {
  constexpr int kReads = S < 3 ? C::TM + C::TN : 0;
  constexpr int kWb = SB ? store_count<LB, C::BN>(S) : 0;
  constexpr int kLb = RB ? reload_count<LB, C::BN>(S) : 0;
  constexpr int kB0 = LB == kMNMajor ? kWb : 0;
  constexpr int kMfma = C::TM * C::TN;
  constexpr int kMax1 = kReads > kWb ? kReads : kWb;
  constexpr int kMax2 = kMax1 > kB0 + kLb ? kMax1 : kB0 + kLb;
  constexpr int kSlots = kMfma > kMax2 ? kMfma : kMax2;
  static_for<kSlots>([&](auto qc) {
    constexpr int q = decltype(qc)::value;
    if constexpr (q < kReads) read_frag<C, q>(fnext, As, Bs, wm, wn, lane, S + 1);
    if constexpr (q < kWb) store_one<LB, C::BN, S, q>(rb, nxtB, tid);
    if constexpr (q >= kB0 && q < kB0 + kLb)
      reload_one<LB, C::BN, S, q - kB0>(rb, bB, ib, k0B, klenB, tid);
    if constexpr (q < kMfma) {
      constexpr int i = q / C::TN, j = q % C::TN;
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fcur.a[i], fcur.b[j], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  });
}

template <class C, int LB, bool SB, bool RB>
__device__ __forceinline__ void dtl_tile(f32x16_t (&acc)[C::TM][C::TN], const char* st, int wm,
                                         int wn, int lane, TileRegs& rb, char* nxtB,
                                         const TileIter& ib, int k0B, int klenB, int tid) {
  const char* As = st;
  const char* Bs = st + C::A_BYTES;
  Frags<C> f0, f1;
  load_frags<C>(f0, As, Bs, wm, wn, lane, 0);
  __builtin_amdgcn_sched_barrier(0);
  const char* bB = ib.base + (int64_t)k0B * ib.kstride;
  dtl_step<C, LB, SB, RB, 0>(acc, f1, f0, As, Bs, wm, wn, lane, rb, nxtB, bB, ib, k0B, klenB, tid);
  dtl_step<C, LB, SB, RB, 1>(acc, f0, f1, As, Bs, wm, wn, lane, rb, nxtB, bB, ib, k0B, klenB, tid);
  dtl_step<C, LB, SB, RB, 2>(acc, f1, f0, As, Bs, wm, wn, lane, rb, nxtB, bB, ib, k0B, klenB, tid);
  dtl_step<C, LB, SB, RB, 3>(acc, f0, f1, As, Bs, wm, wn, lane, rb, nxtB, bB, ib, k0B, klenB, tid);
}

template <class C, int LB>
__device__ __forceinline__ void mainloop_dtl(const Problem& pb, int tm, int tn, int split,
                                             char* stage0, char* stage1,
                                             f32x16_t (&acc)[C::TM][C::TN]) {
  static_assert(C::BM == 256 && C::BN == 256, "direct-to-LDS path: 256 x 256 tiles");
  constexpr bool kBDtl = LB == kKMajor;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave / C::WAVES_N) * C::WM;
  const int wn = (wave % C::WAVES_N) * C::WN;
  const int m0 = tm * C::BM;
  const int n0 = tn * C::BN;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  int nk, k0 = 0;
  if (pb.ksplit > 1) {
    const int total = (pb.seg[0].k_len + kBK - 1) / kBK;
    const int first = split * pb.kps;
    nk = total - first < pb.kps ? total - first : pb.kps;
    k0 = first * kBK;
  } else {
    nk = 0;
    for (int s = 0; s < pb.nseg; ++s) nk += (pb.seg[s].k_len + kBK - 1) / kBK;
  }
  if (nk <= 0) return;

  // Cursors over the K segments: the direct loads run one k-tile ahead of
  // the tile being multiplied, a register-staged B two.
  int segA = 0, k0A = k0, klenA = pb.seg[0].k_len;
  int segB = 0, k0B = k0, klenB = pb.seg[0].k_len;
  DtlIter<C::BM> ita;
  DtlIter<C::BN> itb;
  TileIter ib;
  TileRegs rb;
  setup_dtl<C::BM>(ita, pb.seg[0].a, m0, pb.M, wave);
  if constexpr (kBDtl) setup_dtl<C::BN>(itb, pb.seg[0].b, n0, pb.N, wave);
  else setup_tile<LB, C::BN>(ib, pb.seg[0].b, n0, pb.N, tid);

  auto advanceA = [&]() __attribute__((always_inline)) {
    k0A += kBK;
    if (k0A >= klenA) {
      ++segA;
      k0A = 0;
      klenA = pb.seg[segA].k_len;
      setup_dtl<C::BM>(ita, pb.seg[segA].a, m0, pb.M, wave);
      if constexpr (kBDtl) setup_dtl<C::BN>(itb, pb.seg[segA].b, n0, pb.N, wave);
    }
  };
  auto advanceB = [&]() __attribute__((always_inline)) {  // register-staged B only
    k0B += kBK;
    if (k0B >= klenB) {
      ++segB;
      k0B = 0;
      klenB = pb.seg[segB].k_len;
      setup_tile<LB, C::BN>(ib, pb.seg[segB].b, n0, pb.N, tid);
    }
  };

  // k-tile 0 -> stage 0; a register-staged B also takes k-tile 1 into registers
  dtl_load<C::BM>(ita, stage0, k0A, klenA, wave);
  if constexpr (kBDtl) dtl_load<C::BN>(itb, stage0 + C::A_BYTES, k0A, klenA, wave);
  dtl_zero_tail<C::BM>(stage0, k0A, klenA, wave);
  if constexpr (kBDtl) {
    dtl_zero_tail<C::BN>(stage0 + C::A_BYTES, k0A, klenA, wave);
  } else {
    load_tile<LB, C::BN>(rb, ib, k0B, klenB, tid);
    store_tile<LB, C::BN>(rb, stage0 + C::A_BYTES, tid, k0B, klenB);
    if (nk > 1) {
      advanceB();
      load_tile<LB, C::BN>(rb, ib, k0B, klenB, tid);
    }
  }
  __syncthreads();

  // k-tile t: loads of k-tile t + 1 into stage nx, multiply from stage st.
  // One code path for every t (no branch around the MFMAs, whose 256
  // accumulators would otherwise be merged and copied): past the last
  // k-tile the cursors stay put and the same tile is loaded again into the
  // stage that is no longer read.
  auto iteration = [&](int t, char* st, char* nx) __attribute__((always_inline)) {
    if (t + 1 < nk) advanceA();
    dtl_load<C::BM>(ita, nx, k0A, klenA, wave);
    if constexpr (kBDtl) dtl_load<C::BN>(itb, nx + C::A_BYTES, k0A, klenA, wave);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kBDtl) {
      dtl_tile<C, LB, false, false>(acc, st, wm, wn, lane, rb, nullptr, ib, 0, 0, tid);
    } else {
      const int k0s = k0B, klens = klenB;  // B in registers (k-tile t + 1)
      if (t + 2 < nk) advanceB();          // B to load (k-tile t + 2)
      zero_tail<LB, C::BN>(rb, k0s, klens, tid);
      dtl_tile<C, LB, true, true>(acc, st, wm, wn, lane, rb, nx + C::A_BYTES, ib, k0B, klenB, tid);
    }
    dtl_zero_tail<C::BM>(nx, k0A, klenA, wave);
    if constexpr (kBDtl) dtl_zero_tail<C::BN>(nx + C::A_BYTES, k0A, klenA, wave);
    __syncthreads();
  };
  int t = 0;
  for (; t + 1 < nk; t += 2) {
    iteration(t, stage0, stage1);
    iteration(t + 1, stage1, stage0);
  }
  if (t < nk) iteration(t, stage0, stage1);
}

// The GEMM kernel: mainloop + epilogue functor
//   epi(acc, m_base, n_base, lane, smem, split) with m_base / n_base the
//   origin of this wave's sub-tile. smem may be reused by the epilogue.
template <class C, int LA, int LB, class Epi>
__global__ __launch_bounds__(kThreads) void gemm_kernel(const Problem pb, const Epi epi) {
  __shared__ __attribute__((aligned(16))) char stage0[C::STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char stage1[C::STAGE_BYTES];
  char* smem = stage0;
  int tm, tn, split;
  if (!tile_coords(pb, tm, tn, split)) return;
  f32x16_t acc[C::TM][C::TN];
  if constexpr (LA == kKMajor && C::BM == 256 && C::BN == 256)
    mainloop_dtl<C, LB>(pb, tm, tn, split, stage0, stage1, acc);
  else
    mainloop<C, LA, LB>(pb, tm, tn, split, stage0, stage1, acc);
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  epi(acc, tm * C::BM + (wave / C::WAVES_N) * C::WM, tn * C::BN + (wave % C::WAVES_N) * C::WN,
      tid & 63, smem, split);
}

// --------------------------------------------------------------- epilogues --

// C = alpha * acc + beta * C (C of type TC, row-major with ldc).
template <typename TC>
struct EpiStore {
  TC* C;
  int64_t ldc;
  int M, N;
  float alpha, beta;

  template <int TM, int TN>
  __device__ __forceinline__ void operator()(f32x16_t (&acc)[TM][TN], int m0, int n0, int lane,
                                             char*, int) const {
    const int col = lane & 31;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + 32 * j + col;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
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

// fp32 partial tile of split s at P[s][m][n] (dense M x N per split).
struct EpiPartial {
  float* P;
  int M, N;

  template <int TM, int TN>
  __device__ __forceinline__ void operator()(f32x16_t (&acc)[TM][TN], int m0, int n0, int lane,
                                             char*, int split) const {
    const int col = lane & 31;
    float* base = P + (int64_t)split * M * N;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + 32 * j + col;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int m = m0 + 32 * i + acc_row(v, lane);
          if (m < M) base[(int64_t)m * N + n] = acc[i][j][v];
        }
    }
  }
};

// out[m, n] = alpha * sum_s P[s][m][n] + beta * out[m, n]  (fixed order)
template <typename TC>
__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* __restrict__ P,
                                                              int ksplit, int M, int N,
                                                              TC* __restrict__ out, int64_t ldo,
                                                              float alpha, float beta) {
  const int64_t total = (int64_t)M * N;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * 256) {
    float s = 0.f;
    for (int k = 0; k < ksplit; ++k) s += P[(int64_t)k * total + e];
    const int64_t m = e / N, n = e - m * N;
    TC* p = out + m * ldo + n;
    float r = alpha * s;
    if (beta != 0.f) r += beta * to_f32(*p);
    *p = from_f32<TC>(r);
  }
}

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

template <class C>
inline int make_problem(Problem& pb, int M, int N, int nseg, const Segment* segs, int la, int lb,
                        int group_m, int ksplit = 1) {
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
  int w = 0;
  for (int s = 0; s < pb.nseg; ++s)
    if (pb.seg[s].k_len > 0) pb.seg[w++] = pb.seg[s];
  pb.nseg = w;
  pb.tiles_m = (M + C::BM - 1) / C::BM;
  pb.tiles_n = (N + C::BN - 1) / C::BN;
  pb.group_m = min(group_m > 0 ? group_m : ML_GEMM_GROUP_M, pb.tiles_m);
  pb.ksplit = 1;
  pb.kps = 0;
  if (ksplit > 1 && pb.nseg == 1) {
    const int total = (pb.seg[0].k_len + kBK - 1) / kBK;
    const int kps = (total + ksplit - 1) / ksplit;
    pb.kps = kps;
    pb.ksplit = (total + kps - 1) / kps;  // no empty splits
  }
  return ML_OK;
}

// Big-tile launch with the store epilogue.
template <typename TC>
inline int launch_store(const Problem& pb, int la, int lb, void* C, int64_t ldc, float alpha,
                        float beta, hipStream_t st) {
  EpiStore<TC> epi{static_cast<TC*>(C), ldc, pb.M, pb.N, alpha, beta};
  const dim3 grid(grid_blocks(pb));
#define ML_G(LA, LB) gemm_kernel<BigCfg, LA, LB, EpiStore<TC>><<<grid, kThreads, 0, st>>>(pb, epi)
  if (la == kKMajor && lb == kKMajor) ML_G(kKMajor, kKMajor);
  else if (la == kKMajor && lb == kMNMajor) ML_G(kKMajor, kMNMajor);
  else if (la == kMNMajor && lb == kKMajor) ML_G(kMNMajor, kKMajor);
  else ML_G(kMNMajor, kMNMajor);
#undef ML_G
  ML_LAUNCH_CHECK();
  return ML_OK;
}

// Split-K product of shape C into fp32 partials ws (ksplit * M * N floats),
// then out = alpha * sum + beta * out.
template <class C, int LA, int LB, typename TC>
inline int launch_splitk(const Problem& pb, float* ws, TC* out, int64_t ldo, float alpha, float beta,
                         hipStream_t st) {
  EpiPartial epi{ws, pb.M, pb.N};
  gemm_kernel<C, LA, LB, EpiPartial><<<dim3(grid_blocks(pb)), kThreads, 0, st>>>(pb, epi);
  ML_LAUNCH_CHECK();
  const int64_t total = (int64_t)pb.M * pb.N;
  int64_t blocks = (total + 255) / 256;
  blocks = blocks < 2048 ? blocks : 2048;
  reduce_partials_kernel<TC><<<dim3((unsigned)blocks), 256, 0, st>>>(ws, pb.ksplit, pb.M, pb.N,
                                                                     out, ldo, alpha, beta);
  ML_LAUNCH_CHECK();
  return ML_OK;
}

inline size_t splitk_ws_bytes(const Problem& pb) {
  return (size_t)pb.ksplit * (size_t)pb.M * (size_t)pb.N * sizeof(float);
}

}  // namespace gemm
}  // namespace mla

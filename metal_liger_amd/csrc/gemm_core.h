// bf16 MFMA GEMM core for gfx950 (CDNA4): C[M,N] = sum_k A[m,k] * B[k,n],
// fp32 accumulation, pluggable epilogue. The engines share the problem
// description, the tile order and the epilogues:
//
// 256 x 256 tiles (every large product), v_mfma_f32_16x16x32_bf16, operands
//   filled into LDS by buffer_load ... lds straight from global memory in
//   both layouts, transposing LDS reads (ds_read_b64_tr_b16) for MN-major
//   operands; two engines:
//   - 8 waves, two per SIMD in ping-pong, k-tiles of 32, four LDS stages
//     (see "256 x 256" below): the FLCE dW product, the FLCE products of a
//     repeated (retain_graph) backward and the products with an MN-major A;
//   - r4: 4 waves of 128 x 128, k-tiles of 64, five 32 KB operand slots
//     (see "r4" below):
//     the products with a K-major A (LoRA forward / dX / dH, the FLCE logits
//     and dH products, the plain GEMM entry points).
// Narrow tiles Cfg<BM, BN, WAVES_M> (256 x 32, 64 x 256: the rank-r LoRA
//   products, which would waste most of a 256 x 256 tile on padding):
//   256 threads = 4 wave64s in a WAVES_M x (4 / WAVES_M) grid; a wave owns a
//   (BM / WAVES_M) x (BN / WAVES_N) sub-tile of 32 x 32 tiles of
//   v_mfma_f32_32x32x16_bf16. BK = 64; both operand layouts are staged
//   through registers into LDS as [rows][64 k] bf16 (128-byte rows, 16-byte
//   chunks XOR-swizzled for conflict-free ds_read_b128 fragment reads);
//   MN-major tiles are transposed in registers (8 x 8 bf16 blocks,
//   v_perm_b32) on their way in. Two LDS stages, one barrier per k-tile.
// Operand layouts (per operand, "rows" = M for A, N for B)
//   K-major : element (r, k) at p[r * ld + k]   (A row-major, F.linear weight)
//   MN-major: element (r, k) at p[k * ld + r]   (A^T stored, B row-major)
// K segments
//   K may be a concatenation of up to kMaxSeg segments with their own A/B
//   pointers and leading dimensions (e.g. [dQ | dK | dV | lora] against
//   [Wq; Wk; Wv; A]); a segment's last k-tile is zero-filled past its end.
// Split-K
//   with ksplit > 1 (single segment), split s accumulates the 64-wide
//   k-tiles [s * kps, (s + 1) * kps) and the epilogue receives s;
//   EpiPartial writes fp32 partial tiles that reduce_partials_kernel sums in
//   a fixed order.
// Tile order
//   workgroups are dispatched round-robin over the 8 XCDs, so block b is
//   remapped to logical work item (b % 8) * ceil(W/8) + b / 8: each XCD walks
//   a contiguous range, ordered m-fastest within groups of group_m m-tiles,
//   so concurrently running tiles of one XCD share operands in its L2.
#pragma once

#include <type_traits>
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
// resident per XCD, groups of 4 give each XCD a 4 x 8 patch of tiles.
#ifndef ML_GEMM_GROUP_M
#define ML_GEMM_GROUP_M 4
#endif


// ENGINE_ selects the engine of the 256 x 256 tile: 1 = the big engine (8
// waves, 32-deep k-tiles), 2 = r4 (4 waves, 64-deep k-tiles).
template <int BM_, int BN_, int WAVES_M_, int ENGINE_ = 1>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, ENGINE = ENGINE_;
  static constexpr int WAVES_M = WAVES_M_, WAVES_N = 4 / WAVES_M_;
  static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  static constexpr int TM = WM / 32, TN = WN / 32;
  static constexpr int A_BYTES = BM * kRowBytes, B_BYTES = BN * kRowBytes;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int LDS_BYTES = 2 * STAGE_BYTES;
  // the 256 x 256 tile runs its own engines (8 waves, or 4 for r4)
  static constexpr int THREADS = (BM_ == 256 && BN_ == 256) ? (ENGINE_ == 2 ? 256 : 512) : 256;
  static_assert(WAVES_M * WAVES_N == 4, "4 waves per block");
  static_assert(TM >= 1 && TN >= 1 && WM % 32 == 0 && WN % 32 == 0, "wave tile of 32x32 MFMAs");
  static_assert(BM <= 256 && BN <= 256, "at most one 16-byte chunk set per thread");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
};

using BigCfg = Cfg<256, 256, 2>;   // 2 x 4 waves of 128 x 64 (its own engine)
using R4Cfg = Cfg<256, 256, 2, 2>; // 4 waves of 128 x 128 (the r4 engine)
using TallCfg = Cfg<256, 32, 4>;   // 4 x 1 waves of 64 x 32  (rank-r wide outputs)
using WideCfg = Cfg<64, 256, 1>;   // 1 x 4 waves of 64 x 64  (few-row outputs)


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
// bid: the block's index among the product's blocks (blockIdx.x, or its
// offset inside a grouped launch, whose products start at multiples of 8)
__device__ __forceinline__ bool tile_coords(const Problem& pb, int bid, int& tm, int& tn,
                                            int& split) {
  const int W = pb.tiles_m * pb.tiles_n * pb.ksplit;
  const int W8 = (W + kXcds - 1) / kXcds;
  const int logical = (bid % kXcds) * W8 + bid / kXcds;
  if (logical >= W) return false;
  // the split is the slowest index: an XCD's concurrent workgroups take
  // the tiles of one K range, sharing its A rows and B columns in L2 (split
  // fastest, every tile's splits ran on one XCD and the FLCE dH product
  // re-read its 0.62 GB operands ~5x from HBM)
  const int tiles = pb.tiles_m * pb.tiles_n;
  split = logical / tiles;
  const int t = logical - split * tiles;
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

// The lane id through an opaque move: values derived from it inside a rarely
// taken branch (a K-segment switch) are computed there instead of being
// hoisted out of the main loop and held in registers across it.
__device__ __forceinline__ int opaque_lane() {
  int l = threadIdx.x;
  asm volatile("v_mov_b32 %0, %1" : "=v"(l) : "v"(l));
  return l & 63;
}

// ============================================================ 256 x 256 ==
// The big tile runs its own engine:
//   v_mfma_f32_16x16x32_bf16 (on gfx950 it sustains a larger share of the
//   matrix-core peak than the 32x32x16 form), a wave tile of 128 x 128 =
//   8 x 8 MFMA tiles (256 fp32 accumulators, AGPRs), k-tiles of 32, and four
//   LDS stages of 32 KB, so that loads run three k-tiles ahead of their use.
// Both operands, in either layout, go global -> LDS with
// buffer_load_dwordx4 ... lds (lane l's 16 bytes land at LDS offset 16 l of
// the instruction's base; one instruction fills 1 KB), unconverted:
//   K-major tile  [256 rows][32 k]   64-byte rows; the 16-byte chunk c of
//                                    row r sits at chunk c ^ kswz(r),
//                                    kswz(r) = ((r >> 1) ^ (r >> 2)) & 3
//   MN-major tile [32 k][256 rows]   512-byte k-rows; the 32-byte unit u of
//                                    k-row r sits at unit u ^ h(r),
//                                    h(r) = (r & 3) | ((r >> 3) & 1) << 2
// (the swizzles are applied on the global side: each lane fetches the data
// its LDS slot holds). Fragments are read with ds_read_b128 (K-major) or
// with two ds_read_b64_tr_b16 (MN-major). The transposing read returns, per
// 16-lane group, lane i element j = element (i mod 4) of the 8 bytes
// addressed by lane 4 j + i / 4; with lane 4 a + b addressing rows 4 b ..
// 4 b + 3 of k-row a, lane i receives row i at 4 consecutive k, which is the
// MFMA operand layout. Both swizzles keep every 8-lane group of a fragment
// read within distinct 16-byte bank groups of a 128-byte window (and every
// 16-lane group within a 256-byte one): the reads are free of bank conflicts.
// A lane whose k lies past the end of its K segment loads from an offset past
// the buffer resource's range; the hardware writes zeros for it.
// Pipeline, per k-tile t (stage t % 4):
//   wait for this wave's loads of k-tile t + 1, barrier (publishes t + 1;
//   every wave has its fragments of t in registers, so stage t % 4 is free);
//   the 64 MFMAs of k-tile t, with the fragment reads of k-tile t + 1 in the
//   first 32 slots and the 8 loads of k-tile t + 4 into stage t % 4 in the
//   last 32.

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

namespace big {
constexpr int THREADS = 512;  // 8 waves: two per SIMD
constexpr int BK = 32;
constexpr int TM = 8, TN = 4;  // 16 x 16 MFMA tiles per wave
constexpr int WM = 128, WN = 64;
constexpr int OP_BYTES = 256 * BK * 2;  // 16 KB per operand per stage
constexpr int STAGE_BYTES = 2 * OP_BYTES;
#ifndef ML_BIG_STAGES
#define ML_BIG_STAGES 4
#endif
constexpr int STAGES = ML_BIG_STAGES;
constexpr int DIST = STAGES - 1;  // k-tiles loaded ahead of the one being read
constexpr int LOADS = 2;  // 1-KB loads per wave per operand per k-tile
constexpr int EPI_BYTES = 16384;  // LDS per wave for the epilogue
static_assert(8 * EPI_BYTES <= STAGES * STAGE_BYTES, "epilogue LDS inside the stages");
// s_waitcnt immediate (gfx9 encoding) for vmcnt(n), other counters ignored.
constexpr int wait_vm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }
// With DIST k-tiles of 2 * LOADS loads per wave in flight, k-tile t + 1 has
// landed once at most (DIST - 1) * 2 * LOADS remain.
constexpr int kWaitVmAhead = wait_vm((DIST - 1) * 2 * LOADS);
constexpr int kWaitVm0 = wait_vm(0);
constexpr uint32_t kOob = 0x80000000u;  // past every resource range used here
constexpr uint32_t kRange = 0x7FFFFFFFu;
constexpr uint32_t kDword3 = 0x00020000u;  // raw buffer, 32-bit data format
}  // namespace big

// Raw buffer resource (4 uniform dwords): base, stride 0, range, format.
typedef unsigned int rsrc_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ rsrc_t make_rsrc(const char* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  rsrc_t r;
  r[0] = __builtin_amdgcn_readfirstlane((uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xFFFFu);
  r[2] = big::kRange;
  r[3] = big::kDword3;
  return r;
}

__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p);
}

// buffer_load_dwordx4 ... lds. Issued as inline assembly so that the
// compiler inserts no waits of its own for it: the main loop keeps its own
// vmcnt accounting (s_waitcnt with explicit counts before each barrier) and
// has no other vector-memory operation in flight.
// (m0 is a reserved register: the compiler keeps nothing in it across this
// code - no other instruction of these kernels reads it - so its clobber is
// declared and the warning about clobbering a reserved register is muted.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void buf_load_lds(rsrc_t r, uint32_t voff, char* lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(r), "s"(lds_addr(lds))
               : "m0");
}
// The 4-byte form: lane l's dword lands at LDS offset 4 l (256 B per instruction).
__device__ __forceinline__ void buf_load_lds_dword(rsrc_t r, uint32_t voff, char* lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(r), "s"(lds_addr(lds))
               : "m0");
}
#pragma clang diagnostic pop

// Chunk swizzle of the K-major tile (a function of the row's low 4 bits).
__device__ __forceinline__ int kswz(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }

// Loads of one operand for one k-tile.
template <int L>
struct BigIter {
  const char* base;  // uniform: operand at (first row of the tile, k = 0 of the segment)
  int64_t kstep;     // bytes per unit of k
  uint32_t off[big::LOADS];
  int kr[big::LOADS];  // MN-major: the k-row of each load
};

// Wave w (of 8) issues the 1-KB groups g = w + 8 i (i < 2) of each operand:
// rows 16 g .. 16 g + 15 (K-major) or k-rows 2 g, 2 g + 1 (MN-major).
template <int L>
__device__ __forceinline__ void big_setup(BigIter<L>& it, const Operand& op, int row0, int rows,
                                          int wave) {
  const int l = opaque_lane();
  if constexpr (L == kKMajor) {
    it.base = reinterpret_cast<const char*>(op.ptr + (int64_t)row0 * op.ld);
    it.kstep = 2;
    const int lc = (l & 3) ^ kswz(l >> 2);  // logical chunk of physical chunk l % 4 (row % 16 = l / 4)
    const int last = rows - 1 - row0;
#pragma unroll
    for (int i = 0; i < big::LOADS; ++i) {
      const int r = 16 * (wave + 8 * i) + (l >> 2);
      const int rc = r < last ? r : last;  // rows past the end re-read the last row
      it.off[i] = (uint32_t)(((int64_t)rc * op.ld + 8 * lc) * 2);
      it.kr[i] = 0;
    }
  } else {
    it.base = reinterpret_cast<const char*>(op.ptr + row0);
    it.kstep = 2 * op.ld;
    const int p = l & 31;  // physical 16-byte slot in the k-row
    const int last8 = rows - row0 - 8;  // last 8-row group of the operand (rows % 8 == 0)
#pragma unroll
    for (int i = 0; i < big::LOADS; ++i) {
      const int r = 2 * (wave + 8 * i) + (l >> 5);
      const int h = (r & 3) | (((r >> 3) & 1) << 2);
      int e = 8 * (2 * ((p >> 1) ^ h) + (p & 1));  // first row of the 8 this lane fetches
      e = e < last8 ? e : last8;
      it.off[i] = (uint32_t)(((int64_t)r * op.ld + e) * 2);
      it.kr[i] = r;
    }
  }
}

// Per-lane LDS byte offsets (within an operand tile) of the fragment reads
// of a wave whose sub-tile starts at row wbase of the block tile.
template <int L, int NF>
struct FragAddr {
  uint32_t a[L == kKMajor ? 1 : NF];
};

template <int L, int NF>
__device__ __forceinline__ void frag_addr_setup(FragAddr<L, NF>& fa, int wbase, int lane) {
  if constexpr (L == kKMajor) {
    // row wbase + 16 f + (lane & 15), chunk lane >> 4; the swizzle term
    // kswz(row) only depends on row % 16 = lane & 15
    fa.a[0] = (uint32_t)(wbase * 64 + (lane & 15) * 64 + (((lane >> 4) ^ kswz(lane & 15)) << 4));
  } else {
    // k-row 8 G + (i >> 2) (+ 4 for the second read), rows 4 (i & 3) .. of
    // the fragment's 32-byte unit wbase / 16 + f, swizzled by h(k-row) =
    // ((i >> 2) & 3) | (G & 1) << 2 (G = lane >> 4, i = lane & 15)
    const int G = lane >> 4, i = lane & 15;
    const int h = ((i >> 2) & 3) | ((G & 1) << 2);
    const uint32_t b = (uint32_t)((8 * G + (i >> 2)) * 512 + 8 * (i & 3));
#pragma unroll
    for (int f = 0; f < NF; ++f) fa.a[f] = b + (uint32_t)((((wbase >> 4) + f) ^ h) << 5);
  }
}

struct BigFrags {
  bf16x8_t a[big::TM], b[big::TN];
};

// Read q (compile time) of a k-tile's fragments: B first (the first MFMAs of
// a k-tile use every B fragment), then A; an MN-major fragment takes two
// transposing reads.
template <int L>
constexpr int reads_per_frag() { return L == kKMajor ? 1 : 2; }

template <int L, int NF>
__device__ __forceinline__ void read_big_frag(bf16x8_t& dst, const char* op,
                                              const FragAddr<L, NF>& fa, int f, int half) {
  if constexpr (L == kKMajor) {
    dst = *reinterpret_cast<const bf16x8_t*>(op + fa.a[0] + 1024 * f);
  } else {
    typedef __attribute__((address_space(3))) i16x4_t* lp;
    const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lp)(op + fa.a[f] + 2048 * half));
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    i16x8_t w = __builtin_bit_cast(i16x8_t, dst);
#pragma unroll
    for (int e = 0; e < 4; ++e) w[4 * half + e] = v[e];
    dst = __builtin_bit_cast(bf16x8_t, w);
  }
}

template <int LA, int LB, int Q>
__device__ __forceinline__ void big_read(BigFrags& f, const char* As, const char* Bs,
                                         const FragAddr<LA, big::TM>& fa,
                                         const FragAddr<LB, big::TN>& fb) {
  constexpr int RB = reads_per_frag<LB>(), RA = reads_per_frag<LA>();
  if constexpr (Q < big::TN * RB) {
    read_big_frag<LB>(f.b[Q / RB], Bs, fb, Q / RB, Q % RB);
  } else {
    constexpr int q = Q - big::TN * RB;
    read_big_frag<LA>(f.a[q / RA], As, fa, q / RA, q % RA);
  }
}

template <int L>
__device__ __forceinline__ uint32_t big_oob(const BigIter<L>& it, int i, bool live, int kc, int kb,
                                            int klen) {
  const int k = kc + (L == kKMajor ? kb : it.kr[i]);
  return (live && k < klen) ? 0u : big::kOob;
}

// A barrier the compiler schedules nothing across (the MFMA clusters and the
// memory clusters stay on their own side of it).
__device__ __forceinline__ void big_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
}

// Main loop of the big tile; lds holds STAGES stages of STAGE_BYTES (A tile,
// then B tile). Wave w = 4 g + s computes rows 128 g .. 128 g + 127 and
// columns 64 s .. 64 s + 63 of the block tile.
template <int LA, int LB>
__device__ __forceinline__ void big_mainloop(const Problem& pb, int tm, int tn, int split,
                                             char* lds, f32x4_t (&acc)[big::TM][big::TN]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  const int wm = grp * big::WM;
  const int wn = (wave & 3) * big::WN;
  const int m0 = tm * 256;
  const int n0 = tn * 256;
#pragma unroll
  for (int i = 0; i < big::TM; ++i)
#pragma unroll
    for (int j = 0; j < big::TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  int nk, k0 = 0;
  if (pb.ksplit > 1) {  // splits are counted in 64-wide k units
    const int total = (pb.seg[0].k_len + kBK - 1) / kBK;
    const int first = split * pb.kps;
    const int n64 = total - first < pb.kps ? total - first : pb.kps;
    k0 = first * kBK;
    const int kend = k0 + n64 * kBK < pb.seg[0].k_len ? k0 + n64 * kBK : pb.seg[0].k_len;
    nk = (kend - k0 + big::BK - 1) / big::BK;
  } else {
    nk = 0;
    for (int s = 0; s < pb.nseg; ++s) nk += (pb.seg[s].k_len + big::BK - 1) / big::BK;
  }
  // (nk is block-uniform: every wave returns here or none does)
  if (nk <= 0) return;

  // Load cursor: the next k-tile to load (segment seg, offset kc, length
  // klen); `loaded` k-tiles have been issued. Past the last k-tile the
  // cursor stays and every lane's load is out of range (zeros, no traffic).
  int seg = 0, kc = k0, klen = pb.seg[0].k_len, loaded = 0;
  BigIter<LA> ia;
  BigIter<LB> ib;
  big_setup<LA>(ia, pb.seg[0].a, m0, pb.M, wave);
  big_setup<LB>(ib, pb.seg[0].b, n0, pb.N, wave);
  const int kb = 8 * ((lane & 3) ^ kswz(lane >> 2));  // K-major lanes: k offset in a k-tile
  FragAddr<LA, big::TM> fa;
  FragAddr<LB, big::TN> fb;
  frag_addr_setup<LA, big::TM>(fa, wm, lane);
  frag_addr_setup<LB, big::TN>(fb, wn, lane);

  // Issues this wave's loads of the cursor's k-tile into stage dst.
  auto cursor_loads = [&](char* dst) __attribute__((always_inline)) {
    const bool live = loaded < nk;
    const rsrc_t ra = make_rsrc(ia.base + (int64_t)kc * ia.kstep);
    const rsrc_t rb = make_rsrc(ib.base + (int64_t)kc * ib.kstep);
#pragma unroll
    for (int i = 0; i < big::LOADS; ++i) {
      buf_load_lds(ra, ia.off[i] | big_oob<LA>(ia, i, live, kc, kb, klen),
                   dst + (wave + 8 * i) * 1024);
      buf_load_lds(rb, ib.off[i] | big_oob<LB>(ib, i, live, kc, kb, klen),
                   dst + big::OP_BYTES + (wave + 8 * i) * 1024);
    }
    ++loaded;
    if (loaded >= nk) return;
    kc += big::BK;
    if (kc >= klen) {
      ++seg;
      kc = 0;
      klen = pb.seg[seg].k_len;
      big_setup<LA>(ia, pb.seg[seg].a, m0, pb.M, wave);
      big_setup<LB>(ib, pb.seg[seg].b, n0, pb.N, wave);
    }
  };

  // Prologue: k-tiles 0 .. DIST - 1; k-tile 0 published by the barrier.
#pragma unroll
  for (int j = 0; j < big::DIST; ++j) cursor_loads(lds + j * big::STAGE_BYTES);
  __builtin_amdgcn_s_waitcnt(big::kWaitVmAhead);
  big_barrier();
  // Ping-pong: group 1 runs one phase behind group 0, so that while one
  // wave of a SIMD issues its MFMA cluster the other issues its loads and
  // fragment reads. Each k-tile t is two phases of a group:
  //   memory: loads of k-tile t + DIST into stage (t + DIST) % 4, the
  //           fragment reads of k-tile t, then a wait until this wave's loads
  //           of k-tile t + 1 have landed and its reads are in registers;
  //   compute: the 32 MFMAs of k-tile t.
  // A barrier ends every phase. Stage (t + DIST) % 4 last held k-tile t - 1,
  // whose last reads (group 1's memory phase of t - 1) ended before the
  // barrier that starts group 0's memory phase of t; k-tile t + 1 is
  // published by the barriers that end both groups' memory phases of t.
  if (grp == 1) big_barrier();
  BigFrags f;
  auto iteration = [&](const char* cur, char* ld) __attribute__((always_inline)) {
    cursor_loads(ld);
    static_for<big::TN * reads_per_frag<LB>() + big::TM * reads_per_frag<LA>()>([&](auto qc) {
      big_read<LA, LB, decltype(qc)::value>(f, cur, cur + big::OP_BYTES, fa, fb);
    });
    __builtin_amdgcn_s_waitcnt(big::kWaitVmAhead);
    big_barrier();
#pragma unroll
    for (int i = 0; i < big::TM; ++i)
#pragma unroll
      for (int j = 0; j < big::TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
    big_barrier();
  };
  // The body runs the stages in turn; the k-tile count is rounded up to a
  // multiple of STAGES (the extra k-tiles are zeros and add nothing).
  for (int t = 0; t < nk; t += big::STAGES) {
    static_for<big::STAGES>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      iteration(lds + j * big::STAGE_BYTES, lds + ((j + big::DIST) % big::STAGES) * big::STAGE_BYTES);
    });
  }
  if (grp == 0) big_barrier();
  __builtin_amdgcn_s_waitcnt(big::kWaitVm0);
  __syncthreads();  // loads past the end have landed; the epilogue may reuse the LDS
}

// ====================================================== 256 x 256, r4 ==
// The 256 x 256 tile on 4 waves, one per SIMD (R4Cfg):
//   each wave owns a 128 x 128 sub-tile, 8 x 8 v_mfma_f32_16x16x32_bf16 tiles
//   (256 fp32 accumulators, pinned to AGPRs); k-tiles of 64, so that a
//   K-major row of a tile is one whole 128-byte line; both operands go
//   global -> LDS by buffer_load_dwordx4 ... lds (lane l's 16 bytes land at
//   16 l of the instruction's 1 KB of LDS; no registers, no ds_write), two
//   stages of 64 KB:
//   K-major tile  [256 rows][64 k]   128-byte rows; 16-byte chunk c of row r
//                                    at chunk c ^ r4_swz(r), r4_swz(r) =
//                                    (r & 7) ^ ((r >> 3) & 1); an instruction
//                                    fills 8 rows with 8 whole lines
//   MN-major tile [64 k][256 rows]   512-byte k-rows; 32-byte unit u of k-row
//                                    r at unit u ^ mn_swz(r) (the big engine's
//                                    h(r)); an instruction fills 2 k-rows
// (the swizzles are applied on the global side: each lane fetches the data
// its LDS slot holds). K-major fragments are ds_read_b128 at one per-lane base
// plus a constant per fragment (the swizzle depends on the row modulo 16);
// MN-major fragments are two ds_read_b64_tr_b16 at a per-lane address per
// fragment. Both layouts keep a fragment read within distinct bank groups.
// Edges: each k-tile's buffer resource ends at the operand's last valid byte
// for this tile (K-major: the last valid row; MN-major: the last k-row of the
// K segment), so rows / k-rows past the end read zeros; per lane, K-major
// chunks past the segment's K and MN-major columns past N get an offset past
// every range (zeros as well). No load is ever issued out of the tensor.
// Pipeline: the 160 KB of LDS are five 32 KB operand slots; k-tile t sits
// in two of them, k-tile t + 1 in two more, and one is free. Per k-tile t:
//   phase 0: the 64 MFMAs of k-step 0 (fragments in registers), interleaved
//            with the fragment reads of k-step 1 and the 8 A loads of k-tile
//            t + 2 into the free slot (one every eighth MFMA); then each wave
//            waits for its loads of k-tile t + 1 and its LDS reads, and a
//            barrier publishes k-tile t + 1 and frees t's two slots;
//   phase 1: the 64 MFMAs of k-step 1, interleaved with the fragment reads of
//            k-step 0 of k-tile t + 1 and the 8 B loads of k-tile t + 2 into
//            t's A slot (t's B slot is the next free slot).
// A wave issues its loads in order with its MFMAs, so a load the memory
// pipeline cannot yet take holds the MFMAs behind it: the fifth slot lets
// the 16 loads of a k-tile spread over both phases instead of one (with two
// 64 KB stages and all 16 in phase 1 the products ran 1-2% slower; with
// them bunched into the first half of phase 1, 2-4% slower still).
namespace r4 {
constexpr int THREADS = 256;
constexpr int BK = 64;
constexpr int TM = 8, TN = 8;
constexpr int WM = 128, WN = 128;
constexpr int OP_BYTES = 256 * BK * 2;      // 32 KB: one operand of one k-tile
constexpr int LDS_BYTES = 5 * OP_BYTES;    // five operand slots
constexpr int LOADS = 8;                    // 1-KB loads per wave per operand per k-tile
constexpr int EPI_BYTES = 16384;            // per wave per 128 x 64 half of its sub-tile
static_assert(4 * 2 * EPI_BYTES <= LDS_BYTES, "epilogue LDS inside the slots");
constexpr uint32_t kOob = 0x80000000u;  // past every resource range used here
constexpr int64_t kRangeMax = 0x7FFFFFFF;
constexpr int kRsrcFlags = 0x00020000;  // raw buffer, 32-bit data format
}  // namespace r4

// A workgroup barrier ordering LDS operations only (each wave's LDS reads and
// writes complete before it, s_waitcnt lgkmcnt(0)); global loads in flight
// stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ int r4_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// readfirstlane returns int: each half goes through uint32_t before it is
// widened (a sign-extended low half would set every high bit).
__device__ __forceinline__ uint64_t uniform_u64(uint64_t v) {
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return lo | (hi << 32);
}

// Global-load state of one operand for one wave. Wave w issues, per k-tile,
// the 1-KB groups g = w + 4 i (i < 8) of the operand tile: rows 8 g .. 8 g +
// 7 (K-major) or k-rows 2 g, 2 g + 1 (MN-major). The uniform fields are kept
// in SGPRs; per k-tile the cursor adds kstep to base and subtracts it from
// range.
template <int L>
struct R4Load {
  uint64_t base;     // uniform: the operand at (tile's first row, the cursor's k)
  int64_t range;     // uniform: bytes from base to the end of the tile's valid data
  uint32_t kstep;    // uniform: bytes per k-tile
  uint32_t istride;  // uniform: bytes between the wave's consecutive groups
  uint32_t voff[2];  // per lane: byte offset for even / odd i (kOob: never loads)
  int kb;            // per lane, K-major: k offset of the lane's chunk within a k-tile
};

// Cursor at k = kc of a segment of length klen (kc < klen).
//   K-major: valid data ends with row (rows - 1 - row0), k = klen - 1; rows
//            past it start at or after that end.
//   MN-major: valid data ends with k-row (klen - 1 - kc), column rows - 1 - row0.
template <int L>
__device__ __forceinline__ void r4_setup(R4Load<L>& it, const Operand& op, int row0, int rows,
                                         int kc, int klen, int wave, int lane) {
  const int64_t ld = op.ld;
  const char* p = reinterpret_cast<const char*>(op.ptr);
  if constexpr (L == kKMajor) {
    it.base = uniform_u64(reinterpret_cast<uint64_t>(p + ((int64_t)row0 * ld + kc) * 2));
    it.range = (int64_t)uniform_u64((uint64_t)(((int64_t)(rows - row0 - 1) * ld + (klen - kc)) * 2));
    it.kstep = 2 * r4::BK;
    // group g = wave + 4 i: lane l holds row 8 g + l / 8, physical chunk l % 8,
    // i.e. logical chunk (l % 8) ^ r4_swz(row); the swizzle is the same for
    // every i (row % 16 = 8 (wave % 2) + l / 8)
    const int r = 8 * wave + (lane >> 3);
    const int c = (lane & 7) ^ r4_swz(r);
    it.voff[0] = it.voff[1] = (uint32_t)(((int64_t)r * ld + 8 * c) * 2);
    it.istride = __builtin_amdgcn_readfirstlane((uint32_t)(32 * ld * 2));
    it.kb = 8 * c;
  } else {
    it.base = uniform_u64(reinterpret_cast<uint64_t>(p + ((int64_t)kc * ld + row0) * 2));
    it.range = (int64_t)uniform_u64((uint64_t)(((int64_t)(klen - kc - 1) * ld + (rows - row0)) * 2));
    it.kstep = __builtin_amdgcn_readfirstlane((uint32_t)(r4::BK * ld * 2));
    // group g = wave + 4 i: lane l holds k-row kr = 2 g + l / 32 = 2 wave + 8 i +
    // l / 32, physical 16-byte slot l % 32 of it, i.e. logical 32-byte unit
    // (slot / 2) ^ h(kr), h(kr) = (kr & 3) | ((kr >> 3) & 1) << 2 = h0 | (i & 1) << 2
    const int kr = 2 * wave + (lane >> 5);
    const int slot = lane & 31;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int h = (kr & 3) | (e << 2);
      const int col = 16 * ((slot >> 1) ^ h) + 8 * (slot & 1);
      it.voff[e] = col < rows - row0 ? (uint32_t)(((int64_t)kr * ld + col) * 2) : r4::kOob;
    }
    it.istride = __builtin_amdgcn_readfirstlane((uint32_t)(8 * ld * 2));
    it.kb = 0;
  }
}

// Buffer resource and lane offsets of the cursor's k-tile (live: the k-tile
// exists; otherwise every load reads zeros); kc / klen: the cursor's k and
// its segment length (K-major chunks past klen read zeros).
template <int L>
__device__ __forceinline__ void r4_tile_rsrc(const R4Load<L>& it, int kc, int klen, bool live,
                                             rsrc_t& rs, uint32_t (&voffs)[2]) {
  int64_t range = it.range < r4::kRangeMax ? it.range : r4::kRangeMax;
  range = live ? range : 0;
  if constexpr (L == kKMajor) {
    voffs[0] = voffs[1] = kc + it.kb < klen ? it.voff[0] : r4::kOob;
  } else {
    voffs[0] = it.voff[0];
    voffs[1] = it.voff[1];
  }
  const uint64_t b = uniform_u64(it.base);
  rs[0] = (uint32_t)b;
  rs[1] = (uint32_t)(b >> 32) & 0xFFFFu;
  rs[2] = (uint32_t)__builtin_amdgcn_readfirstlane((int)range);
  rs[3] = (uint32_t)r4::kRsrcFlags;
}

// Per-lane fragment read offsets of a wave sub-tile starting at row wbase.
// K-major: one per k-step (fragment f adds 2048 f); MN-major: one per
// fragment (the second half adds 4 k-rows, k-step 1 adds 32 k-rows).
template <int L>
struct R4Frag {
  uint32_t a[L == kKMajor ? 2 : 8];
};

template <int L>
__device__ __forceinline__ void r4_frag_setup(R4Frag<L>& fa, int wbase, int lane) {
  if constexpr (L == kKMajor) {
    const int r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int s = 0; s < 2; ++s)
      fa.a[s] = (uint32_t)((wbase + r) * 128 + (((4 * s + g) ^ r4_swz(r)) << 4));
  } else {
    // lane 16 G + i: k-row 8 G + i / 4, columns wbase + 16 f + 4 (i % 4) .. + 3
    const int G = lane >> 4, i = lane & 15;
    const int h = ((i >> 2) & 3) | ((G & 1) << 2);
    const uint32_t b = (uint32_t)((8 * G + (i >> 2)) * 512 + 8 * (i & 3));
#pragma unroll
    for (int f = 0; f < 8; ++f) fa.a[f] = b + (uint32_t)((((wbase >> 4) + f) ^ h) << 5);
  }
}

// Fragment f of k-step s (an MN-major fragment is two transposing reads,
// combined into a fresh register).
template <int L>
__device__ __forceinline__ bf16x8_t r4_read_frag(const char* op, const R4Frag<L>& fa, int s, int f) {
  if constexpr (L == kKMajor) {
    return *reinterpret_cast<const bf16x8_t*>(op + fa.a[s] + 2048 * f);
  } else {
    typedef __attribute__((address_space(3))) i16x4_t* lp;
    const char* p = op + fa.a[f] + 16384 * s;
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lp)(p));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lp)(p + 2048));
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    const i16x8_t w = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8_t, w);
  }
}

// acc += a b on the matrix cores, with acc pinned to AGPRs and the operands
// to VGPRs (left to itself the register allocator splits the 256
// accumulators between AGPRs and VGPRs and copies them every k-step).
__device__ __forceinline__ void r4_mfma(f32x4_t& acc, const bf16x8_t& a, const bf16x8_t& b) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

struct R4Frags {
  bf16x8_t a[r4::TM], b[r4::TN];
};

// Main loop of the r4 engine; lds holds the five operand slots.
// Wave w computes rows 128 (w >> 1) .. + 127 and columns 128 (w & 1) .. +
// 127 of the block tile; acc[h][i][j] is MFMA tile (i, 4 h + j).
template <int LA, int LB>
__device__ __forceinline__ void r4_mainloop(const Problem& pb, int tm, int tn, int split, char* lds,
                                            f32x4_t (&acc)[2][r4::TM][4]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave >> 1) * r4::WM;
  const int wn = (wave & 1) * r4::WN;
  const int m0 = tm * 256;
  const int n0 = tn * 256;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int i = 0; i < r4::TM; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[h][i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  int nk, k0 = 0;
  if (pb.ksplit > 1) {  // splits are counted in 64-wide k-tiles
    const int total = (pb.seg[0].k_len + kBK - 1) / kBK;
    const int first = split * pb.kps;
    nk = total - first < pb.kps ? total - first : pb.kps;
    k0 = first * kBK;
  } else {
    nk = 0;
    for (int s = 0; s < pb.nseg; ++s) nk += (pb.seg[s].k_len + r4::BK - 1) / r4::BK;
  }
  if (nk <= 0) return;  // block-uniform

  // Load cursor: the next k-tile to load; `loaded` k-tiles have been issued.
  int seg = 0, kc = k0, klen = pb.seg[0].k_len, loaded = 0;
  R4Load<LA> ia;
  R4Load<LB> ib;
  r4_setup<LA>(ia, pb.seg[0].a, m0, pb.M, kc, klen, wave, lane);
  r4_setup<LB>(ib, pb.seg[0].b, n0, pb.N, kc, klen, wave, lane);
  R4Frag<LA> fa;
  R4Frag<LB> fb;
  r4_frag_setup<LA>(fa, wm, lane);
  r4_frag_setup<LB>(fb, wn, lane);

  rsrc_t rsa, rsb;
  uint32_t va[2], vb[2], sa, sb;
  // Resources of the cursor's k-tile (with its segment's group stride: the
  // cursor may move to the next segment before the loads are issued), then
  // advance the cursor.
  auto next_tile = [&]() __attribute__((always_inline)) {
    const bool live = loaded < nk;
    r4_tile_rsrc<LA>(ia, kc, klen, live, rsa, va);
    r4_tile_rsrc<LB>(ib, kc, klen, live, rsb, vb);
    sa = ia.istride;
    sb = ib.istride;
    ++loaded;
    if (loaded < nk) {
      kc += r4::BK;
      if (kc >= klen) {
        ++seg;
        kc = 0;
        klen = pb.seg[seg].k_len;
        r4_setup<LA>(ia, pb.seg[seg].a, m0, pb.M, 0, klen, wave, lane);
        r4_setup<LB>(ib, pb.seg[seg].b, n0, pb.N, 0, klen, wave, lane);
      } else {
        ia.base += ia.kstep;
        ia.range -= ia.kstep;
        ib.base += ib.kstep;
        ib.range -= ib.kstep;
      }
    }
  };
  // Load i (0 .. 7) of operand A (OPB false) or B of the current resources
  // into the operand slot `slot`.
  auto load = [&](auto opb, char* slot, int i) __attribute__((always_inline)) {
    char* dst = slot + (wave + 4 * i) * 1024;
    if constexpr (decltype(opb)::value)
      buf_load_lds(rsb, vb[i & 1] + (uint32_t)i * sb, dst);
    else
      buf_load_lds(rsa, va[i & 1] + (uint32_t)i * sa, dst);
  };
  using OpA = std::integral_constant<bool, false>;
  using OpB = std::integral_constant<bool, true>;

  // Five 32 KB operand slots: k-tile t in (ca, cb), t + 1 in (na, nb), and
  // a free slot fr. Phase 0 of k-tile t loads A of t + 2 into fr; phase 1
  // (after the barrier has freed ca and cb) loads B of t + 2 into ca.
  char* ca = lds;
  char* cb = lds + r4::OP_BYTES;
  char* na = lds + 2 * r4::OP_BYTES;
  char* nb = lds + 3 * r4::OP_BYTES;
  char* fr = lds + 4 * r4::OP_BYTES;
  R4Frags f0, f1;
  next_tile();
#pragma unroll
  for (int i = 0; i < r4::LOADS; ++i) load(OpA{}, ca, i);
#pragma unroll
  for (int i = 0; i < r4::LOADS; ++i) load(OpB{}, cb, i);
  next_tile();
#pragma unroll
  for (int i = 0; i < r4::LOADS; ++i) load(OpA{}, na, i);
#pragma unroll
  for (int i = 0; i < r4::LOADS; ++i) load(OpB{}, nb, i);
  __builtin_amdgcn_s_waitcnt(big::wait_vm(2 * r4::LOADS));  // this wave's k-tile 0 landed
  lds_barrier();
#pragma unroll
  for (int j = 0; j < r4::TN; ++j) f0.b[j] = r4_read_frag<LB>(cb, fb, 0, j);
#pragma unroll
  for (int i = 0; i < r4::TM; ++i) f0.a[i] = r4_read_frag<LA>(ca, fa, 0, i);

  // One phase: the 64 MFMAs of fragment set fc, with the reads of the next
  // k-step (k-step NS of slots ra_ / rb_) into fn interleaved; phase 0 moves
  // the cursor to k-tile t + 2 and issues its A loads into ld, phase 1 its
  // B loads into ld.
  auto phase = [&](auto pc, R4Frags& fc, R4Frags& fn, const char* ra_, const char* rb_, char* ld)
                   __attribute__((always_inline)) {
    constexpr int P = decltype(pc)::value;
    constexpr int NS = P ^ 1;
    if constexpr (P == 0) next_tile();
    static_for<r4::TM * r4::TN>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      constexpr int i = q / r4::TN, j = q % r4::TN;
      if constexpr ((q & 1) == 0 && q < 16) fn.b[q >> 1] = r4_read_frag<LB>(rb_, fb, NS, q >> 1);
      if constexpr ((q & 1) == 0 && q >= 16 && q < 32) fn.a[(q - 16) >> 1] = r4_read_frag<LA>(ra_, fa, NS, (q - 16) >> 1);
      if constexpr ((q & 7) == 3) {
        if constexpr (P == 0) load(OpA{}, ld, q >> 3);
        else load(OpB{}, ld, q >> 3);
      }
      r4_mfma(acc[j >> 2][i][j & 3], fc.a[i], fc.b[j]);
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  for (int t = 0; t < nk; ++t) {
    phase(std::integral_constant<int, 0>{}, f0, f1, ca, cb, fr);
    // this wave's loads of k-tile t + 1 have landed (only the A loads of
    // t + 2 may still be in flight); the barrier publishes them and frees
    // ca and cb
    __builtin_amdgcn_s_waitcnt(big::wait_vm(r4::LOADS));
    lds_barrier();
    phase(std::integral_constant<int, 1>{}, f1, f0, na, nb, ca);
    char* const oa = ca;
    char* const ob = cb;
    ca = na;
    cb = nb;
    na = fr;
    nb = oa;
    fr = ob;
  }
  // the epilogue reads the accumulators: wait for the last MFMAs (the
  // asm statements carry no hazard information for the compiler), and for
  // the loads past the end (they write LDS the epilogue reuses)
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_s_waitcnt(big::kWaitVm0);
  lds_barrier();  // every wave's reads are done; the epilogue may reuse the LDS
}

// Per-element view of a wave's accumulators: f(m, n, value) for the
// elements of MFMA-tile row i (for_each_acc_row) or of the whole wave
// sub-tile at (m0, n0) (for_each_acc), in either MFMA layout:
//   16 x 16 tiles (f32x4_t): element v of tile (i, j) is row 16 i + 4 (lane / 16) + v,
//                            column 16 j + lane % 16
//   32 x 32 tiles (f32x16_t): row 32 i + 8 (v / 4) + 4 (lane / 32) + v % 4,
//                            column 32 j + lane % 32
// The TN * (4 or 16) elements of a row are visited in the order (j, v).
template <int TM, int TN, class F>
__device__ __forceinline__ void for_each_acc_row(f32x4_t (&acc)[TM][TN], int i, int m0, int n0,
                                                 int lane, F&& f) {
  const int r0 = m0 + 16 * i + 4 * (lane >> 4), c0 = n0 + (lane & 15);
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) f(r0 + v, c0 + 16 * j, acc[i][j][v]);
}

template <int TM, int TN, class F>
__device__ __forceinline__ void for_each_acc_row(f32x16_t (&acc)[TM][TN], int i, int m0, int n0,
                                                 int lane, F&& f) {
  const int r0 = m0 + 32 * i + 4 * (lane >> 5), c0 = n0 + (lane & 31);
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) f(r0 + 8 * (v >> 2) + (v & 3), c0 + 32 * j, acc[i][j][v]);
}

template <typename AccT, int TM, int TN, class F>
__device__ __forceinline__ void for_each_acc(AccT (&acc)[TM][TN], int m0, int n0, int lane, F&& f) {
#pragma unroll
  for (int i = 0; i < TM; ++i) for_each_acc_row(acc, i, m0, n0, lane, f);
}

// ------------------------------------------------ staged bf16 epilogues --
// Global stores of single bf16 elements (the accumulator layout gives a lane
// one column of 4 consecutive rows) use a 64-lane instruction for 128 bytes
// in 2-byte pieces. Instead, a wave stages its 128 x 64 results, rounded to
// bf16, in LDS of its own (512 bytes per MFMA tile) and takes them back as rows of 8
// consecutive columns, one 16-byte vector per lane:
//   phase 1: lane (G = lane / 16, c = lane % 16) writes rows 4 G .. 4 G + 3 of
//            column c of each 16 x 16 block as one 8-byte ds_write_b64; the
//            blocks are stored column-major ([16 columns][16 rows]).
//   phase 2: two ds_read_b64_tr_b16 per 16-lane group read columns cb .. cb + 3
//            and cb + 4 .. cb + 7 (cb = 0 or 8) of a block: lane 4 a + b
//            addresses column cb + a, rows 4 b .. 4 b + 3, so lane i receives
//            row i at 4 consecutive columns. Lanes 32-63 take the next block.
// val(i, j, v) gives the value of accumulator element (i, j, v). The 16
// row vectors of a lane go to rows(m, n, x) in batches of BATCH (default kStageBatch):
// x[q][0..7] = columns n[q] .. n[q] + 7 of row m[q] (n[q] a multiple of 8),
// so a functor that reads global memory can issue all of a batch's loads
// before its first store (store-only functors use smaller batches: fewer
// live registers).
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
constexpr int kStageBatch = 8;

template <int BATCH = kStageBatch, int TM = big::TM, int TN = big::TN, class Val, class Rows>
__device__ __forceinline__ void stage_rows_bf16(char* lds, int lane, int m0, int n0, Val&& val,
                                                Rows&& rows) {
  const int G = lane >> 4, c = lane & 15;
  char* wr = lds + (c * 16 + 4 * G) * 2;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      bf16x4_t w;
#pragma unroll
      for (int v = 0; v < 4; ++v) w[v] = static_cast<bf16>(val(i, j, v));
      *reinterpret_cast<bf16x4_t*>(wr + (i * TN + j) * 512) = w;
    }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's writes are in LDS
  __builtin_amdgcn_wave_barrier();
  typedef __attribute__((address_space(3))) i16x4_t* lp;
  const int L = lane & 15, a = L >> 2, b = L & 3;
  const int cb = 8 * ((lane >> 4) & 1);
  const int jo = lane >> 5;
  const char* rd = lds + jo * 512 + ((cb + a) * 16 + 4 * b) * 2;
  constexpr int kVecs = TM * TN / 2;  // row vectors per lane
  static_assert(kVecs % BATCH == 0, "whole batches");
#pragma unroll
  for (int q0 = 0; q0 < kVecs; q0 += BATCH) {
    int m[BATCH], n[BATCH];
    float x[BATCH][8];
#pragma unroll
    for (int q = 0; q < BATCH; ++q) {
      const int i = (q0 + q) / (TN / 2), jp = (q0 + q) % (TN / 2);
      const char* blk = rd + (i * TN + 2 * jp) * 512;
      const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lp)(blk));
      const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lp)(blk + 4 * 32));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[q][e] = __builtin_bit_cast(float, (uint32_t)(uint16_t)lo[e] << 16);
        x[q][4 + e] = __builtin_bit_cast(float, (uint32_t)(uint16_t)hi[e] << 16);
      }
      m[q] = m0 + 16 * i + L;
      n[q] = n0 + 16 * (2 * jp + jo) + cb;
    }
    rows(m, n, x);
  }
}

// Staged read-modify-write of a wave's 128 x 64 bf16 sub-tile:
//   C[m, n] = bf16(bf16(alpha acc) + beta C[m, n])
// in the layout of stage_rows_bf16. The lane's 16 old row vectors (8
// columns each) are loaded, kept packed, before the tile is staged, so one
// memory latency per tile is exposed instead of one per batch of rows.
__device__ __forceinline__ void stage_rmw_bf16(char* lds, int lane, int m0, int n0,
                                               const f32x4_t (&acc)[big::TM][big::TN], float alpha,
                                               float beta, bf16* C, int64_t ldc, int M, int N) {
  constexpr int TN = big::TN, kVecs = big::TM * big::TN / 2;
  typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
  const int G = lane >> 4, c = lane & 15;
  const int L = lane & 15, a = L >> 2, b = L & 3;
  const int cb = 8 * ((lane >> 4) & 1);
  const int jo = lane >> 5;
  u32x4_t old[kVecs];
#pragma unroll
  for (int q = 0; q < kVecs; ++q) {
    const int i = q / (TN / 2), jp = q % (TN / 2);
    const int m = m0 + 16 * i + L, n = n0 + 16 * (2 * jp + jo) + cb;
    old[q] = u32x4_t{0u, 0u, 0u, 0u};
    if (m < M && n + 8 <= N) old[q] = *reinterpret_cast<const u32x4_t*>(C + (int64_t)m * ldc + n);
  }
  char* wr = lds + (c * 16 + 4 * G) * 2;
#pragma unroll
  for (int i = 0; i < big::TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      bf16x4_t w;
#pragma unroll
      for (int v = 0; v < 4; ++v) w[v] = static_cast<bf16>(alpha * acc[i][j][v]);
      *reinterpret_cast<bf16x4_t*>(wr + (i * TN + j) * 512) = w;
    }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's writes are in LDS
  __builtin_amdgcn_wave_barrier();
  typedef __attribute__((address_space(3))) i16x4_t* lp;
  const char* rd = lds + jo * 512 + ((cb + a) * 16 + 4 * b) * 2;
#pragma unroll
  for (int q = 0; q < kVecs; ++q) {
    const int i = q / (TN / 2), jp = q % (TN / 2);
    const char* blk = rd + (i * TN + 2 * jp) * 512;
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lp)(blk));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lp)(blk + 4 * 32));
    const int m = m0 + 16 * i + L, n = n0 + 16 * (2 * jp + jo) + cb;
    if (m >= M || n >= N) continue;
    float x[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = __builtin_bit_cast(float, (uint32_t)(uint16_t)lo[e] << 16);
      x[4 + e] = __builtin_bit_cast(float, (uint32_t)(uint16_t)hi[e] << 16);
    }
    bf16* p = C + (int64_t)m * ldc + n;
    if (n + 8 <= N) {
      float y[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t w = old[q][k >> 1];
        const float o = __builtin_bit_cast(float, (k & 1) ? (w & 0xFFFF0000u) : (w << 16));
        y[k] = x[k] + beta * o;
      }
      store_n<bf16, 8>(p, y);
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (n + k < N) p[k] = from_f32<bf16>(x[k] + beta * to_f32(p[k]));
    }
  }
}

// Stores x[0..7] at p[0..7] as bf16 (one 16-byte store when all 8 columns are
// inside [.., N), element by element otherwise).
__device__ __forceinline__ void store_row8_bf16(bf16* p, int n, int N, const float (&x)[8]) {
  if (n + 8 <= N) {
    store_n<bf16, 8>(p, x);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (n + k < N) p[k] = from_f32<bf16>(x[k]);
  }
}

__device__ __forceinline__ void load_row8_bf16(const bf16* p, int n, int N, float (&x)[8]) {
  if (n + 8 <= N) {
    load_n<bf16, 8>(p, x);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = n + k < N ? to_f32(p[k]) : 0.f;
  }
}

// The GEMM kernel: mainloop + epilogue functor
//   epi(acc, m_base, n_base, lane, smem, split) with m_base / n_base the
//   origin of this wave's sub-tile and acc in the path's MFMA layout
//   (f32x4_t[8][4] for the 256 x 256 tile, f32x16_t[TM][TN] otherwise).
//   smem: LDS the epilogue may use - for the 256 x 256 tile, 16 KB private
//   to the wave (staged bf16 epilogues); otherwise the block's stage 0.
// An epilogue may declare skip_tile(tm): work items of row tiles it skips
// return before the main loop (a block-uniform test, no barrier reached).
template <class E, class = void>
struct HasSkipTile : std::false_type {};
template <class E>
struct HasSkipTile<E, std::void_t<decltype(std::declval<const E&>().skip_tile(0))>>
    : std::true_type {};

// An epilogue of the r4 engine may take a wave's whole 128 x 128 sub-tile in
// one call: full_tile(acc, m0, n0, lane, lds) with acc[h][i][j] the MFMA
// tile (i, 4 h + j) and lds the wave's 2 x 16 KB; otherwise it is called per
// 128 x 64 half.
template <class E, class = void>
struct HasFullTile : std::false_type {};
template <class E>
struct HasFullTile<E, std::void_t<decltype(std::declval<const E&>().full_tile(
                          std::declval<f32x4_t (&)[2][r4::TM][4]>(), 0, 0, 0,
                          static_cast<char*>(nullptr)))>> : std::true_type {};

template <class C, int LA, int LB, class Epi>
__global__ __launch_bounds__(C::THREADS) void gemm_kernel(const Problem pb, const Epi epi) {
  int tm, tn, split;
  if (!tile_coords(pb, blockIdx.x, tm, tn, split)) return;
  if constexpr (HasSkipTile<Epi>::value) {
    if (epi.skip_tile(tm)) return;
  }
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  if constexpr (C::BM == 256 && C::BN == 256 && C::ENGINE == 2) {
    __shared__ __attribute__((aligned(16))) char lds[r4::LDS_BYTES];
    f32x4_t acc[2][r4::TM][4];
    r4_mainloop<LA, LB>(pb, tm, tn, split, lds, acc);
    // each wave gets 2 x 16 KB of LDS of its own for the two 128 x 64 halves
    // of its sub-tile
    const int w = __builtin_amdgcn_readfirstlane(wave);
    char* wl = lds + w * 2 * r4::EPI_BYTES;
    const int em = tm * 256 + (w >> 1) * r4::WM, en = tn * 256 + (w & 1) * r4::WN;
    if constexpr (HasFullTile<Epi>::value) {
      epi.full_tile(acc, em, en, tid & 63, wl);
    } else {
      epi(acc[0], em, en, tid & 63, wl, split);
      epi(acc[1], em, en + 64, tid & 63, wl + r4::EPI_BYTES, split);
    }
  } else if constexpr (C::BM == 256 && C::BN == 256) {
    __shared__ __attribute__((aligned(16))) char lds[big::STAGES * big::STAGE_BYTES];
    f32x4_t acc[big::TM][big::TN];
    big_mainloop<LA, LB>(pb, tm, tn, split, lds, acc);
    // each wave gets 16 KB of LDS of its own for its epilogue
    char* wl = lds + __builtin_amdgcn_readfirstlane(wave) * big::EPI_BYTES;
    epi(acc, tm * 256 + (wave >> 2) * big::WM, tn * 256 + (wave & 3) * big::WN, tid & 63, wl,
        split);
  } else {
    __shared__ __attribute__((aligned(16))) char stage0[C::STAGE_BYTES];
    __shared__ __attribute__((aligned(16))) char stage1[C::STAGE_BYTES];
    f32x16_t acc[C::TM][C::TN];
    mainloop<C, LA, LB>(pb, tm, tn, split, stage0, stage1, acc);
    epi(acc, tm * C::BM + (wave / C::WAVES_N) * C::WM, tn * C::BN + (wave % C::WAVES_N) * C::WN,
        tid & 63, stage0, split);
  }
}

// Up to kMaxGroup independent r4 products in one launch: blocks
// [first[g], first[g + 1]) run product g. Products too small to fill the GPU
// on their own (the LoRA k and v projections: 128 tiles each, half of the
// CUs) share rounds of tiles instead of each taking a round of its own.
constexpr int kMaxGroup = 3;

template <class Epi>
struct GemmGroup {
  Problem pb[kMaxGroup];
  Epi epi[kMaxGroup];
  int first[kMaxGroup + 1];
  int count;
};

template <int LA, int LB, class Epi>
__global__ __launch_bounds__(R4Cfg::THREADS) void gemm_group_kernel(const GemmGroup<Epi> g) {
  const int bid = blockIdx.x;
  const int p = (g.count > 2 && bid >= g.first[2]) ? 2 : (g.count > 1 && bid >= g.first[1]) ? 1 : 0;
  const Problem& pb = p == 0 ? g.pb[0] : p == 1 ? g.pb[1] : g.pb[2];
  const Epi& epi = p == 0 ? g.epi[0] : p == 1 ? g.epi[1] : g.epi[2];
  int tm, tn, split;
  if (!tile_coords(pb, bid - g.first[p], tm, tn, split)) return;
  const int tid = threadIdx.x;
  __shared__ __attribute__((aligned(16))) char lds[r4::LDS_BYTES];
  f32x4_t acc[2][r4::TM][4];
  r4_mainloop<LA, LB>(pb, tm, tn, split, lds, acc);
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  char* wl = lds + w * 2 * r4::EPI_BYTES;
  const int em = tm * 256 + (w >> 1) * r4::WM, en = tn * 256 + (w & 1) * r4::WN;
  epi(acc[0], em, en, tid & 63, wl, split);
  epi(acc[1], em, en + 64, tid & 63, wl + r4::EPI_BYTES, split);
}

// --------------------------------------------------------------- epilogues --

// C = alpha * acc + beta * C (C of type TC, row-major with ldc). With beta,
// the old values of a whole MFMA-tile row (i) are loaded before any is
// written, so the loads overlap instead of each waiting for the last.
template <typename TC>
struct EpiStore {
  TC* C;
  int64_t ldc;
  int M, N;
  float alpha, beta;

  // 256 x 256 tile, bf16 C: staged through LDS, 16-byte accesses (with beta,
  // alpha * acc is rounded to bf16 before beta * C is added).
  __device__ __forceinline__ void operator()(f32x4_t (&acc)[big::TM][big::TN], int m0, int n0,
                                             int lane, char* lds, int) const {
    if constexpr (std::is_same_v<TC, bf16>) {
      if (beta != 0.f) {
        stage_rmw_bf16(lds, lane, m0, n0, acc, alpha, beta, C, ldc, M, N);
        return;
      }
      stage_rows_bf16(
          lds, lane, m0, n0, [&](int i, int j, int v) { return alpha * acc[i][j][v]; },
          [&](const int (&m)[kStageBatch], const int (&n)[kStageBatch],
              const float (&x)[kStageBatch][8]) {
            float o[kStageBatch][8];
            if (beta != 0.f) {
#pragma unroll
              for (int q = 0; q < kStageBatch; ++q) {
                if (m[q] < M && n[q] < N)
                  load_row8_bf16(C + (int64_t)m[q] * ldc + n[q], n[q], N, o[q]);
              }
            }
#pragma unroll
            for (int q = 0; q < kStageBatch; ++q) {
              if (m[q] >= M || n[q] >= N) continue;
              float y[8];
#pragma unroll
              for (int k = 0; k < 8; ++k) y[k] = beta != 0.f ? x[q][k] + beta * o[q][k] : x[q][k];
              store_row8_bf16(C + (int64_t)m[q] * ldc + n[q], n[q], N, y);
            }
          });
    } else {
      generic(acc, m0, n0, lane);
    }
  }

  template <int TM, int TN>
  __device__ __forceinline__ void operator()(f32x16_t (&acc)[TM][TN], int m0, int n0, int lane,
                                             char*, int) const {
    generic(acc, m0, n0, lane);
  }

  template <typename AccT, int TM, int TN>
  __device__ __forceinline__ void generic(AccT (&acc)[TM][TN], int m0, int n0, int lane) const {
    if (beta == 0.f) {
      for_each_acc(acc, m0, n0, lane, [&](int m, int n, float v) {
        if (m < M && n < N) C[(int64_t)m * ldc + n] = from_f32<TC>(alpha * v);
      });
      return;
    }
    constexpr int V = sizeof(AccT) / sizeof(float);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float old[TN * V];
      int k = 0;
      for_each_acc_row(acc, i, m0, n0, lane, [&](int m, int n, float) {
        old[k++] = (m < M && n < N) ? to_f32(C[(int64_t)m * ldc + n]) : 0.f;
      });
      k = 0;
      for_each_acc_row(acc, i, m0, n0, lane, [&](int m, int n, float v) {
        const float o = old[k++];
        if (m < M && n < N) C[(int64_t)m * ldc + n] = from_f32<TC>(alpha * v + beta * o);
      });
    }
  }
};

// fp32 partial tile of split s at P[s][m][n] (dense M x N per split).
struct EpiPartial {
  float* P;
  int M, N;

  template <typename AccT, int TM, int TN>
  __device__ __forceinline__ void operator()(AccT (&acc)[TM][TN], int m0, int n0, int lane, char*,
                                             int split) const {
    float* base = P + (int64_t)split * M * N;
    for_each_acc(acc, m0, n0, lane, [&](int m, int n, float v) {
      if (m < M && n < N) base[(int64_t)m * N + n] = v;
    });
  }
};

// out[m, n] = alpha * row_scale[m] * sum_s P[s][m][n] + beta * out[m, n]
// (fixed order; row_scale null: 1). Four consecutive elements per thread when
// N % 4 == 0 (16-byte partial loads, the splits unrolled so several loads are
// in flight), one otherwise.
template <typename TC>
__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* __restrict__ P,
                                                              int ksplit, int M, int N,
                                                              TC* __restrict__ out, int64_t ldo,
                                                              float alpha, float beta,
                                                              const float* __restrict__ row_scale = nullptr) {
  const int64_t total = (int64_t)M * N;
  if (N % 4 == 0) {
    const int64_t nv = total / 4;
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < nv;
         q += (int64_t)gridDim.x * 256) {
      const int64_t e = q * 4;
      float s[4] = {0.f, 0.f, 0.f, 0.f};
      int k = 0;
      for (; k + 4 <= ksplit; k += 4) {
        float v[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) load_n<float, 4>(P + (int64_t)(k + u) * total + e, v[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int c = 0; c < 4; ++c) s[c] += v[u][c];
      }
      for (; k < ksplit; ++k) {
        float v[4];
        load_n<float, 4>(P + (int64_t)k * total + e, v);
#pragma unroll
        for (int c = 0; c < 4; ++c) s[c] += v[c];
      }
      const int64_t m = e / N, n = e - m * N;
      TC* p = out + m * ldo + n;
      const float a = row_scale ? alpha * row_scale[m] : alpha;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float r = a * s[c];
        if (beta != 0.f) r += beta * to_f32(p[c]);
        p[c] = from_f32<TC>(r);
      }
    }
    return;
  }
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * 256) {
    float s = 0.f;
    for (int k = 0; k < ksplit; ++k) s += P[(int64_t)k * total + e];
    const int64_t m = e / N, n = e - m * N;
    TC* p = out + m * ldo + n;
    float r = (row_scale ? alpha * row_scale[m] : alpha) * s;
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

// 256 x 256 launch with the store epilogue (engine of CF: BigCfg or R4Cfg).
template <typename TC, class CF = BigCfg>
inline int launch_store(const Problem& pb, int la, int lb, void* C, int64_t ldc, float alpha,
                        float beta, hipStream_t st) {
  EpiStore<TC> epi{static_cast<TC*>(C), ldc, pb.M, pb.N, alpha, beta};
  const dim3 grid(grid_blocks(pb));
#define ML_G(LA, LB) \
  gemm_kernel<CF, LA, LB, EpiStore<TC>><<<grid, CF::THREADS, 0, st>>>(pb, epi)
  if (la == kKMajor) {
    if (lb == kKMajor) ML_G(kKMajor, kKMajor);
    else ML_G(kKMajor, kMNMajor);
  } else if constexpr (CF::ENGINE == 2) {
    // r4 is used where A is K-major (its MN-major A path is not instantiated)
    set_error("gemm: the r4 engine takes a K-major A");
    return ML_ERR_INVALID;
  } else {
    if (lb == kKMajor) ML_G(kMNMajor, kKMajor);
    else ML_G(kMNMajor, kMNMajor);
  }
#undef ML_G
  ML_LAUNCH_CHECK();
  return ML_OK;
}

// count (1..kMaxGroup) products on the r4 engine in one launch, each with the
// store epilogue into its own C (A K-major).
template <typename TC>
inline int launch_store_group(const Problem* pbs, int count, int lb, void* const* C,
                              const int64_t* ldc, float alpha, float beta, hipStream_t st) {
  ML_CHECK(count >= 1 && count <= kMaxGroup, "gemm: 1..%d grouped products (got %d)", kMaxGroup,
           count);
  GemmGroup<EpiStore<TC>> g{};
  g.count = count;
  int blocks = 0;
  for (int i = 0; i < count; ++i) {
    g.pb[i] = pbs[i];
    g.epi[i] = EpiStore<TC>{static_cast<TC*>(C[i]), ldc[i], pbs[i].M, pbs[i].N, alpha, beta};
    g.first[i] = blocks;
    blocks += grid_blocks(pbs[i]);  // a multiple of 8: every product keeps its XCD order
  }
  for (int i = count; i <= kMaxGroup; ++i) g.first[i] = blocks;
  if (lb == kKMajor)
    gemm_group_kernel<kKMajor, kKMajor, EpiStore<TC>><<<dim3(blocks), R4Cfg::THREADS, 0, st>>>(g);
  else
    gemm_group_kernel<kKMajor, kMNMajor, EpiStore<TC>><<<dim3(blocks), R4Cfg::THREADS, 0, st>>>(g);
  ML_LAUNCH_CHECK();
  return ML_OK;
}

// Split-K product of shape C into fp32 partials ws (ksplit * M * N floats),
// then out = alpha * sum + beta * out.
template <class C, int LA, int LB, typename TC>
inline int launch_splitk(const Problem& pb, float* ws, TC* out, int64_t ldo, float alpha, float beta,
                         hipStream_t st, const float* row_scale = nullptr) {
  EpiPartial epi{ws, pb.M, pb.N};
  gemm_kernel<C, LA, LB, EpiPartial><<<dim3(grid_blocks(pb)), C::THREADS, 0, st>>>(pb, epi);
  ML_LAUNCH_CHECK();
  const int64_t total = (int64_t)pb.M * pb.N;
  const int64_t per_thread = pb.N % 4 == 0 ? 4 : 1;
  int64_t blocks = (total / per_thread + 255) / 256;
  blocks = blocks < 2048 ? (blocks > 0 ? blocks : 1) : 2048;
  reduce_partials_kernel<TC><<<dim3((unsigned)blocks), 256, 0, st>>>(ws, pb.ksplit, pb.M, pb.N,
                                                                     out, ldo, alpha, beta,
                                                                     row_scale);
  ML_LAUNCH_CHECK();
  return ML_OK;
}

inline size_t splitk_ws_bytes(const Problem& pb) {
  return (size_t)pb.ksplit * (size_t)pb.M * (size_t)pb.N * sizeof(float);
}

}  // namespace gemm
}  // namespace mla

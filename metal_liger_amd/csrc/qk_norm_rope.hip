// Qwen3 attention's head-dim RMSNorm (q_norm / k_norm) fused with rotate-half
// RoPE from cos/sin tables, forward and backward, q and k in one launch.
//
// The reference's patcher leaves these norms on transformers' Qwen3RMSNorm
// (patch.py:104-131 replaces only the layer norms): five fp32 passes over q
// and k, then the rotary step's own passes. The semantics followed are
// transformers' models/qwen3/modeling_qwen3.py: Qwen3RMSNorm.forward, then
// apply_rotary_pos_emb with rotate_half.
//
// A work item is one token and a group of consecutive heads of one tensor
// (kHeadsPerItemFwd / Bwd). G = (D/2) / V threads own an item (V elements per 16-byte
// access): thread g holds elements [V g, V g + V) of the first half of each
// head and the same V of the second half, so each rotate-half pair (j, j +
// D/2) sits in one thread and the rotation needs no lane exchange. A row's
// sum of squares (and, in the backward, the dot product of the rescaled
// gradient with the normalised row) is a reduction over the G lanes. The
// item's index arithmetic and its cos/sin loads are shared by its heads, and
// all of the heads' loads are issued before any arithmetic. The items of a
// launch are q's, then k's; a block owns a contiguous range of one tensor's
// items, so that tensor's pointers and strides are uniform across the block.
//
// Backward, exact for any tables (not only duplicated-half ones):
//   dn[j]     = dy[j] c[j] + dy[j+h] s[j+h]
//   dn[j+h]   = dy[j+h] c[j+h] - dy[j] s[j]            (h = D/2, j < h)
//   g = dn w,  n^ = x r,  r = rsqrt(mean(x^2) + eps)
//   dx = r (g - n^ mean(g n^)),   dw = sum over rows of dn n^
// dw is summed per block in a fixed order into one partial row; a second
// launch sums the partial rows in a fixed order (deterministic).
#include <algorithm>
#include <initializer_list>

#include "common.h"

namespace mla {
namespace {

constexpr int kQknThreads = 256;
// Heads per work item, forward and backward (MI355X, q [4, 16, 2048, 128] +
// k [4, 8, 2048, 128] bf16: 1 and 2 are within 2% of the best of 1, 2, 4;
// 4 in the backward is 10% slower).
constexpr int kHeadsPerItemFwd = 1;
constexpr int kHeadsPerItemBwd = 2;
constexpr int64_t kQknTargetBlocks = 2048;
constexpr int kDwThreads = 256;
constexpr int kDwCols = 16;   // columns per reduction block
constexpr int kDwUnroll = 8;

struct QknTensor {
  const void* x;   // pre-norm rows
  const void* dy;  // backward: gradient of the rotated rows
  void* out;       // forward: rotated rows; backward: dx
  const void* w;   // norm weight [D]
  float* part;     // backward: one dw partial row per block, or null
  int64_t H, groups, items, blocks;  // groups = ceil(H / heads per item)
  int64_t xb, xh, xs;  // strides (elements) of x
  int64_t db, dh, ds;  // of dy
  int64_t ob, oh, os;  // of out
};

struct QknArgs {
  QknTensor t[2];
  int64_t S, items_per_block;
  float eps, inv_d;
  const void* cos;
  const void* sin;
  int64_t cb, ch, cs, sb, sh, ss;
};

// Sum over the G lanes of an aligned lane group.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <typename T, int N>
__device__ __forceinline__ void cvt(const Pack<T, N>& p, float (&o)[N]) {
#pragma unroll
  for (int e = 0; e < N; ++e) o[e] = to_f32(p.v[e]);
}

template <typename T, int N>
__device__ __forceinline__ Pack<T, N> ldp(const T* p) {
  return *reinterpret_cast<const Pack<T, N>*>(p);
}

// Threads per item for D and an element type: (D / 2) / (16 / sizeof(T)).
constexpr int qkn_group(int D, int elem_bytes) { return (D / 2) / (16 / elem_bytes); }

template <typename TX, typename TW, int D, bool BWD>
__global__ __launch_bounds__(kQknThreads) void qkn_rope_kernel(const QknArgs a) {
  constexpr int V = 16 / (int)sizeof(TX);   // elements per 16-byte access
  constexpr int HALF = D / 2;
  constexpr int G = qkn_group(D, (int)sizeof(TX));
  constexpr int IPP = kQknThreads / G;      // items per block per pass
  constexpr int HPI = BWD ? kHeadsPerItemBwd : kHeadsPerItemFwd;
  static_assert(HALF % V == 0 && G >= 1 && G <= 64, "head dim / vector width");
  const int op = (int64_t)blockIdx.x < a.t[0].blocks ? 0 : 1;
  const QknTensor& t = a.t[op];
  const int64_t blk = (int64_t)blockIdx.x - (op ? a.t[0].blocks : 0);
  const int g = threadIdx.x % G;
  const int il = threadIdx.x / G;
  const int j = V * g;

  float w_lo[V], w_hi[V];
  load_n<TW, V>(static_cast<const TW*>(t.w) + j, w_lo);
  load_n<TW, V>(static_cast<const TW*>(t.w) + HALF + j, w_hi);
  float dw_lo[BWD ? V : 1], dw_hi[BWD ? V : 1];
  if constexpr (BWD) {
#pragma unroll
    for (int e = 0; e < V; ++e) dw_lo[e] = dw_hi[e] = 0.f;
  }

  const int64_t i_begin = blk * a.items_per_block;
  const int64_t i_end = std::min(i_begin + a.items_per_block, t.items);
  const uint32_t NG = (uint32_t)t.groups, S = (uint32_t)a.S;
  const int H = (int)t.H;
  const bool table_per_head = (a.ch | a.sh) != 0;
  const TX* xbase = static_cast<const TX*>(t.x);
  const TX* dbase = static_cast<const TX*>(t.dy);
  const TX* cbase = static_cast<const TX*>(a.cos);
  const TX* sbase = static_cast<const TX*>(a.sin);
  TX* obase = static_cast<TX*>(t.out);

  for (int64_t base = i_begin; base < i_end; base += IPP) {
    const int64_t item = base + il;
    const bool live = item < i_end;
    // Items past the end re-load the block's last item (no branch around
    // the loads); their results are neither stored nor added to dw.
    const uint32_t ii = (uint32_t)(live ? item : i_end - 1);
    const uint32_t tok = ii / NG, grp = ii - tok * NG;
    const uint32_t b = tok / S, s = tok - b * S;
    const int h0 = (int)grp * HPI;
    const int64_t xo = (int64_t)b * t.xb + (int64_t)s * t.xs + j;
    const int64_t dox = BWD ? (int64_t)b * t.db + (int64_t)s * t.ds + j : 0;
    const int64_t oo = (int64_t)b * t.ob + (int64_t)s * t.os + j;
    const int64_t co = (int64_t)b * a.cb + (int64_t)s * a.cs + j;
    const int64_t so = (int64_t)b * a.sb + (int64_t)s * a.ss + j;

    // Heads past H re-load the last head; they are not stored.
    Pack<TX, V> xl[HPI], xh[HPI];
    Pack<TX, V> dl[BWD ? HPI : 1], dh[BWD ? HPI : 1];
#pragma unroll
    for (int u = 0; u < HPI; ++u) {
      const int64_t hh = std::min(h0 + u, H - 1);
      const TX* xp = xbase + (xo + hh * t.xh);
      xl[u] = load_pack_nt<TX, V>(xp);
      xh[u] = load_pack_nt<TX, V>(xp + HALF);
      if constexpr (BWD) {
        const TX* dp = dbase + (dox + hh * t.dh);
        dl[u] = load_pack_nt<TX, V>(dp);
        dh[u] = load_pack_nt<TX, V>(dp + HALF);
      }
    }
    float c_lo[V], c_hi[V], s_lo[V], s_hi[V];
    auto load_tables = [&](int64_t hh) {
      const TX* cp = cbase + (co + hh * a.ch);
      const TX* sp = sbase + (so + hh * a.sh);
      cvt(ldp<TX, V>(cp), c_lo);
      cvt(ldp<TX, V>(cp + HALF), c_hi);
      cvt(ldp<TX, V>(sp), s_lo);
      cvt(ldp<TX, V>(sp + HALF), s_hi);
    };
    if (!table_per_head) load_tables(0);

#pragma unroll
    for (int u = 0; u < HPI; ++u) {
      const int hh = std::min(h0 + u, H - 1);
      const bool store = live && h0 + u < H;
      if (table_per_head) load_tables(hh);
      float x_lo[V], x_hi[V];
      cvt(xl[u], x_lo);
      cvt(xh[u], x_hi);
      float ssq = 0.f;
#pragma unroll
      for (int e = 0; e < V; ++e) ssq += x_lo[e] * x_lo[e] + x_hi[e] * x_hi[e];
      ssq = group_sum<G>(ssq);
      const float r = rsqrtf(ssq * a.inv_d + a.eps);
      float o_lo[V], o_hi[V];
      if constexpr (!BWD) {
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float nl = x_lo[e] * r * w_lo[e];
          const float nh = x_hi[e] * r * w_hi[e];
          // n * cos + rotate_half(n) * sin, rotate_half([n1, n2]) = [-n2, n1]
          o_lo[e] = nl * c_lo[e] - nh * s_lo[e];
          o_hi[e] = nh * c_hi[e] + nl * s_hi[e];
        }
      } else {
        float d_lo[V], d_hi[V];
        cvt(dl[u], d_lo);
        cvt(dh[u], d_hi);
        float gl[V], gh[V];
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float dnl = d_lo[e] * c_lo[e] + d_hi[e] * s_hi[e];
          const float dnh = d_hi[e] * c_hi[e] - d_lo[e] * s_lo[e];
          x_lo[e] *= r;  // n^
          x_hi[e] *= r;
          gl[e] = dnl * w_lo[e];
          gh[e] = dnh * w_hi[e];
          dot += gl[e] * x_lo[e] + gh[e] * x_hi[e];
          if (store) {
            dw_lo[e] += dnl * x_lo[e];
            dw_hi[e] += dnh * x_hi[e];
          }
        }
        const float m = group_sum<G>(dot) * a.inv_d;
#pragma unroll
        for (int e = 0; e < V; ++e) {
          o_lo[e] = r * (gl[e] - x_lo[e] * m);
          o_hi[e] = r * (gh[e] - x_hi[e] * m);
        }
      }
      if (store) {
        TX* yp = obase + (oo + (int64_t)hh * t.oh);
        store_n_nt<TX, V>(yp, o_lo);
        store_n_nt<TX, V>(yp + HALF, o_hi);
      }
    }
  }

  if constexpr (BWD) {
    if (t.part == nullptr) return;  // uniform across the block
    __shared__ float red[IPP][D];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      red[il][j + e] = dw_lo[e];
      red[il][HALF + j + e] = dw_hi[e];
    }
    __syncthreads();
    for (int c = threadIdx.x; c < D; c += kQknThreads) {
      float acc = 0.f;
      for (int q = 0; q < IPP; ++q) acc += red[q][c];
      t.part[blk * D + c] = acc;
    }
  }
}

struct DwReduceArgs {
  const float* part[2];
  int64_t G[2];
  void* dw[2];
};

// dw[c] = sum over the G partial rows, in a fixed order. A block owns
// kDwCols columns of one tensor: each thread sums a strided subset of the
// rows for 4 columns (kDwUnroll loads in flight), then a fixed tree over the
// subsets.
template <typename TW, int D>
__global__ __launch_bounds__(kDwThreads) void qkn_dw_reduce(const DwReduceArgs a) {
  constexpr int CV = kDwCols / 4;          // column vectors per block
  constexpr int NSL = kDwThreads / CV;     // row subsets
  const int op = blockIdx.y;
  if (a.dw[op] == nullptr) return;  // uniform across the block
  const int c4 = threadIdx.x % CV, sl = threadIdx.x / CV;
  const int col = blockIdx.x * kDwCols + 4 * c4;
  const float* part = a.part[op];
  const int64_t G = a.G[op];
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t g0 = sl; g0 < G; g0 += (int64_t)NSL * kDwUnroll) {
    float v[kDwUnroll][4];
#pragma unroll
    for (int u = 0; u < kDwUnroll; ++u) {
      const int64_t g = g0 + (int64_t)u * NSL;
      if (g < G) {
        load_n<float, 4>(part + g * D + col, v[u]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[u][e] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kDwUnroll; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) s[e] += v[u][e];
  }
  __shared__ float sm[NSL][kDwCols];
#pragma unroll
  for (int e = 0; e < 4; ++e) sm[sl][4 * c4 + e] = s[e];
  __syncthreads();
#pragma unroll
  for (int half = NSL / 2; half >= 1; half >>= 1) {
    if (sl < half) {
#pragma unroll
      for (int e = 0; e < 4; ++e) sm[sl][4 * c4 + e] += sm[sl + half][4 * c4 + e];
    }
    __syncthreads();
  }
  if (sl == 0) {
    TW* dw = static_cast<TW*>(a.dw[op]);
#pragma unroll
    for (int e = 0; e < 4; ++e) dw[col + e] = from_f32<TW>(sm[0][4 * c4 + e]);
  }
}

struct QknPlan {
  int64_t items_per_block;
  int64_t blocks[2];
};

// Items per block: a multiple of one pass of 2-byte elements (the plan, and
// so the workspace size, does not depend on the dtype), about
// kQknTargetBlocks blocks in all.
QknPlan make_plan(int64_t items_q, int64_t items_k, int64_t D) {
  const int64_t step = kQknThreads / qkn_group((int)D, 2);
  const int64_t total = items_q + items_k;
  int64_t ipb = (total + kQknTargetBlocks - 1) / kQknTargetBlocks;
  ipb = std::max(step, (ipb + step - 1) / step * step);
  QknPlan p;
  p.items_per_block = ipb;
  p.blocks[0] = (items_q + ipb - 1) / ipb;
  p.blocks[1] = (items_k + ipb - 1) / ipb;
  return p;
}

int64_t head_groups(int64_t H, bool bwd) {
  const int64_t hpi = bwd ? kHeadsPerItemBwd : kHeadsPerItemFwd;
  return (H + hpi - 1) / hpi;
}

bool supported_d(int64_t D) { return D == 32 || D == 64 || D == 128 || D == 256; }

// Fills the parts of a tensor shared by the forward and backward geometry
// forms; returns false when B / S differ from the first tensor's.
bool fill_dims(QknTensor& t, const int64_t* g, int64_t& B, int64_t& S, bool first) {
  t.H = g[1];
  if (first) {
    B = g[0];
    S = g[2];
    return true;
  }
  return g[0] == B && g[2] == S;
}

// Every access is 16 bytes (or, for fp32 weights, two of them): base
// pointers 16-byte aligned and strides in multiples of 16 bytes.
template <typename T>
bool aligned_operand(const void* p, std::initializer_list<int64_t> strides) {
  if (reinterpret_cast<uintptr_t>(p) % 16) return false;
  for (int64_t s : strides)
    if (s < 0 || (s * (int64_t)sizeof(T)) % 16) return false;
  return true;
}

template <typename TX, typename TW, bool BWD>
int launch_qkn(QknArgs& a, int64_t B, int64_t D, const DwReduceArgs* red, hipStream_t st) {
  for (int i = 0; i < 2; ++i) {
    QknTensor& t = a.t[i];
    if (t.items == 0) continue;
    ML_CHECK(aligned_operand<TX>(t.x, {t.xb, t.xh, t.xs}) &&
                 aligned_operand<TX>(t.out, {t.ob, t.oh, t.os}) &&
                 (!BWD || aligned_operand<TX>(t.dy, {t.db, t.dh, t.ds})) &&
                 aligned_operand<TW>(t.w, {}),
             "qk_norm_rope: tensors must be 16-byte aligned with strides in multiples of 16 bytes");
  }
  if (a.t[0].items + a.t[1].items > 0)
    ML_CHECK(aligned_operand<TX>(a.cos, {a.cb, a.ch, a.cs}) &&
                 aligned_operand<TX>(a.sin, {a.sb, a.sh, a.ss}),
             "qk_norm_rope: cos/sin must be 16-byte aligned with strides in multiples of 16 bytes");
  const int64_t blocks = a.t[0].blocks + a.t[1].blocks;
  ML_CHECK(blocks <= 0x7fffffffLL, "qk_norm_rope: problem too large");
  if (blocks > 0) {
#define ML_QKN(DD) qkn_rope_kernel<TX, TW, DD, BWD><<<dim3((unsigned)blocks), kQknThreads, 0, st>>>(a)
    if (D == 32) ML_QKN(32); else if (D == 64) ML_QKN(64); else if (D == 128) ML_QKN(128); else ML_QKN(256);
#undef ML_QKN
    ML_LAUNCH_CHECK();
  }
  // The reduction also runs for a tensor without rows: its dw is zero.
  if (BWD && red != nullptr && (red->dw[0] != nullptr || red->dw[1] != nullptr)) {
#define ML_RED(DD) qkn_dw_reduce<TW, DD><<<dim3((DD) / kDwCols, 2), kDwThreads, 0, st>>>(*red)
    if (D == 32) ML_RED(32); else if (D == 64) ML_RED(64); else if (D == 128) ML_RED(128); else ML_RED(256);
#undef ML_RED
    ML_LAUNCH_CHECK();
  }
  (void)B;
  return ML_OK;
}

// Calls f(TX{}, TW{}) for x dtype x_dtype and weight dtype w_dtype (the same
// as x, or fp32).
template <typename F>
int dispatch_qkn(int x_dtype, int w_dtype, F&& f) {
  return dispatch_dtype(x_dtype, [&](auto tx) -> int {
    if (w_dtype == ML_F32) return f(tx, float{});
    ML_CHECK(w_dtype == x_dtype, "qk_norm_rope: weight dtype %d must be fp32 or x's dtype %d",
             w_dtype, x_dtype);
    return f(tx, tx);
  });
}

// k is given when its pointer is, or when its geometry describes no
// elements (an empty tensor's pointer may be null); NULL k with no geometry
// or a non-empty one means q only.
bool k_given(const void* k, const int64_t* k_geom) {
  return k != nullptr || (k_geom != nullptr && k_geom[0] * k_geom[1] * k_geom[2] == 0);
}

int setup_qkn(QknArgs& a, int64_t& B, const int64_t* q_geom, const int64_t* k_geom, bool has_k,
              int64_t D, float eps, const void* cos, const void* sin, const int64_t* cs_geom,
              bool bwd) {
  ML_CHECK(q_geom != nullptr, "qk_norm_rope: null q geometry");
  ML_CHECK(supported_d(D), "qk_norm_rope: head dim must be 32, 64, 128 or 256 (got %lld)",
           (long long)D);
  a = QknArgs{};
  int64_t S = 0;
  fill_dims(a.t[0], q_geom, B, S, true);
  if (has_k) {
    ML_CHECK(k_geom != nullptr, "qk_norm_rope: null k geometry");
    ML_CHECK(fill_dims(a.t[1], k_geom, B, S, false),
             "qk_norm_rope: q and k must share batch and sequence sizes");
  }
  ML_CHECK(B >= 0 && S >= 0 && a.t[0].H >= 0 && a.t[1].H >= 0, "qk_norm_rope: negative size");
  for (int i = 0; i < 2; ++i) {
    a.t[i].groups = head_groups(a.t[i].H, bwd);
    a.t[i].items = B * S * a.t[i].groups;
    ML_CHECK(a.t[i].items < ((int64_t)1 << 31) && a.t[i].H < ((int64_t)1 << 30),
             "qk_norm_rope: problem too large");
  }
  const QknPlan p = make_plan(a.t[0].items, a.t[1].items, D);
  a.items_per_block = p.items_per_block;
  a.t[0].blocks = p.blocks[0];
  a.t[1].blocks = p.blocks[1];
  a.S = S;
  a.eps = eps;
  a.inv_d = 1.f / (float)D;
  ML_CHECK(cs_geom != nullptr && (a.t[0].items + a.t[1].items == 0 || (cos && sin)),
           "qk_norm_rope: null cos/sin");
  a.cos = cos;
  a.sin = sin;
  a.cb = cs_geom[0];
  a.ch = cs_geom[1];
  a.cs = cs_geom[2];
  a.sb = cs_geom[3];
  a.sh = cs_geom[4];
  a.ss = cs_geom[5];
  return ML_OK;
}

}  // namespace
}  // namespace mla

using namespace mla;

extern "C" int ml_qk_norm_rope_fwd(const void* q, void* q_out, const int64_t* q_geom,
                                   const void* q_weight, const void* k, void* k_out,
                                   const int64_t* k_geom, const void* k_weight, int64_t D,
                                   float eps, const void* cos, const void* sin,
                                   const int64_t* cs_geom, int x_dtype, int w_dtype,
                                   void* stream) {
  QknArgs a;
  int64_t B = 0;
  int rc = setup_qkn(a, B, q_geom, k_geom, k_given(k, k_geom), D, eps, cos, sin, cs_geom, false);
  if (rc) return rc;
  const void* xs[2] = {q, k};
  void* outs[2] = {q_out, k_out};
  const void* ws[2] = {q_weight, k_weight};
  const int64_t* geoms[2] = {q_geom, k_geom};
  for (int i = 0; i < 2; ++i) {
    QknTensor& t = a.t[i];
    if (t.items == 0) continue;
    ML_CHECK(xs[i] && outs[i] && ws[i], "qk_norm_rope: null %s tensor", i ? "k" : "q");
    const int64_t* g = geoms[i];
    t.x = xs[i];
    t.out = outs[i];
    t.w = ws[i];
    t.xb = g[3];
    t.xh = g[4];
    t.xs = g[5];
    t.ob = g[6];
    t.oh = g[7];
    t.os = g[8];
  }
  hipStream_t st = (hipStream_t)stream;
  return dispatch_qkn(x_dtype, w_dtype, [&](auto tx, auto tw) -> int {
    return launch_qkn<decltype(tx), decltype(tw), false>(a, B, D, nullptr, st);
  });
}

extern "C" size_t ml_qk_norm_rope_bwd_workspace_bytes(int64_t B, int64_t S, int64_t Hq,
                                                      int64_t Hk, int64_t D) {
  if (!supported_d(D) || B < 0 || S < 0 || Hq < 0 || Hk < 0) return 0;
  const QknPlan p = make_plan(B * S * head_groups(Hq, true), B * S * head_groups(Hk, true), D);
  return (size_t)((p.blocks[0] + p.blocks[1]) * D) * sizeof(float);
}

extern "C" int ml_qk_norm_rope_bwd(const void* q, const void* dq_out, void* dq,
                                   const int64_t* q_geom, const void* q_weight, void* dq_weight,
                                   const void* k, const void* dk_out, void* dk,
                                   const int64_t* k_geom, const void* k_weight, void* dk_weight,
                                   int64_t D, float eps, const void* cos, const void* sin,
                                   const int64_t* cs_geom, int x_dtype, int w_dtype,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  QknArgs a;
  int64_t B = 0;
  int rc = setup_qkn(a, B, q_geom, k_geom, k_given(k, k_geom), D, eps, cos, sin, cs_geom, true);
  if (rc) return rc;
  const void* xs[2] = {q, k};
  const void* dys[2] = {dq_out, dk_out};
  void* outs[2] = {dq, dk};
  const void* ws[2] = {q_weight, k_weight};
  void* dws[2] = {dq_weight, dk_weight};
  const int64_t* geoms[2] = {q_geom, k_geom};
  const bool want_dw = (dq_weight != nullptr && a.t[0].items > 0) ||
                       (dk_weight != nullptr && a.t[1].items > 0);
  const size_t need = ml_qk_norm_rope_bwd_workspace_bytes(B, a.S, a.t[0].H, a.t[1].H, D);
  ML_CHECK(!want_dw || (workspace != nullptr && workspace_bytes >= need),
           "qk_norm_rope: workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
           need);
  DwReduceArgs red{};
  float* part = static_cast<float*>(workspace);
  for (int i = 0; i < 2; ++i) {
    QknTensor& t = a.t[i];
    if (dws[i] != nullptr && (i == 0 || k_given(k, k_geom))) {
      // part stays null for a tensor without rows (its reduction reads none)
      t.part = t.items > 0 ? part + (i ? a.t[0].blocks * D : 0) : nullptr;
      red.part[i] = t.part;
      red.G[i] = t.blocks;
      red.dw[i] = dws[i];
    }
    if (t.items == 0) continue;
    ML_CHECK(xs[i] && dys[i] && outs[i] && ws[i], "qk_norm_rope: null %s tensor", i ? "k" : "q");
    const int64_t* g = geoms[i];
    t.x = xs[i];
    t.dy = dys[i];
    t.out = outs[i];
    t.w = ws[i];
    t.xb = g[3];
    t.xh = g[4];
    t.xs = g[5];
    t.db = g[6];
    t.dh = g[7];
    t.ds = g[8];
    t.ob = g[9];
    t.oh = g[10];
    t.os = g[11];
  }
  hipStream_t st = (hipStream_t)stream;
  return dispatch_qkn(x_dtype, w_dtype, [&](auto tx, auto tw) -> int {
    return launch_qkn<decltype(tx), decltype(tw), true>(a, B, D, &red, st);
  });
}

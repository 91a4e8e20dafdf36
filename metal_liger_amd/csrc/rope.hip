// Rotate-half rotary embedding for gfx950 (ops/fused_rope.py:22-75, :110-127).
//
// One launch rotates q and k together. A thread owns one (b, s) position and
// VEC consecutive pairs (j, j + D/2) of the head dimension, gets the VEC
// cos/sin values once (from the tables, or computed in-kernel from the
// position and inv_freq), then rotates up to kHeadsPerThread heads of the
// concatenated [q heads | k heads] list with them, issuing all of those
// heads' loads before any arithmetic (measured on MI355X: hoisted loads move
// the q+k config at 5.4-5.6 TB/s, against 3.8 TB/s for heads loaded one at a
// time; 4 heads per thread is slightly ahead of 2, 3 and 8). Eight threads cover a
// 128-wide head; a wave covers 8 consecutive positions, so each 16-byte
// load/store instruction of a wave touches 2 KiB of contiguous rows for a
// contiguous [B, H, S, D] tensor (and whole rows for HF's transposed views).
#include <algorithm>

#include "common.h"

#pragma clang fp contract(off)

namespace mla {
namespace {

constexpr int kThreads = 256;
constexpr int kHeadsPerThread = 4;

struct RopeTensor {
  const void* in;
  void* out;
  int64_t H;
  int64_t sb, sh, ss;     // input strides (elements)
  int64_t osb, osh, oss;  // output strides
};

struct RopeArgs {
  RopeTensor t[2];  // q, k (k.H == 0 when absent)
  int64_t B, S;
  int half;          // D / 2
  int chunks;        // half / VEC
  int groups;        // ceil((Hq + Hk) / kHeadsPerThread)
  float sgn;
  // table mode
  const void* cos;
  const void* sin;
  int64_t csb, csh, css, ssb, ssh, sss;
  // position mode
  const int64_t* pos;
  int64_t psb, pss;
  const float* inv_freq;
};

template <typename T, int N>
__device__ __forceinline__ void load_any(const T* p, float* out) {
  if constexpr (N * sizeof(T) >= 16 || N == 1) {
    load_n<T, N>(p, out);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = to_f32(p[i]);
  }
}

// Outputs are streamed (never re-read by this kernel): 16-byte stores carry
// the non-temporal hint, so they do not sit in L2 as dirty lines to be
// written back when the kernel ends.
template <typename T, int N>
__device__ __forceinline__ void store_any(T* p, const float* in) {
  if constexpr (N * sizeof(T) >= 16) {
    store_n_nt<T, N>(p, in);
  } else if constexpr (N == 1) {
    store_n<T, N>(p, in);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = from_f32<T>(in[i]);
  }
}

// sin and cos of an fp32 angle: reduction by pi/2 in two fp32 parts with
// fused multiply-adds (Cody-Waite; the quotient is exact for |a| < 2^22),
// then the Taylor series of sin to r^9 and cos to r^10 on |r| <= pi/4 and the
// quadrant's sign / swap. Largest error against the exact values, checked
// on 10^5 angles per range up to |a| = 10^6 in simulated fp32: 6.5e-8.
// Angles of 2^21 and more (far beyond any rotary position) use sincosf.
__device__ __forceinline__ void rope_sincos(float a, float& sn, float& cs) {
  if (__builtin_expect(fabsf(a) >= 2097152.f, 0)) {
    sincosf(a, &sn, &cs);
    return;
  }
  const float kTwoOverPi = 0.636619746685028076f;
  const float kHalfPiHi = 1.57079637050628662f;    // fp32(pi / 2)
  const float kHalfPiLo = -4.37113882867379300e-8f;  // pi / 2 - kHalfPiHi
  const float n = rintf(a * kTwoOverPi);
  float r = fmaf(n, -kHalfPiHi, a);
  r = fmaf(n, -kHalfPiLo, r);
  const float r2 = r * r;
  float ps = fmaf(r2, 2.75573188e-6f, -1.98412701e-4f);  // 1/9!, -1/7!
  ps = fmaf(r2, ps, 8.33333377e-3f);                      // 1/5!
  ps = fmaf(r2, ps, -0.166666672f);                       // -1/3!
  const float sr = fmaf(r * r2, ps, r);
  float pc = fmaf(r2, -2.75573200e-7f, 2.48015876e-5f);  // -1/10!, 1/8!
  pc = fmaf(r2, pc, -1.38888892e-3f);                     // -1/6!
  pc = fmaf(r2, pc, 4.16666679e-2f);                      // 1/4!
  pc = fmaf(r2, pc, -0.5f);                               // -1/2!
  const float cr = fmaf(r2, pc, 1.0f);
  const int q = (int)n & 3;
  const float s0 = (q & 1) ? cr : sr;  // quadrant q: sin = (sr, cr, -sr, -cr)[q]
  const float c0 = (q & 1) ? sr : cr;  //             cos = (cr, -sr, -cr, sr)[q]
  sn = (q & 2) ? -s0 : s0;
  cs = ((q + 1) & 2) ? -c0 : c0;
}

// POS_MODE: cos/sin from positions; otherwise from tables of type TC.
// IDX: int32_t when every element offset of every operand fits in 31 bits
// (checked on the host), which halves the address registers per head.
template <typename TX, typename TC, typename TO, int VEC, bool POS_MODE, typename IDX>
__global__ __launch_bounds__(kThreads) void rope_kernel(const RopeArgs a) {
  // blockIdx.y picks the head group, so head selection (q or k, strides)
  // is uniform across the block and lives in scalar registers.
  const int64_t per_group = a.B * a.S * a.chunks;
  const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (gid >= per_group) return;
  const int group = (int)blockIdx.y;
  int64_t rem = gid;
  const int chunk = (int)(rem % a.chunks);
  rem /= a.chunks;
  const IDX s = (IDX)(rem % a.S);
  const IDX b = (IDX)(rem / a.S);
  const int j0 = chunk * VEC;

  const int64_t Hq = a.t[0].H;
  const int64_t Htot = Hq + a.t[1].H;
  const int64_t h_begin = (int64_t)group * kHeadsPerThread;

  // Issue every head's loads before any math: up to 2 * kHeadsPerThread
  // 16-byte loads in flight per thread, kept as raw packs until used. Heads
  // past the end re-load the last head (no branch around the loads); their
  // results are not stored.
  Pack<TX, VEC> raw_lo[kHeadsPerThread], raw_hi[kHeadsPerThread];
#pragma unroll
  for (int t = 0; t < kHeadsPerThread; ++t) {
    const int64_t vh = (h_begin + t < Htot) ? h_begin + t : Htot - 1;
    {
      const int ti = vh < Hq ? 0 : 1;
      const RopeTensor& tt = a.t[ti];
      const int64_t h = vh - (ti ? Hq : 0);
      const TX* xp = static_cast<const TX*>(tt.in) + (b * (IDX)tt.sb + (IDX)h * (IDX)tt.sh + s * (IDX)tt.ss + j0);
      raw_lo[t] = load_pack_nt<TX, VEC>(xp);
      raw_hi[t] = load_pack_nt<TX, VEC>(xp + a.half);
    }
  }

  // cos/sin are computed while the loads above are in flight.
  float c_lo[VEC], s_lo[VEC];
  float c_hi_t[POS_MODE ? 1 : VEC], s_hi_t[POS_MODE ? 1 : VEC];
  // position mode duplicates the angle across the two halves (HF layout)
  float* c_hi = POS_MODE ? c_lo : c_hi_t;
  float* s_hi = POS_MODE ? s_lo : s_hi_t;
  const bool table_per_head = !POS_MODE && (a.csh != 0 || a.ssh != 0);
  if constexpr (POS_MODE) {
    const float p = (float)a.pos[(int64_t)b * a.psb + (int64_t)s * a.pss];
    float invf[VEC];
    load_any<float, VEC>(a.inv_freq + j0, invf);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float ang = p * invf[e];
      float sn, cs;
      rope_sincos(ang, sn, cs);
      c_lo[e] = cs;
      s_lo[e] = sn * a.sgn;
    }
  }
  auto load_table = [&](int64_t h) {
    const TC* cp = static_cast<const TC*>(a.cos) + (b * (IDX)a.csb + (IDX)h * (IDX)a.csh + s * (IDX)a.css + j0);
    const TC* sp = static_cast<const TC*>(a.sin) + (b * (IDX)a.ssb + (IDX)h * (IDX)a.ssh + s * (IDX)a.sss + j0);
    load_any<TC, VEC>(cp, c_lo);
    load_any<TC, VEC>(cp + a.half, c_hi);
    load_any<TC, VEC>(sp, s_lo);
    load_any<TC, VEC>(sp + a.half, s_hi);
#pragma unroll
    for (int e = 0; e < VEC; ++e) s_lo[e] *= a.sgn;
    if constexpr (!POS_MODE) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) s_hi[e] *= a.sgn;
    }
  };
  if constexpr (!POS_MODE) {
    if (!table_per_head) load_table(0);
  }

#pragma unroll
  for (int t = 0; t < kHeadsPerThread; ++t) {
    const int64_t vh = h_begin + t;
    if (vh < Htot) {
      const int ti = vh < Hq ? 0 : 1;
      const RopeTensor& tt = a.t[ti];
      const int64_t h = vh - (ti ? Hq : 0);
      if constexpr (!POS_MODE) {
        if (table_per_head) load_table(h);
      }
      TO* yp = static_cast<TO*>(tt.out) + (b * (IDX)tt.osb + (IDX)h * (IDX)tt.osh + s * (IDX)tt.oss + j0);
      float y_lo[VEC], y_hi[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float xl = to_f32(raw_lo[t].v[e]);
        const float xh = to_f32(raw_hi[t].v[e]);
        // x * cos + rotate_half(x) * sin, rotate_half([x1, x2]) = [-x2, x1]
        y_lo[e] = xl * c_lo[e] + (-xh) * s_lo[e];
        y_hi[e] = xh * c_hi[e] + xl * s_hi[e];
      }
      store_any<TO, VEC>(yp, y_lo);
      store_any<TO, VEC>(yp + a.half, y_hi);
    }
  }
}

bool fill_tensor(RopeTensor& t, const void* in, void* out, const int64_t* g, int64_t& B,
                 int64_t& S, bool first) {
  t.in = in;
  t.out = out;
  t.H = g[1];
  t.sb = g[3];
  t.sh = g[4];
  t.ss = g[5];
  t.osb = g[6];
  t.osh = g[7];
  t.oss = g[8];
  if (first) {
    B = g[0];
    S = g[2];
    return true;
  }
  return g[0] == B && g[2] == S;
}

template <typename TX, typename TC, typename TO, bool POS_MODE>
int launch_rope(RopeArgs& a, int64_t D, hipStream_t st) {
  constexpr int V_FULL = vec16<TX>();
  // Vector path: every 16-byte chunk of x / out / tables stays aligned.
  bool vec_ok = (a.half % V_FULL) == 0;
  for (int i = 0; i < 2 && vec_ok; ++i) {
    const RopeTensor& t = a.t[i];
    if (t.H == 0) continue;
    vec_ok = aligned16(t.in) && aligned16(t.out) &&
             ((t.sb | t.sh | t.ss) * (int64_t)sizeof(TX)) % 16 == 0 &&
             ((t.osb | t.osh | t.oss) * (int64_t)sizeof(TO)) % 16 == 0;
  }
  if (POS_MODE && vec_ok) vec_ok = aligned16(a.inv_freq);
  if (!POS_MODE && vec_ok)
    vec_ok = aligned16(a.cos) && aligned16(a.sin) &&
             ((a.csb | a.csh | a.css | a.ssb | a.ssh | a.sss) * (int64_t)sizeof(TC)) % 16 == 0 &&
             ((int64_t)a.half * (int64_t)sizeof(TC)) % 16 == 0;
  const int vec = vec_ok ? V_FULL : 1;
  a.chunks = a.half / vec;
  const int64_t Htot = a.t[0].H + a.t[1].H;
  a.groups = (int)((Htot + kHeadsPerThread - 1) / kHeadsPerThread);
  const int64_t per_group = a.B * a.S * (int64_t)a.chunks;
  if (per_group == 0 || a.groups == 0) return ML_OK;
  const int64_t blocks = (per_group + kThreads - 1) / kThreads;
  ML_CHECK(blocks <= 0x7fffffffLL && a.groups <= 65535, "rope: problem too large");
  const dim3 grid((unsigned)blocks, (unsigned)a.groups);
  // Largest element offset any thread forms (all strides are non-negative).
  auto span = [](int64_t B, int64_t H, int64_t S, int64_t sb, int64_t sh, int64_t ss, int64_t D) {
    return (B - 1) * sb + (H > 0 ? H - 1 : 0) * sh + (S - 1) * ss + D;
  };
  int64_t max_off = 0;
  for (int i = 0; i < 2; ++i) {
    const RopeTensor& t = a.t[i];
    if (t.H == 0) continue;
    max_off = std::max(max_off, span(a.B, t.H, a.S, t.sb, t.sh, t.ss, D));
    max_off = std::max(max_off, span(a.B, t.H, a.S, t.osb, t.osh, t.oss, D));
    if (!POS_MODE) {
      max_off = std::max(max_off, span(a.B, t.H, a.S, a.csb, a.csh, a.css, D));
      max_off = std::max(max_off, span(a.B, t.H, a.S, a.ssb, a.ssh, a.sss, D));
    }
  }
  const bool small = max_off < ((int64_t)1 << 31);
#define ML_ROPE(V, I) rope_kernel<TX, TC, TO, V, POS_MODE, I><<<grid, kThreads, 0, st>>>(a)
  if (vec_ok) {
    if (small) ML_ROPE(V_FULL, int32_t); else ML_ROPE(V_FULL, int64_t);
  } else {
    if (small) ML_ROPE(1, int32_t); else ML_ROPE(1, int64_t);
  }
#undef ML_ROPE
  ML_LAUNCH_CHECK();
  return ML_OK;
}

int setup_common(RopeArgs& a, const void* q, void* q_out, const int64_t* q_geom, const void* k,
                 void* k_out, const int64_t* k_geom, int64_t D, float sgn) {
  ML_CHECK(q_geom != nullptr, "rope: null q geometry");
  ML_CHECK(D > 0 && D % 2 == 0, "rope: head dim must be even and positive (got %lld)",
           (long long)D);
  ML_CHECK(D / 2 <= 0x7fffffff, "rope: head dim too large");
  a = RopeArgs{};
  fill_tensor(a.t[0], q, q_out, q_geom, a.B, a.S, true);
  if (k != nullptr) {
    ML_CHECK(k_geom != nullptr, "rope: null k geometry");
    ML_CHECK(fill_tensor(a.t[1], k, k_out, k_geom, a.B, a.S, false),
             "rope: q and k must share batch and sequence sizes");
  } else {
    a.t[1] = RopeTensor{};
  }
  ML_CHECK(a.B >= 0 && a.S >= 0 && a.t[0].H >= 0 && a.t[1].H >= 0, "rope: negative size");
  const int64_t elems = a.B * a.S * (a.t[0].H + a.t[1].H);
  ML_CHECK(elems == 0 || (q && q_out), "rope: null tensor pointer");
  ML_CHECK(k == nullptr || a.t[1].H == 0 || k_out != nullptr, "rope: null k output");
  a.half = (int)(D / 2);
  a.sgn = sgn;
  return ML_OK;
}

}  // namespace
}  // namespace mla

using namespace mla;

extern "C" int ml_rope_table(const void* q, void* q_out, const int64_t* q_geom, const void* k,
                             void* k_out, const int64_t* k_geom, int64_t D, const void* cos,
                             const void* sin, const int64_t* cs_geom, float sgn, int x_dtype,
                             int cs_dtype, int out_dtype, void* stream) {
  RopeArgs a;
  int rc = setup_common(a, q, q_out, q_geom, k, k_out, k_geom, D, sgn);
  if (rc) return rc;
  const bool empty = a.B * a.S * (a.t[0].H + a.t[1].H) == 0;  // nothing is read
  ML_CHECK(cs_geom && (empty || (cos && sin)), "rope: null cos/sin");
  a.cos = cos;
  a.sin = sin;
  a.csb = cs_geom[0];
  a.csh = cs_geom[1];
  a.css = cs_geom[2];
  a.ssb = cs_geom[3];
  a.ssh = cs_geom[4];
  a.sss = cs_geom[5];
  hipStream_t st = (hipStream_t)stream;
  // Output dtype is torch's promotion: x's dtype when the tables match it,
  // fp32 for any mixed pair of {fp32, bf16, fp16}.
  const int expect_out = (x_dtype == cs_dtype) ? x_dtype : ML_F32;
  ML_CHECK(out_dtype == expect_out,
           "rope: output dtype %d is not the promotion of x dtype %d and table dtype %d",
           out_dtype, x_dtype, cs_dtype);
  return dispatch_dtype(x_dtype, [&](auto tx) -> int {
    using TX = decltype(tx);
    return dispatch_dtype(cs_dtype, [&](auto tc) -> int {
      using TC = decltype(tc);
      if constexpr (std::is_same<TX, TC>::value) {
        return launch_rope<TX, TC, TX, false>(a, D, st);
      } else {
        return launch_rope<TX, TC, float, false>(a, D, st);
      }
    });
  });
}

extern "C" int ml_rope_pos(const void* q, void* q_out, const int64_t* q_geom, const void* k,
                           void* k_out, const int64_t* k_geom, int64_t D,
                           const int64_t* positions, int64_t pos_sb, int64_t pos_ss,
                           const float* inv_freq, float sgn, int x_dtype, void* stream) {
  RopeArgs a;
  int rc = setup_common(a, q, q_out, q_geom, k, k_out, k_geom, D, sgn);
  if (rc) return rc;
  const bool empty = a.B * a.S * (a.t[0].H + a.t[1].H) == 0;  // nothing is read
  ML_CHECK(empty || (positions && inv_freq), "rope: null positions / inv_freq");
  a.pos = positions;
  a.psb = pos_sb;
  a.pss = pos_ss;
  a.inv_freq = inv_freq;
  hipStream_t st = (hipStream_t)stream;
  return dispatch_dtype(x_dtype, [&](auto tx) -> int {
    using TX = decltype(tx);
    return launch_rope<TX, float, TX, true>(a, D, st);
  });
}

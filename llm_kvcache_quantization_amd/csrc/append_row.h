// The append's row quantizer, shared by the append kernel (quant_append.hip) and the tiled
// decode kernel's fused append (decode_tiled.h), so that both write the same bits: one
// wavefront quantises one (b, h, s) row of D = 128 values (2 per lane).
//
// Every product and sum here is rounded on its own, as torch rounds each tensor op: each
// function body turns fp contraction off (the file that includes this header keeps its own
// setting), so the compiler cannot fuse a * b + c.  The interpolation of torch.quantile,
// which ATen does compute as a fused multiply-add, calls fmaf explicitly.
#pragma once
#include "kvq_common.h"
#include "kvq.h"

#include <string>

namespace kvq {

int fail(int code, const std::string& msg);

// The INT4 group rescue's threshold (torch.quantile over every (row, group) dynamic scale of
// the append): up to kRescueRank scales it is found inside the launch that quantizes (the
// append kernel's work-groups, or the fused decode step's writer wave), walking down from the
// maximum when its ranks lie within kTopWalk of the top; rows are loaded kRowBatch at a time.
constexpr int kRescueRank = 1024;
constexpr int kRowBatch = 8;
constexpr int kTopWalk = 32;

struct AppendDev {
  int valid;
  int fmt;
  const half_t* x;
  int64_t xsb, xsh, xss;
  int B, H, S, gs;
  const void* st;
  int st_f32;
  int64_t st_sh, st_sg;
  const half_t* st_zp;
  int adaptive;
  float margin;
  int mixed;
  float rq;
  int rescue_all;
  uint8_t* codes;
  int64_t csb, csh, cst;
  void* so;
  int so_f32;
  int64_t sosb, sosh, sost, sosg;
  int n_out;
  const int32_t* oidx;
  half_t* oo;
  int64_t oosb, oosh, oost;
  int64_t wpos;
  int32_t* status;
  int tile32;  // codes in KVQ_LAYOUT_TILE32 (INT4_ASYM)
  float dq;              // dynamic scales: fp32(percentile / 100), or 0 for the absmax
  float dq_lo;           // KIVI V: fp32((100 - percentile) / 100), the low quantile
  const float* thr_ptr;  // group-rescue threshold computed by the large-n select, or NULL
  int64_t st_sb;         // INT4_KIVI K: batch stride of the per-channel parameters
  float* zo;             // INT4_KIVI V: per-token zero-point out (scale_out's strides)
};

// Scratch of the group rescue over more than kRescueMax (row, group) scales: an exact radix
// select, over the fp32 bit patterns of the append's dynamic group scales (all positive,
// so their bit patterns sort as their values; a NaN sorts last as in torch.sort), of
// sorted[lo] (4 histogram passes of 8 bits), then sorted[hi] (lo + 1) from the count of
// values <= sorted[lo] and the least value above it, then torch.quantile's interpolation.

__device__ __forceinline__ float ld_static(const AppendDev& a, int h, int g) {
#pragma clang fp contract(off)
  const int64_t off = (int64_t)h * a.st_sh + (int64_t)g * a.st_sg;
  return a.st_f32 ? reinterpret_cast<const float*>(a.st)[off]
                  : (float)reinterpret_cast<const half_t*>(a.st)[off];
}

// max over the lanes of one quantisation group (gs/2 consecutive lanes)
__device__ __forceinline__ float group_max(float v, int gs) {
#pragma clang fp contract(off)
  for (int o = 1; o < gs / 2; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// torch.quantile's linear interpolation between the order statistics a <= b with weight
// w = rank - floor(rank), as ATen's CPU lerp computes it: one fused multiply-add,
// fma(w, b - a, a) for w < 0.5, else fma(w - 1, b - a, b) (w - 1 is exact).  The unfused
// a + w (b - a) differs from it in the last bit for about 1 in 1000 inputs.
__device__ __forceinline__ float quantile_lerp(float a, float b, float w) {
#pragma clang fp contract(off)
  const float diff = b - a;
  return w < 0.5f ? fmaf(w, diff, a) : fmaf(w - 1.0f, diff, b);
}


// torch.quantile(|x|, q) over the gs values of the lane's quantisation group (gs / 2
// consecutive lanes holding 2 values each; a0, a1 = |x| of the lane's values), as the
// reference's percentile-clipped dynamic quantizers take it (src/quant/int8_basic.py:78-83,
// src/quant/int4_basic.py:84-90): every value's rank in the group (ties broken by channel
// index) selects the order statistics at floor / ceil of fp32(q) * (gs - 1), which are
// interpolated by quantile_lerp.  The group's lanes all return the result.
__device__ __forceinline__ int group_sum(int v, int gs) {
#pragma clang fp contract(off)
  for (int o = 1; o < gs / 2; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// The order statistics v[lo] <= v[hi] (ascending ranks, ties broken by channel index) of
// the gs finite values of the lane's group (a0, a1 = the lane's two values, any sign).  Near
// the top (the reference's 99.9 percentile over groups of up to 128 takes the two largest
// values) they come from walking the distinct values down from the maximum: value m with
// multiplicity c holds the ranks [gs - above - c, gs - above), `above` counting the values
// already passed, and gs - lo steps reach rank lo.  Near the bottom the same walk runs on
// the negated values (v[r] = -(-v)[gs - 1 - r]).  Elsewhere every value's rank is counted.
// The group's lanes all return the results.
__device__ inline void group_order_stats(float a0, float a1, int gs, int lo, int hi, int lane,
                                  float& vlo, float& vhi) {
#pragma clang fp contract(off)
  const bool top = gs - 1 - lo < 4, bottom = !top && hi < 4;
  if (top || bottom) {
    const float sg = top ? 1.0f : -1.0f;  // bottom: walk -v from its top
    const float b0 = sg * a0, b1 = sg * a1;
    const int rlo = top ? lo : gs - 1 - hi, rhi = top ? hi : gs - 1 - lo;  // ranks in -v
    const int steps = gs - rlo;
    float t = __builtin_inff(), wlo = 0.f, whi = 0.f;
    int above = 0;
    for (int it = 0; it < steps; ++it) {
      const float m = group_max(fmaxf(b0 < t ? b0 : -__builtin_inff(), b1 < t ? b1 : -__builtin_inff()), gs);
      const int c = group_sum((int)(b0 == m) + (int)(b1 == m), gs);
      const int r0 = gs - above - c, r1 = gs - above;  // ranks [r0, r1) hold m
      if (rlo >= r0 && rlo < r1) wlo = m;
      if (rhi >= r0 && rhi < r1) whi = m;
      above += c;
      t = m;
    }
    vlo = top ? wlo : -whi;
    vhi = top ? whi : -wlo;
    return;
  }
  const int nl = gs >> 1;
  const int base = lane & ~(nl - 1);
  const int e0 = 2 * (lane - base), e1 = e0 + 1;
  int r0 = 0, r1 = 0;
  for (int j = 0; j < nl; ++j) {
    const float b0 = __shfl(a0, base + j, 64), b1 = __shfl(a1, base + j, 64);
    const int f0 = 2 * j, f1 = 2 * j + 1;
    r0 += (b0 < a0 || (b0 == a0 && f0 < e0)) + (b1 < a0 || (b1 == a0 && f1 < e0));
    r1 += (b0 < a1 || (b0 == a1 && f0 < e1)) + (b1 < a1 || (b1 == a1 && f1 < e1));
  }
  // the values of ranks lo and hi, spread over the group
  vlo = group_max(fmaxf(r0 == lo ? a0 : -__builtin_inff(), r1 == lo ? a1 : -__builtin_inff()), gs);
  vhi = group_max(fmaxf(r0 == hi ? a0 : -__builtin_inff(), r1 == hi ? a1 : -__builtin_inff()), gs);
}

// torch.quantile(v, q) over the gs values of the lane's group (linear interpolation in fp32:
// rank = fp32(q) * (gs - 1), w = rank - floor(rank))
__device__ inline float group_quantile(float a0, float a1, int gs, float q, int lane) {
#pragma clang fp contract(off)
  const float rank = q * (float)(gs - 1);
  const int lo = (int)floorf(rank), hi = (int)ceilf(rank);
  float vlo, vhi;
  group_order_stats(a0, a1, gs, lo, hi, lane, vlo, vhi);
  return quantile_lerp(vlo, vhi, rank - (float)lo);
}

// group_max for values >= +0 (absolute values: the order of the maxima cannot change a bit)
// with DPP instead of the LDS crossbar: xor 1 and 2 within the quad, then the half-row and
// row mirrors (lane i with 7 - i, 15 - i), which pair lanes of the two already reduced halves
__device__ __forceinline__ float group_absmax(float v, int gs) {
#pragma clang fp contract(off)
  v = fmaxf(v, dppf<0xB1>(v));                       // quad_perm [1, 0, 3, 2]
  if (gs >= 8) v = fmaxf(v, dppf<0x4E>(v));          // quad_perm [2, 3, 0, 1]
  if (gs >= 16) v = fmaxf(v, dppf<0x141>(v));        // row_half_mirror
  if (gs >= 32) v = fmaxf(v, dppf<0x140>(v));        // row_mirror
  if (gs >= 64) v = fmaxf(v, __shfl_xor(v, 16, 64));
  if (gs >= 128) v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}

// Scale of group g for a row, before the per-format final clamp.
//  dyn_abs: absmax of the group's fp16 values (as float)
//  stv: the static scale of the group (ld_static)
__device__ __forceinline__ float int4_scale(const AppendDev& a, float stv, float dyn_abs, float thr) {
#pragma clang fp contract(off)
  float s = fmaxf(stv, 1e-5f);                                 // int4_cache.py:342
  const float dyn = __fdiv_rn(fmaxf(dyn_abs, 1e-5f), 7.0f);   // int4_cache.py:358
  if (a.adaptive) s = fmaxf(s * a.margin, dyn);                // :451-455
  if (a.mixed) s = fmaxf(s, dyn);                              // :457-458
  if (a.rescue_all) s = fmaxf(s, dyn);                         // :381-382
  else if (a.rq > 0.f && dyn >= thr) s = fmaxf(s, dyn);        // :384-390
  return fmaxf(s, 1e-5f);                                      // int4_basic.py:154
}

// dyn_abs: the group's absmax, or with a percentile its fp32 quantile of |x|
// dyn_abs: the group's absmax, or with a percentile its fp32 quantile of |x|; stv: the static
// scale of the group (ld_static; unused without a static table)
__device__ __forceinline__ half_t int8_scale16(const AppendDev& a, float stv, float dyn_abs) {
#pragma clang fp contract(off)
  if (a.st == nullptr) {
    // dynamic path: the fp16 absmax clamped in fp16 (int8_basic.py:85, :91-92), or the fp32
    // quantile clamped in fp32 then rounded to fp16 (:78-83, :91-92); then abs_max / 127 in
    // fp16 arithmetic (:94)
    const half_t am = a.dq > 0.f ? (half_t)fmaxf(dyn_abs, 1e-5f)
                                 : (half_t)fmaxf(dyn_abs, (float)(half_t)1e-5f);
    return (half_t)__fdiv_rn((float)am, 127.0f);
  }
  float s = stv;
  if (a.adaptive) {
    s = fmaxf(s, 1e-5f) * a.margin;                            // int8_cache.py:326,398
    const float dyn = __fdiv_rn(fmaxf(dyn_abs, 1e-5f), 127.0f);  // :348
    s = fmaxf(s, dyn);
  }
  if (!a.adaptive) return int8_static_scale16(s, a.st_f32);
  return (half_t)fmaxf(s, 1e-5f);                              // int8_basic.py:159
}

// the lane's two input values of append row `row` (row = (b * H + h) * S + s)
__device__ __forceinline__ const half_t* row_x(const AppendDev& a, int row) {
#pragma clang fp contract(off)
  const int s_idx = row % a.S, bh = row / a.S, h = bh % a.H, b = bh / a.H;
  return a.x + (int64_t)b * a.xsb + (int64_t)h * a.xsh + (int64_t)s_idx * a.xss;
}
__device__ __forceinline__ half2v load_x(const AppendDev& a, int row, int lane) {
#pragma clang fp contract(off)
  return *reinterpret_cast<const half2v*>(row_x(a, row) + 2 * lane);
}

// The static scale of the lane's group in append row `row` as its raw bits (fp32, or fp16 in
// the low half; 0 without a static table), and their value.  The fused step's writer requests
// the bits at the start of the kernel and converts them where it quantizes: converting at the
// load (one branch per table dtype) made the compiler wait for every outstanding load there,
// the q loads and the first cache tiles included.
__device__ __forceinline__ uint32_t row_static_bits(const AppendDev& a, int row, int lane) {
  if (a.st == nullptr || a.fmt == KVQ_FMT_INT4_ASYM || a.fmt == KVQ_FMT_INT4_KIVI ||
      a.fmt == KVQ_FMT_INT8_KIVI)
    return 0u;
  const int64_t off = (int64_t)((row / a.S) % a.H) * a.st_sh + (int64_t)((2 * lane) / a.gs) * a.st_sg;
  return a.st_f32 ? reinterpret_cast<const uint32_t*>(a.st)[off]
                  : (uint32_t)reinterpret_cast<const uint16_t*>(a.st)[off];
}
__device__ __forceinline__ float static_value(const AppendDev& a, uint32_t bits) {
  return a.st_f32 ? __builtin_bit_cast(float, bits) : (float)__builtin_bit_cast(half_t, (uint16_t)bits);
}
// the static scale of the lane's group in append row `row` (0 without a static table)
__device__ __forceinline__ float row_static(const AppendDev& a, int row, int lane) {
#pragma clang fp contract(off)
  if (a.st == nullptr || a.fmt == KVQ_FMT_INT4_ASYM || a.fmt == KVQ_FMT_INT4_KIVI ||
      a.fmt == KVQ_FMT_INT8_KIVI)
    return 0.f;
  return ld_static(a, (row / a.S) % a.H, (2 * lane) / a.gs);
}

// Quantizes append row `row` = (b * H + h) * S + s_idx whose lane values xv (and static
// scale stv, row_static) were loaded by the caller.  FMT: the side's format when the caller
// knows it at compile time (the fused decode step's writer: only that format's code is
// built into its kernel), or -1 for a.fmt.
template <int FMT = -1>
__device__ __forceinline__ void quant_row_bhs(const AppendDev& a, int b, int h, int s_idx, int row,
                                              int lane, float thr, half2v xv, float stv) {
#pragma clang fp contract(off)
  const int fmt = FMT >= 0 ? FMT : a.fmt;
  const int64_t t = a.wpos + s_idx;
  const half_t* xr = row_x(a, row);
  const float x0 = (float)xv.x, x1 = (float)xv.y;
  const int d0 = 2 * lane;
  const int g = d0 / a.gs;

  // NaN / Inf detection (src/quant/_common.py:13-20): reported through status[0]
  const bool bad = !(__builtin_isfinite(x0) && __builtin_isfinite(x1));
  const unsigned long long badmask = __ballot(bad);
  if (badmask && lane == 0 && a.status) atomicOr(&a.status[0], 1);

  // the group's absmax, or for a percentile-clipped dynamic scale its quantile of |x|
  const bool pct = a.st == nullptr && a.dq > 0.f &&
                   (fmt == KVQ_FMT_INT8_SYM || fmt == KVQ_FMT_INT4_SYM);
  const float am = pct ? group_quantile(fabsf(x0), fabsf(x1), a.gs, a.dq, lane)
                       : group_absmax(fmaxf(fabsf(x0), fabsf(x1)), a.gs);
  uint8_t* crow = a.codes + (int64_t)b * a.csb + (int64_t)h * a.csh + t * a.cst;
  int clipped = 0;

  if (fmt == KVQ_FMT_INT8_SYM) {
    const half_t s16 = int8_scale16(a, stv, am);
    const float sf = (float)s16;
    *reinterpret_cast<uint16_t*>(crow + d0) = int8_pack_pair(x0, x1, s16, clipped);
    // the clip statistic is the static-scale path's (int8_cache.py:401-419)
    if (a.st == nullptr) clipped = 0;
    if (a.so && (d0 % a.gs) == 0) {
      const int64_t off = (int64_t)b * a.sosb + (int64_t)h * a.sosh + t * a.sost + (int64_t)g * a.sosg;
      if (a.so_f32) reinterpret_cast<float*>(a.so)[off] = sf;
      else reinterpret_cast<half_t*>(a.so)[off] = s16;
    }
  } else if (fmt == KVQ_FMT_INT4_SYM) {
    float s;
    if (a.st == nullptr) {
      // the fp16 absmax clamped in fp16, or the fp32 quantile clamped in fp32, then divided
      // in fp32 (int4_basic.py:84-99)
      s = __fdiv_rn(pct ? fmaxf(am, 1e-5f) : fmaxf(am, (float)(half_t)1e-5f), 7.0f);
    } else {
      s = int4_scale(a, stv, am, thr);
    }
    const float q0 = fminf(fmaxf(rintf(__fdiv_rn(x0, s)), -7.f), 7.f);
    const float q1 = fminf(fmaxf(rintf(__fdiv_rn(x1, s)), -7.f), 7.f);
    crow[lane] = (uint8_t)((((int)q0 + 8) << 4) | ((int)q1 + 8));
    if (a.st != nullptr) {
      const float bound = s * 7.0f;                          // int4_cache.py:473-476
      clipped = (fabsf(x0) > bound) + (fabsf(x1) > bound);
    }
    if (a.so && (d0 % a.gs) == 0) {
      const int64_t off = (int64_t)b * a.sosb + (int64_t)h * a.sosh + t * a.sost + (int64_t)g * a.sosg;
      if (a.so_f32) reinterpret_cast<float*>(a.so)[off] = s;
      else reinterpret_cast<half_t*>(a.so)[off] = (half_t)s;
    }
  } else if (fmt == KVQ_FMT_INT4_KIVI || fmt == KVQ_FMT_INT8_KIVI) {
    // asymmetric_quant.py:24-141 with qmin, qmax = -8, 7 (4 bits) or -128, 127 (8 bits)
    const bool b8 = fmt == KVQ_FMT_INT8_KIVI;
    const float qmin = b8 ? -128.f : -8.f, qmax = b8 ? 127.f : 7.f;
    float s0, s1, z0, z1;
    if (a.st != nullptr) {
      // K: frozen per-channel parameters (kivi_style_cache.py:548-566)
      const int64_t o = (int64_t)b * a.st_sb + (int64_t)h * a.st_sh + (int64_t)d0 * a.st_sg;
      const float* ps = reinterpret_cast<const float*>(a.st);
      const float* pz = reinterpret_cast<const float*>(a.st_zp);
      s0 = ps[o]; s1 = ps[o + a.st_sg];
      z0 = pz[o]; z1 = pz[o + a.st_sg];
    } else {
      // V: per-token range over the 128 channels (asymmetric_quant.py:97-141): min / max, or
      // with a percentile below 100 torch.quantile at (100 - p) / 100 and p / 100
      float mn, mx;
      if (a.dq > 0.f) {
        mn = group_quantile(x0, x1, 128, a.dq_lo, lane);
        mx = group_quantile(x0, x1, 128, a.dq, lane);
      } else {
        mn = fminf(x0, x1);
        mx = fmaxf(x0, x1);
        for (int o = 32; o > 0; o >>= 1) {
          mn = fminf(mn, __shfl_xor(mn, o, 64));
          mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        }
      }
      // range floor max(1e-5, fp16 tiny * (qmax - qmin)) = (qmax - qmin) * 2^-14;
      // z = min - qmin s (qmin s is exact)
      const float span = qmax - qmin;
      s0 = s1 = __fdiv_rn(fmaxf(mx - mn, span * 6.103515625e-05f), span);
      z0 = z1 = mn - qmin * s0;
      if (lane == 0 && a.so) {
        const int64_t off = (int64_t)b * a.sosb + (int64_t)h * a.sosh + t * a.sost;
        reinterpret_cast<float*>(a.so)[off] = s0;
        a.zo[off] = z0;
      }
    }
    const float u0 = __fdiv_rn(x0 - z0, s0), u1 = __fdiv_rn(x1 - z1, s1);
    // frozen-K out-of-range count, of the unrounded quotient (kivi_style_cache.py:549-560)
    if (a.st != nullptr) clipped = (u0 < qmin || u0 > qmax) + (u1 < qmin || u1 > qmax);
    const float r0 = rintf(u0), r1 = rintf(u1);
    const int q0 = (int)fminf(fmaxf(r0, qmin), qmax), q1 = (int)fminf(fmaxf(r1, qmin), qmax);
    if (b8)
      *reinterpret_cast<uint16_t*>(crow + d0) = (uint16_t)((q0 & 0xFF) | ((q1 & 0xFF) << 8));
    else
      crow[lane] = (uint8_t)(((q0 + 8) << 4) | (q1 + 8));
  } else if (fmt == KVQ_FMT_FP16) {  // a 16-bit side stores the row as it comes
    *reinterpret_cast<half2v*>(crow + 4 * lane) = xv;
  } else {  // KVQ_FMT_INT4_ASYM, static parameters
    const int64_t off = (int64_t)h * a.st_sh + (int64_t)g * a.st_sg;
    const float s = (float)reinterpret_cast<const half_t*>(a.st)[off];
    const float z = (float)a.st_zp[off];
    const uint8_t byte = asym_pack_pair(x0, x1, s, z, clipped);
    if (a.tile32)
      a.codes[(int64_t)b * a.csb + (int64_t)h * a.csh + tile32_offset(t, lane)] = byte;
    else
      crow[lane] = byte;
    if (a.n_out > 0 && lane < a.n_out) {
      const int ch = min(max(a.oidx[h * a.n_out + lane], 0), 127);
      half_t* orow = a.oo + (int64_t)b * a.oosb + (int64_t)h * a.oosh + t * a.oost;
      orow[lane] = xr[ch];
    }
  }
  // clipped-element count (int8_cache.py:407-419, int4_cache.py:468-485)
  // (each lane clips 0, 1 or 2 values: two ballots count them on the scalar unit)
  const int nclip = __builtin_popcountll(__ballot(clipped & 1)) + 2 * __builtin_popcountll(__ballot(clipped & 2));
  if (lane == 0 && a.status && nclip) atomicAdd(&a.status[1], nclip);
}

template <int FMT = -1>
__device__ __forceinline__ void quant_row_x(const AppendDev& a, int row, int lane, float thr,
                                            half2v xv, float stv) {
  const int s_idx = row % a.S;
  const int bh = row / a.S;
  quant_row_bhs<FMT>(a, bh / a.H, bh % a.H, s_idx, row, lane, thr, xv, stv);
}


// lds_top_quantile by one wave alone, without barriers: lane l holds the scales v[l + 64 r]
// (r < R, n <= 64 R) in registers; the maximum of each step is a DPP wave reduction and its
// multiplicity the population count of one ballot per slot.  Every lane returns the result.
template <int R>
__device__ __forceinline__ float wave_top_quantile(const float* v, int n, int lo, int hi, float w, int lane) {
#pragma clang fp contract(off)
  float x[R];
#pragma unroll
  for (int r = 0; r < R; ++r) x[r] = lane + 64 * r < n ? v[lane + 64 * r] : -1.0f;  // below every scale
  float t = __builtin_inff(), vlo = 0.f, vhi = 0.f;
  int above = 0;
  for (int it = 0; it < kTopWalk && above <= n - 1 - lo; ++it) {
    float m = -1.0f;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (x[r] < t) m = fmaxf(m, x[r]);
    m = wave_max64(m);
    int c = 0;  // the multiplicity: a ballot per slot, counted on the scalar unit
#pragma unroll
    for (int r = 0; r < R; ++r) c += __builtin_popcountll(__ballot(x[r] == m));
    const int r0 = n - above - c, r1 = n - above;
    if (lo >= r0 && lo < r1) vlo = m;
    if (hi >= r0 && hi < r1) vhi = m;
    above += c;
    t = m;
  }
  return quantile_lerp(vlo, vhi, w);
}

// The rank of torch.quantile's lower order statistic for level q over n values, and whether
// the walk from the top reaches it (host and device compute the same fp32 rank).
__host__ __device__ inline bool rescue_walk_ok(float q, int n) {
#pragma clang fp contract(off)
  if (n <= 0 || n > kRescueRank) return false;
  const float rank = q * (float)(n - 1);
  const int lo = (int)floorf(rank);
  return n - 1 - lo < kTopWalk;
}

// The group-rescue threshold of a one-token append side found by one wave alone (the fused
// decode step's writer), over at most kRescueRows rows (rows = B * H) in groups of 16 or more.
// rescue_fetch issues the rows' loads early (lane l: the 32 dwords of channels
// 64 (l % 2) .. + 63 of row l / 2); rescue_thr_rows then takes each lane's group maxima (a
// group of 128 with its partner lane), writes the scales fmax(absmax, 1e-5) / 7 to dyn (LDS
// of this wave alone; a wave barrier orders the writes before the walk's reads) and walks
// from the top.  Needs
// rescue_walk_ok(a.rq, rows * 128 / gs).
constexpr int kRescueRows = 32;
struct RescueRows {
  uint32_t w[32];
};
__device__ __forceinline__ void rescue_fetch(const AppendDev& a, int lane, RescueRows& x) {
  const int rows = a.B * a.H * a.S, r = lane >> 1;
  const uint32_t* p = reinterpret_cast<const uint32_t*>(row_x(a, r < rows ? r : 0)) + 32 * (lane & 1);
#pragma unroll
  for (int i = 0; i < 32; ++i) x.w[i] = p[i];
}
__device__ __forceinline__ float rescue_thr_rows(const AppendDev& a, int lane, const RescueRows& x,
                                                 float* dyn) {
#pragma clang fp contract(off)
  const int rows = a.B * a.H * a.S, gs = a.gs, G = 128 / gs, n = rows * G;
  const int r = lane >> 1, hh = lane & 1;
  float m16[4];  // the maxima of |x| over the lane's four runs of 16 channels
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const half2v h = as_h2(x.w[8 * k + i]);
      m = fmaxf(m, fmaxf(fabsf((float)h.x), fabsf((float)h.y)));
    }
    m16[k] = m;
  }
  float mm[4] = {m16[0], m16[1], m16[2], m16[3]};
  int ng = 4;  // the lane's groups
  if (gs == 32) {
    mm[0] = fmaxf(m16[0], m16[1]);
    mm[1] = fmaxf(m16[2], m16[3]);
    ng = 2;
  } else if (gs >= 64) {
    mm[0] = fmaxf(fmaxf(m16[0], m16[1]), fmaxf(m16[2], m16[3]));
    ng = 1;
    if (gs == 128) {
      mm[0] = fmaxf(mm[0], dppf<0xB1>(mm[0]));  // with the partner lane's half
      ng = hh == 0 ? 1 : 0;
    }
  }
  if (r < rows)
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < ng) dyn[r * G + hh * ng + k] = __fdiv_rn(fmaxf(mm[k], 1e-5f), 7.0f);
  // the walk below reads other lanes' writes: a wave-scope fence and barrier keep the
  // compiler from moving those reads above the writes (the LDS executes one wave's
  // instructions in order)
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float rank = a.rq * (float)(n - 1);
  const int lo = (int)floorf(rank), hi = (int)ceilf(rank);
  const float w = rank - (float)lo;
  return n <= 64    ? wave_top_quantile<1>(dyn, n, lo, hi, w, lane)
         : n <= 128 ? wave_top_quantile<2>(dyn, n, lo, hi, w, lane)
                    : wave_top_quantile<4>(dyn, n, lo, hi, w, lane);
}

// The device description of one side of an append call (validated)
inline int fill_dev(const kvq_append_params* p, AppendDev& d, const char* name) {
  d = AppendDev{};
  if (!p) return KVQ_OK;
  const std::string n(name);
  if (p->format != KVQ_FMT_INT8_SYM && p->format != KVQ_FMT_INT4_SYM &&
      p->format != KVQ_FMT_INT4_ASYM && p->format != KVQ_FMT_INT4_KIVI &&
      p->format != KVQ_FMT_INT8_KIVI && p->format != KVQ_FMT_FP16)
    return fail(KVQ_ERR_INVALID, n + ": unknown format");
  const bool kivi = p->format == KVQ_FMT_INT4_KIVI || p->format == KVQ_FMT_INT8_KIVI;
  if (p->head_dim != 128) return fail(KVQ_ERR_UNSUPPORTED, n + ": head_dim must be 128");
  const int gs = p->group_size;
  if (gs != 8 && gs != 16 && gs != 32 && gs != 64 && gs != 128)
    return fail(KVQ_ERR_UNSUPPORTED, n + ": group_size must be 8, 16, 32, 64 or 128");
  if (p->batch < 0 || p->heads < 0 || p->seq_new < 0)
    return fail(KVQ_ERR_INVALID, n + ": negative size");
  if (!p->x || !p->codes) return fail(KVQ_ERR_INVALID, n + ": x/codes is NULL");
  if (((uintptr_t)p->x % 4) || (p->x_stride_b % 2) || (p->x_stride_h % 2) || (p->x_stride_s % 2))
    return fail(KVQ_ERR_UNSUPPORTED, n + ": x rows must be 4-byte aligned");
  if ((p->format == KVQ_FMT_INT8_SYM || p->format == KVQ_FMT_INT8_KIVI) &&
      (((uintptr_t)p->codes % 2) || p->codes_stride_b % 2 || p->codes_stride_h % 2 ||
       p->codes_stride_t % 2))
    return fail(KVQ_ERR_UNSUPPORTED, n + ": int8 code rows must be 2-byte aligned");
  if (p->format == KVQ_FMT_FP16) {
    if (((uintptr_t)p->codes % 4) || p->codes_stride_b % 4 || p->codes_stride_h % 4 ||
        p->codes_stride_t % 4)
      return fail(KVQ_ERR_UNSUPPORTED, n + ": fp16 rows must be 4-byte aligned");
    if (p->codes_layout != KVQ_LAYOUT_ROWS || p->static_scale || p->scale_out)
      return fail(KVQ_ERR_INVALID, n + ": an FP16 side takes token rows and no scales");
  }
  if (p->write_pos < 0 || p->write_pos + p->seq_new > p->capacity)
    return fail(KVQ_ERR_INVALID, n + ": write_pos + seq_new exceeds capacity");
  if (p->format == KVQ_FMT_INT4_ASYM) {
    if (gs != 32) return fail(KVQ_ERR_UNSUPPORTED, n + ": INT4_ASYM needs group_size 32");
    if (!p->static_scale || !p->static_zp || p->static_scale_dtype != KVQ_DTYPE_F16)
      return fail(KVQ_ERR_INVALID, n + ": INT4_ASYM needs fp16 static scale and zero-point");
    if (p->n_outlier != 0 && (p->n_outlier != 4 || !p->outlier_idx || !p->outlier_out))
      return fail(KVQ_ERR_INVALID, n + ": outliers need n_outlier == 4 and both pointers");
  } else if (p->n_outlier != 0) {
    return fail(KVQ_ERR_UNSUPPORTED, n + ": outlier channels need INT4_ASYM");
  }
  if (kivi) {
    if (p->codes_layout != KVQ_LAYOUT_ROWS)
      return fail(KVQ_ERR_UNSUPPORTED, n + ": KIVI codes are in token rows");
    if (p->static_scale) {
      if (!p->static_zp || p->static_scale_dtype != KVQ_DTYPE_F32)
        return fail(KVQ_ERR_INVALID, n + ": KIVI K needs fp32 static scale and zero-point");
    } else if (!p->scale_out || !p->zp_out || p->scale_out_dtype != KVQ_DTYPE_F32) {
      return fail(KVQ_ERR_INVALID, n + ": KIVI V needs fp32 scale_out and zp_out");
    }
  }
  if (!(p->dyn_quantile >= 0.f && p->dyn_quantile < 1.f))
    return fail(KVQ_ERR_INVALID, n + ": dyn_quantile must lie in [0, 1)");
  if (p->dyn_quantile_lo != 0.f &&
      !(kivi && !p->static_scale && p->dyn_quantile > 0.f && p->dyn_quantile_lo > 0.f &&
        p->dyn_quantile_lo < p->dyn_quantile))
    return fail(KVQ_ERR_INVALID, n + ": dyn_quantile_lo is for KIVI V, in (0, dyn_quantile)");
  if (kivi && !p->static_scale && p->dyn_quantile > 0.f && p->dyn_quantile_lo == 0.f)
    return fail(KVQ_ERR_INVALID, n + ": KIVI V with a percentile needs dyn_quantile_lo");
  if (p->codes_layout != KVQ_LAYOUT_ROWS && p->codes_layout != KVQ_LAYOUT_TILE32)
    return fail(KVQ_ERR_INVALID, n + ": unknown codes_layout");
  if (p->codes_layout == KVQ_LAYOUT_TILE32) {
    if (p->format != KVQ_FMT_INT4_ASYM)
      return fail(KVQ_ERR_UNSUPPORTED, n + ": the TILE32 layout is for INT4_ASYM only");
    if (p->codes_stride_t != 64 || p->capacity % 32)
      return fail(KVQ_ERR_INVALID, n + ": TILE32 needs codes_stride_t == 64 and capacity % 32 == 0");
  }
  d.valid = p->batch * p->heads * p->seq_new > 0;
  d.fmt = p->format;
  d.x = reinterpret_cast<const half_t*>(p->x);
  d.xsb = p->x_stride_b; d.xsh = p->x_stride_h; d.xss = p->x_stride_s;
  d.B = p->batch; d.H = p->heads; d.S = p->seq_new; d.gs = gs;
  d.st = p->static_scale;
  d.st_f32 = p->static_scale_dtype == KVQ_DTYPE_F32;
  d.st_sh = p->static_stride_h; d.st_sg = p->static_stride_g;
  d.st_zp = reinterpret_cast<const half_t*>(p->static_zp);
  d.adaptive = p->adaptive; d.margin = p->adaptive_margin;
  d.mixed = p->mixed_rescue; d.rq = p->rescue_quantile; d.rescue_all = p->rescue_all;
  d.codes = reinterpret_cast<uint8_t*>(p->codes);
  d.csb = p->codes_stride_b; d.csh = p->codes_stride_h; d.cst = p->codes_stride_t;
  d.so = p->scale_out; d.so_f32 = p->scale_out_dtype == KVQ_DTYPE_F32;
  d.sosb = p->so_stride_b; d.sosh = p->so_stride_h; d.sost = p->so_stride_t; d.sosg = p->so_stride_g;
  d.n_out = p->n_outlier; d.oidx = p->outlier_idx;
  d.oo = reinterpret_cast<half_t*>(p->outlier_out);
  d.oosb = p->oo_stride_b; d.oosh = p->oo_stride_h; d.oost = p->oo_stride_t;
  d.wpos = p->write_pos;
  d.status = p->status;
  d.tile32 = p->codes_layout == KVQ_LAYOUT_TILE32;
  d.st_sb = p->static_stride_b;
  d.zo = reinterpret_cast<float*>(p->zp_out);
  d.dq = p->dyn_quantile;
  d.dq_lo = p->dyn_quantile_lo;
  return KVQ_OK;
}

}  // namespace kvq

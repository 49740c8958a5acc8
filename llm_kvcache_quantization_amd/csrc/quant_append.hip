// Quantize-on-append for gfx950: new K/V rows (fp16) -> cache codes (+ scales).
//
// One wavefront quantises one (b, h, s) row of D = 128 values (2 per lane); the
// grid's y dimension selects K (0) or V (1) so one launch appends a layer.  The
// arithmetic restates the reference torch quantizers element for element:
//   INT8  sym: q = clamp(rne(fp16(x / s16)), -127, 127), s16 = fp16(max(s, 1e-5))
//              src/quant/int8_basic.py:111-164 (static), :18-108 (dynamic absmax)
//   INT4  sym: q = clamp(rne(x / s32), -7, 7), s32 = max(s, 1e-5) [+ rescue]
//              src/quant/int4_basic.py:115-159, src/cache/int4_cache.py:317-390
//   INT4 asym: q = clamp(rne((x - zp) / s), -8, 7)   (static s, zp per group)
//              src/kernels/triton_quantize_pack_int4.py:18-62,
//              tests/test_fused_quantize_pack.py:8-17
// Packing: byte = ((q[2i] + 8) << 4) | (q[2i+1] + 8)   src/quant/int4_basic.py:263-270
// Divisions are IEEE fp32 (__fdiv_rn) and rounding is ties-to-even (rintf), which is
// what torch does for tensor/tensor ops on both CPU and GPU.
#include "kvq_common.h"
#include "kvq.h"

#include <string>

// Every product and sum below is rounded on its own, as torch rounds each tensor op: the
// compiler must not contract a * b + c into one fused multiply-add.  HIP's __fmul_rn /
// __fsub_rn do not prevent that (they are inline operators compiled outside this pragma),
// so this file writes plain operators.  The interpolation of torch.quantile, which ATen
// does compute as a fused multiply-add, calls fmaf explicitly.
#pragma clang fp contract(off)

namespace kvq {

extern thread_local std::string g_last_error;
int fail(int code, const std::string& msg);

constexpr int kAppendWaves = 4;
constexpr int kRescueMax = 4096;  // (rows x groups) handled by the single-work-group rescue path
constexpr int kRescueRank = 1024;  // (rows x groups) up to which every work-group finds the
                                   // threshold itself by rank counting (decode-sized appends)
constexpr int kRowBatch = 8;      // rows per wave loaded at once on that path
constexpr int kTopWalk = 32;      // that path walks down from the maximum when the quantile's
                                  // ranks lie within kTopWalk of the top; else it sorts

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
struct RescueScratch {
  uint32_t hist[256];
  uint32_t prefix;  // bits of sorted[lo] fixed so far (all 32 after the last pass)
  uint32_t rank;    // rank of sorted[lo] among the values that match prefix
  uint32_t cnt_le;  // number of values <= sorted[lo]
  uint32_t min_gt;  // least bit pattern above sorted[lo]
  float thr;
  uint32_t pad[3];
};

__device__ __forceinline__ float ld_static(const AppendDev& a, int h, int g) {
  const int64_t off = (int64_t)h * a.st_sh + (int64_t)g * a.st_sg;
  return a.st_f32 ? reinterpret_cast<const float*>(a.st)[off]
                  : (float)reinterpret_cast<const half_t*>(a.st)[off];
}

// max over the lanes of one quantisation group (gs/2 consecutive lanes)
__device__ __forceinline__ float group_max(float v, int gs) {
  for (int o = 1; o < gs / 2; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// group_max for values >= +0 (absolute values: the order of the maxima cannot change a bit)
// with DPP instead of the LDS crossbar: xor 1 and 2 within the quad, then the half-row and
// row mirrors (lane i with 7 - i, 15 - i), which pair lanes of the two already reduced halves
__device__ __forceinline__ float group_absmax(float v, int gs) {
  v = fmaxf(v, dppf<0xB1>(v));                       // quad_perm [1, 0, 3, 2]
  if (gs >= 8) v = fmaxf(v, dppf<0x4E>(v));          // quad_perm [2, 3, 0, 1]
  if (gs >= 16) v = fmaxf(v, dppf<0x141>(v));        // row_half_mirror
  if (gs >= 32) v = fmaxf(v, dppf<0x140>(v));        // row_mirror
  if (gs >= 64) v = fmaxf(v, __shfl_xor(v, 16, 64));
  if (gs >= 128) v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}

// torch.quantile's linear interpolation between the order statistics a <= b with weight
// w = rank - floor(rank), as ATen's CPU lerp computes it: one fused multiply-add,
// fma(w, b - a, a) for w < 0.5, else fma(w - 1, b - a, b) (w - 1 is exact).  The unfused
// a + w (b - a) differs from it in the last bit for about 1 in 1000 inputs.
__device__ __forceinline__ float quantile_lerp(float a, float b, float w) {
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
__device__ void group_order_stats(float a0, float a1, int gs, int lo, int hi, int lane,
                                  float& vlo, float& vhi) {
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
__device__ float group_quantile(float a0, float a1, int gs, float q, int lane) {
  const float rank = q * (float)(gs - 1);
  const int lo = (int)floorf(rank), hi = (int)ceilf(rank);
  float vlo, vhi;
  group_order_stats(a0, a1, gs, lo, hi, lane, vlo, vhi);
  return quantile_lerp(vlo, vhi, rank - (float)lo);
}

// Scale of group g for a row, before the per-format final clamp.
//  dyn_abs: absmax of the group's fp16 values (as float)
//  stv: the static scale of the group (ld_static)
__device__ __forceinline__ float int4_scale(const AppendDev& a, float stv, float dyn_abs, float thr) {
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

// Calls f(bits) for the fp32 bit pattern of the dynamic scale fmax(absmax, 1e-5) / 7 of every
// (row, group) of the append (int4_cache.py:344-358), one wave per row, grid-stride.
template <class F>
__device__ __forceinline__ void for_each_dyn(const AppendDev& a, F f) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rows = a.B * a.H * a.S;
  for (int row = blockIdx.x * kAppendWaves + wave; row < rows; row += gridDim.x * kAppendWaves) {
    const int s_idx = row % a.S, bh = row / a.S, h = bh % a.H, b = bh / a.H;
    const half_t* xr = a.x + (int64_t)b * a.xsb + (int64_t)h * a.xsh + (int64_t)s_idx * a.xss;
    const half2v xv = *reinterpret_cast<const half2v*>(xr + 2 * lane);
    const float am = group_max(fmaxf(fabsf((float)xv.x), fabsf((float)xv.y)), a.gs);
    if ((2 * lane) % a.gs == 0) f(__float_as_uint(__fdiv_rn(fmaxf(am, 1e-5f), 7.0f)));
  }
}

// rank of torch.quantile's lower order statistic: lo = floor(fp32(q) * (n - 1)); hi = ceil
__device__ __forceinline__ void quantile_ranks(float q, int64_t n, int64_t& lo, int64_t& hi, float& w) {
  const float rank = q * (float)(n - 1);
  lo = (int64_t)floorf(rank);
  hi = (int64_t)ceilf(rank);
  w = rank - (float)lo;
}

__global__ void rescue_init_kernel(RescueScratch* s, float q, int64_t n) {
  for (int i = threadIdx.x; i < 256; i += blockDim.x) s->hist[i] = 0;
  if (threadIdx.x == 0) {
    int64_t lo, hi;
    float w;
    quantile_ranks(q, n, lo, hi, w);
    s->prefix = 0;
    s->rank = (uint32_t)lo;
    s->cnt_le = 0;
    s->min_gt = 0xFFFFFFFFu;
  }
}

// histogram of digit `pass` (bits [24 - 8 pass, 32 - 8 pass)) over the values whose higher
// digits equal the prefix found so far
__global__ __launch_bounds__(kAppendWaves * 64) void rescue_hist_kernel(AppendDev a, RescueScratch* s,
                                                                         int pass) {
  __shared__ uint32_t h[256];
  for (int i = threadIdx.x; i < 256; i += blockDim.x) h[i] = 0;
  __syncthreads();
  const uint32_t pre = s->prefix;
  const int sh = 24 - 8 * pass;
  for_each_dyn(a, [&](uint32_t bits) {
    if (pass == 0 || (bits >> (sh + 8)) == (pre >> (sh + 8))) atomicAdd(&h[(bits >> sh) & 255u], 1u);
  });
  __syncthreads();
  for (int i = threadIdx.x; i < 256; i += blockDim.x)
    if (h[i]) atomicAdd(&s->hist[i], h[i]);
}

// picks the digit whose bucket holds the remaining rank, and clears the histogram
__global__ void rescue_select_kernel(RescueScratch* s, int pass) {
  __shared__ uint32_t digit, before;
  if (threadIdx.x == 0) {
    uint32_t cum = 0, d = 255, r = s->rank;
    for (uint32_t i = 0; i < 256; ++i) {
      const uint32_t c = s->hist[i];
      if (r < cum + c) {
        d = i;
        break;
      }
      cum += c;
    }
    digit = d;
    before = cum;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 256; i += blockDim.x) s->hist[i] = 0;
  if (threadIdx.x == 0) {
    s->prefix |= digit << (24 - 8 * pass);
    s->rank -= before;
  }
}

// number of values <= sorted[lo] and the least value above it
__global__ __launch_bounds__(kAppendWaves * 64) void rescue_count_kernel(AppendDev a, RescueScratch* s) {
  __shared__ uint32_t cnt, mn;
  if (threadIdx.x == 0) {
    cnt = 0;
    mn = 0xFFFFFFFFu;
  }
  __syncthreads();
  const uint32_t lo_bits = s->prefix;
  for_each_dyn(a, [&](uint32_t bits) {
    if (bits <= lo_bits) atomicAdd(&cnt, 1u);
    else atomicMin(&mn, bits);
  });
  __syncthreads();
  if (threadIdx.x == 0) {
    if (cnt) atomicAdd(&s->cnt_le, cnt);
    if (mn != 0xFFFFFFFFu) atomicMin(&s->min_gt, mn);
  }
}

// torch.quantile's interpolation of sorted[lo] and sorted[hi] (sorted_quantile's arithmetic)
__global__ void rescue_thr_kernel(RescueScratch* s, float q, int64_t n) {
  int64_t lo, hi;
  float w;
  quantile_ranks(q, n, lo, hi, w);
  const float va = __uint_as_float(s->prefix);
  const float vb = (hi < (int64_t)s->cnt_le) ? va : __uint_as_float(s->min_gt);
  s->thr = quantile_lerp(va, vb, w);
}

// the lane's two input values of append row `row` (row = (b * H + h) * S + s)
__device__ __forceinline__ const half_t* row_x(const AppendDev& a, int row) {
  const int s_idx = row % a.S, bh = row / a.S, h = bh % a.H, b = bh / a.H;
  return a.x + (int64_t)b * a.xsb + (int64_t)h * a.xsh + (int64_t)s_idx * a.xss;
}
__device__ __forceinline__ half2v load_x(const AppendDev& a, int row, int lane) {
  return *reinterpret_cast<const half2v*>(row_x(a, row) + 2 * lane);
}

// the static scale of the lane's group in append row `row` (0 without a static table)
__device__ __forceinline__ float row_static(const AppendDev& a, int row, int lane) {
  if (a.st == nullptr || a.fmt == KVQ_FMT_INT4_ASYM || a.fmt == KVQ_FMT_INT4_KIVI ||
      a.fmt == KVQ_FMT_INT8_KIVI)
    return 0.f;
  return ld_static(a, (row / a.S) % a.H, (2 * lane) / a.gs);
}

// Quantizes append row `row` whose lane values xv (and static scale stv, row_static) were
// loaded by the caller.
__device__ __forceinline__ void quant_row_x(const AppendDev& a, int row, int lane, float thr,
                                            half2v xv, float stv) {
  const int s_idx = row % a.S;
  const int bh = row / a.S;
  const int h = bh % a.H, b = bh / a.H;
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
                   (a.fmt == KVQ_FMT_INT8_SYM || a.fmt == KVQ_FMT_INT4_SYM);
  const float am = pct ? group_quantile(fabsf(x0), fabsf(x1), a.gs, a.dq, lane)
                       : group_max(fmaxf(fabsf(x0), fabsf(x1)), a.gs);
  uint8_t* crow = a.codes + (int64_t)b * a.csb + (int64_t)h * a.csh + t * a.cst;
  int clipped = 0;

  if (a.fmt == KVQ_FMT_INT8_SYM) {
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
  } else if (a.fmt == KVQ_FMT_INT4_SYM) {
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
  } else if (a.fmt == KVQ_FMT_INT4_KIVI || a.fmt == KVQ_FMT_INT8_KIVI) {
    // asymmetric_quant.py:24-141 with qmin, qmax = -8, 7 (4 bits) or -128, 127 (8 bits)
    const bool b8 = a.fmt == KVQ_FMT_INT8_KIVI;
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
  for (int o = 32; o > 0; o >>= 1) clipped += __shfl_xor(clipped, o, 64);
  if (lane == 0 && a.status && clipped) atomicAdd(&a.status[1], clipped);
}

__device__ __forceinline__ void quant_row(const AppendDev& a, int row, int lane, float thr) {
  quant_row_x(a, row, lane, thr, load_x(a, row, lane), row_static(a, row, lane));
}

// Bitonic sort of n_pad (power of two) floats in LDS, ascending.
__device__ void lds_bitonic_sort(float* v, int n_pad) {
  for (int k = 2; k <= n_pad; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n_pad; i += blockDim.x) {
        const int p = i ^ j;
        if (p > i) {
          const bool up = (i & k) == 0;
          const float x = v[i], y = v[p];
          if ((x > y) == up) {
            v[i] = y;
            v[p] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

// torch.quantile of the n floats v[0, n) (LDS, one work-group) when the ranks lo <= hi lie
// near the top (n - 1 - lo < kTopWalk): the distinct values are walked down from the maximum
// (value m with multiplicity c holds the ranks [n - above - c, n - above)); w = rank - lo.
// Every thread returns the result.
__device__ float lds_top_quantile(const float* v, int n, int lo, int hi, float w) {
  __shared__ float red_m[kAppendWaves];
  __shared__ int red_c[kAppendWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float t = __builtin_inff(), vlo = 0.f, vhi = 0.f;
  int above = 0;
  for (int it = 0; it < kTopWalk && above <= n - 1 - lo; ++it) {
    float m = -1.0f;  // the scales are positive
    for (int i = threadIdx.x; i < n; i += blockDim.x)
      if (v[i] < t) m = fmaxf(m, v[i]);
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (lane == 0) red_m[wave] = m;
    __syncthreads();
    m = red_m[0];
    for (int i = 1; i < kAppendWaves; ++i) m = fmaxf(m, red_m[i]);
    int c = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) c += v[i] == m;
    for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
    if (lane == 0) red_c[wave] = c;
    __syncthreads();
    c = 0;
    for (int i = 0; i < kAppendWaves; ++i) c += red_c[i];
    const int r0 = n - above - c, r1 = n - above;
    if (lo >= r0 && lo < r1) vlo = m;
    if (hi >= r0 && hi < r1) vhi = m;
    above += c;
    t = m;
    __syncthreads();  // red_m / red_c are rewritten by the next step
  }
  return quantile_lerp(vlo, vhi, w);
}

// lds_top_quantile by one wave alone, without barriers: lane l holds the scales v[l + 64 r]
// (r < R, n <= 64 R) in registers, and the maximum and multiplicity of each step are DPP
// wave reductions (the count summed as an exact small float).  Every lane returns the
// result.
template <int R>
__device__ float wave_top_quantile(const float* v, int n, int lo, int hi, float w, int lane) {
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
    float cf = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) cf += x[r] == m ? 1.f : 0.f;
    const int c = (int)wave_sum64(cf);
    const int r0 = n - above - c, r1 = n - above;
    if (lo >= r0 && lo < r1) vlo = m;
    if (hi >= r0 && hi < r1) vhi = m;
    above += c;
    t = m;
  }
  return quantile_lerp(vlo, vhi, w);
}

// torch.quantile(x, q) with linear interpolation, float32 arithmetic:
// rank = fp32(q) * (n - 1); lo = floor(rank); hi = ceil(rank); w = rank - lo;
// quantile_lerp(v[lo], v[hi], w)
__device__ float sorted_quantile(const float* v, int n, float q) {
  const float rank = q * (float)(n - 1);
  const int lo = (int)floorf(rank), hi = (int)ceilf(rank);
  return quantile_lerp(v[lo], v[hi], rank - (float)lo);
}

// rescue: 0 none (or the threshold in a.thr_ptr), 1 one work-group finds the threshold and
// quantizes every row, 2 every work-group finds it (rank counting) and quantizes its own rows
__device__ __forceinline__ void append_side(const AppendDev& a, int rescue) {
  if (!a.valid) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rows = a.B * a.H * a.S;
  float thr = a.thr_ptr ? *a.thr_ptr : 0.f;
  __shared__ float dyn[kRescueMax];
  const bool resc_side = a.fmt == KVQ_FMT_INT4_SYM && a.st != nullptr && a.rq > 0.f && !a.rescue_all;
  if (rescue == 2 && resc_side) {
    // Global threshold over every (row, group) dynamic scale of this append
    // (int4_cache.py:384-389), found by each work-group over all rows (n <= kRescueRank):
    // near the top (the reference's ratio 0.01) every wave walks down from the maximum on
    // its own (wave_top_quantile); elsewhere the scale at ascending position p of the
    // stable order is the one with p smaller values or equal values at lower indices, which
    // gives sorted[lo] and sorted[hi] without sorting.  Wave w then quantizes row
    // 4 blockIdx.x + w, which it loads first (the rows are visited rotated by 4 blockIdx.x).
    __shared__ float ord[2];
    const int G = 128 / a.gs;
    const int n = rows * G;
    const int n4 = (n + 3) & ~3;
    const int own = blockIdx.x * kAppendWaves + wave;
    const int rot = (int)(((int64_t)blockIdx.x * kAppendWaves) % rows);
    for (int i = n + threadIdx.x; i < n4; i += blockDim.x) dyn[i] = __builtin_inff();
    if (threadIdx.x < 2) ord[threadIdx.x] = 0.f;
    const float own_st = own < rows ? row_static(a, own, lane) : 0.f;
    half2v own_x = half2v{(half_t)0.f, (half_t)0.f};
    for (int r0 = wave; r0 < rows; r0 += kRowBatch * kAppendWaves) {
      half2v xb[kRowBatch];
#pragma unroll
      for (int u = 0; u < kRowBatch; ++u) {
        const int r = r0 + u * kAppendWaves;
        if (r < rows) xb[u] = load_x(a, (r + rot) % rows, lane);
      }
      if (r0 == wave) own_x = xb[0];  // row (wave + rot) % rows == own when own < rows
#pragma unroll
      for (int u = 0; u < kRowBatch; ++u) {
        const int r = r0 + u * kAppendWaves;
        if (r >= rows) break;
        const int row = (r + rot) % rows;
        const float am = group_absmax(fmaxf(fabsf((float)xb[u].x), fabsf((float)xb[u].y)), a.gs);
        if ((2 * lane) % a.gs == 0) dyn[row * G + (2 * lane) / a.gs] = __fdiv_rn(fmaxf(am, 1e-5f), 7.0f);
      }
    }
    __syncthreads();
    const float rank = a.rq * (float)(n - 1);
    const int lo = (int)floorf(rank), hi = (int)ceilf(rank);
    const float wgt = rank - (float)lo;
    if (n - 1 - lo < kTopWalk) {  // uniform over the work-group
      thr = n <= 64    ? wave_top_quantile<1>(dyn, n, lo, hi, wgt, lane)
            : n <= 128 ? wave_top_quantile<2>(dyn, n, lo, hi, wgt, lane)
            : n <= 256 ? wave_top_quantile<4>(dyn, n, lo, hi, wgt, lane)
            : n <= 512 ? wave_top_quantile<8>(dyn, n, lo, hi, wgt, lane)
                       : wave_top_quantile<kRescueRank / 64>(dyn, n, lo, hi, wgt, lane);
    } else {
      const float4* d4 = reinterpret_cast<const float4*>(dyn);
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float vi = dyn[i];
        int c = 0;
        for (int j = 0; j < n4; j += 4) {
          const float4 w = d4[j >> 2];  // padding (+inf) is neither smaller nor equal at a lower index
          c += (w.x < vi) | ((w.x == vi) & (j < i));
          c += (w.y < vi) | ((w.y == vi) & (j + 1 < i));
          c += (w.z < vi) | ((w.z == vi) & (j + 2 < i));
          c += (w.w < vi) | ((w.w == vi) & (j + 3 < i));
        }
        if (c == lo) ord[0] = vi;
        if (c == hi) ord[1] = vi;
      }
      __syncthreads();
      thr = quantile_lerp(ord[0], ord[1], wgt);
    }
    if (own < rows) quant_row_x(a, own, lane, thr, own_x, own_st);
    return;
  }
  if (rescue == 1 && resc_side) {
    // Global threshold over every (row, group) dynamic scale of this append
    // (int4_cache.py:384-389).  Single work-group: grid.x == 1 on this path.  Each wave
    // handles rows wave, wave + 8, ..: kRowBatch of them loaded at once, so one memory
    // latency covers the batch; the values stay in registers for the quantization.
    __shared__ float thr_sh;
    const int G = 128 / a.gs;
    const int n = rows * G;
    int n_pad = 1;
    while (n_pad < n) n_pad <<= 1;
    const float rank = a.rq * (float)(n - 1);
    const int lo = (int)floorf(rank), hi = (int)ceilf(rank);
    const bool top = n - 1 - lo < kTopWalk;
    if (!top)
      for (int i = threadIdx.x; i < n_pad; i += blockDim.x) dyn[i] = __builtin_inff();
    __syncthreads();
    half2v xb[kRowBatch];
    float sb[kRowBatch];  // the rows' static scales (loaded with them)
    const bool cached = rows <= kRowBatch * kAppendWaves;  // every row of the wave in xb
    for (int r0 = wave; r0 < rows; r0 += kRowBatch * kAppendWaves) {
#pragma unroll
      for (int u = 0; u < kRowBatch; ++u) {
        const int row = r0 + u * kAppendWaves;
        if (row < rows) {
          xb[u] = load_x(a, row, lane);
          sb[u] = row_static(a, row, lane);
        }
      }
#pragma unroll
      for (int u = 0; u < kRowBatch; ++u) {
        const int row = r0 + u * kAppendWaves;
        if (row >= rows) break;
        const float am = group_max(fmaxf(fabsf((float)xb[u].x), fabsf((float)xb[u].y)), a.gs);
        if ((2 * lane) % a.gs == 0) dyn[row * G + (2 * lane) / a.gs] = __fdiv_rn(fmaxf(am, 1e-5f), 7.0f);
      }
    }
    __syncthreads();
    if (top) {
      const float t = lds_top_quantile(dyn, n, lo, hi, rank - (float)lo);
      if (threadIdx.x == 0) thr_sh = t;
    } else {
      lds_bitonic_sort(dyn, n_pad);
      if (threadIdx.x == 0) thr_sh = sorted_quantile(dyn, n, a.rq);
    }
    __syncthreads();
    thr = thr_sh;
    for (int r0 = wave; r0 < rows; r0 += kRowBatch * kAppendWaves) {
      if (!cached) {
#pragma unroll
        for (int u = 0; u < kRowBatch; ++u) {
          const int row = r0 + u * kAppendWaves;
          if (row < rows) {
            xb[u] = load_x(a, row, lane);
            sb[u] = row_static(a, row, lane);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kRowBatch; ++u) {
        const int row = r0 + u * kAppendWaves;
        if (row < rows) quant_row_x(a, row, lane, thr, xb[u], sb[u]);
      }
    }
    return;
  }
  for (int row = blockIdx.x * kAppendWaves + wave; row < rows; row += gridDim.x * kAppendWaves)
    quant_row(a, row, lane, thr);
}

// grid.y selects the side; each branch reads its own kernel arguments directly (selecting
// between the two structs field by field costs scalar registers)
__global__ __launch_bounds__(kAppendWaves * 64) void append_kernel(AppendDev k, AppendDev v,
                                                                    int rescue) {
  if (blockIdx.y == 0)
    append_side(k, rescue);
  else
    append_side(v, rescue);
}

static int fill_dev(const kvq_append_params* p, AppendDev& d, const char* name) {
  d = AppendDev{};
  if (!p) return KVQ_OK;
  const std::string n(name);
  if (p->format != KVQ_FMT_INT8_SYM && p->format != KVQ_FMT_INT4_SYM &&
      p->format != KVQ_FMT_INT4_ASYM && p->format != KVQ_FMT_INT4_KIVI &&
      p->format != KVQ_FMT_INT8_KIVI)
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

static bool needs_rescue(const kvq_append_params* p) {
  return p && p->format == KVQ_FMT_INT4_SYM && p->static_scale && p->rescue_quantile > 0.f &&
         !p->rescue_all && p->batch * p->heads * p->seq_new > 0;
}

// (row, group) scales the group rescue of p takes its quantile over
static int64_t rescue_n(const kvq_append_params* p) {
  return (int64_t)p->batch * p->heads * p->seq_new * (128 / p->group_size);
}

// the threshold of p's group rescue over more than kRescueMax scales, into its scratch
static int rescue_large(const kvq_append_params* p, AppendDev& d, const char* name, hipStream_t st) {
  const std::string n(name);
  if (!p->scratch || p->scratch_bytes < (int64_t)sizeof(RescueScratch) || ((uintptr_t)p->scratch % 16))
    return fail(KVQ_ERR_INVALID, n + ": outlier rescue over more than 4096 (row, group) scales needs "
                                     "a 16-byte aligned scratch of kvq_append_scratch_bytes() bytes");
  RescueScratch* s = reinterpret_cast<RescueScratch*>(p->scratch);
  const int64_t cnt = rescue_n(p);
  if (cnt >= ((int64_t)1 << 31)) return fail(KVQ_ERR_UNSUPPORTED, n + ": too many (row, group) scales");
  const int64_t rows = (int64_t)p->batch * p->heads * p->seq_new;
  int64_t gx = (rows + kAppendWaves - 1) / kAppendWaves;
  if (gx > 2048) gx = 2048;
  const dim3 grid((unsigned)gx), block(kAppendWaves * 64);
  hipLaunchKernelGGL(rescue_init_kernel, dim3(1), dim3(256), 0, st, s, p->rescue_quantile, cnt);
  for (int pass = 0; pass < 4; ++pass) {
    hipLaunchKernelGGL(rescue_hist_kernel, grid, block, 0, st, d, s, pass);
    hipLaunchKernelGGL(rescue_select_kernel, dim3(1), dim3(256), 0, st, s, pass);
  }
  hipLaunchKernelGGL(rescue_count_kernel, grid, block, 0, st, d, s);
  hipLaunchKernelGGL(rescue_thr_kernel, dim3(1), dim3(1), 0, st, s, p->rescue_quantile, cnt);
  d.thr_ptr = &s->thr;
  return KVQ_OK;
}

}  // namespace kvq

using namespace kvq;

extern "C" int kvq_quant_append(const kvq_append_params* k, const kvq_append_params* v,
                                kvq_stream_t stream) {
  AppendDev dk, dv;
  int rc = fill_dev(k, dk, "k");
  if (rc) return rc;
  rc = fill_dev(v, dv, "v");
  if (rc) return rc;
  if (!dk.valid && !dv.valid) return KVQ_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // the group rescue takes its threshold from one work-group's LDS sort when every side
  // that needs one has at most kRescueMax scales, else from the radix select (scratch)
  const bool large = (needs_rescue(k) && rescue_n(k) > kRescueMax) ||
                     (needs_rescue(v) && rescue_n(v) > kRescueMax);
  if (large) {
    if (needs_rescue(k) && (rc = rescue_large(k, dk, "k", s))) return rc;
    if (needs_rescue(v) && (rc = rescue_large(v, dv, "v", s))) return rc;
  }
  // decode-sized rescues (at most kRescueRank scales per side): every work-group finds the
  // threshold; else one work-group does
  int rescue = 0;
  if (!large && (needs_rescue(k) || needs_rescue(v))) {
    const int64_t nk = needs_rescue(k) ? rescue_n(k) : 0, nv = needs_rescue(v) ? rescue_n(v) : 0;
    rescue = (nk > nv ? nk : nv) <= kRescueRank ? 2 : 1;
  }
  int64_t rows = 0;
  if (dk.valid) rows = (int64_t)dk.B * dk.H * dk.S;
  if (dv.valid) rows = rows > (int64_t)dv.B * dv.H * dv.S ? rows : (int64_t)dv.B * dv.H * dv.S;
  int64_t gx = rescue == 1 ? 1 : (rows + kAppendWaves - 1) / kAppendWaves;
  if (gx > 65535) gx = 65535;
  hipLaunchKernelGGL(append_kernel, dim3((unsigned)gx, 2), dim3(kAppendWaves * 64), 0, s, dk, dv,
                     rescue);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(KVQ_ERR_LAUNCH, std::string("launch: ") + hipGetErrorString(e));
  return KVQ_OK;
}

extern "C" int64_t kvq_append_scratch_bytes(const kvq_append_params* p) {
  return (needs_rescue(p) && rescue_n(p) > kRescueMax) ? (int64_t)sizeof(RescueScratch) : 0;
}

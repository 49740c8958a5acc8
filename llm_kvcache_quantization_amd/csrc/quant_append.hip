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
#include "append_row.h"
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

struct RescueScratch {
  uint32_t hist[256];
  uint32_t prefix;  // bits of sorted[lo] fixed so far (all 32 after the last pass)
  uint32_t rank;    // rank of sorted[lo] among the values that match prefix
  uint32_t cnt_le;  // number of values <= sorted[lo]
  uint32_t min_gt;  // least bit pattern above sorted[lo]
  float thr;
  uint32_t pad[3];
};

// Calls f(bits) for the fp32 bit pattern of the dynamic scale fmax(absmax, 1e-5) / 7 of every
// (row, group) of the append (int4_cache.py:344-358), one wave per row, grid-stride.
template <class F>
__device__ __forceinline__ void for_each_dyn(const AppendDev& a, F f) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
  // the wave index is uniform: the row index arithmetic (divisions by H and S) runs on the
  // scalar unit, not as vector integer division in every lane
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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

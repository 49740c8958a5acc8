// Definitions shared by the split-K decode kernels (decode_attn.hip, decode_tiled.h).
#pragma once
#include "append_row.h"
#include "kvq_common.h"
#include "kvq.h"

#include <string>

namespace kvq {

constexpr int kWaves = 4;       // waves per work-group of the row-layout split-K kernel
constexpr int kTiledWaves = 8;  // waves per work-group of the tiled kernel (two per SIMD)
constexpr int kTile = 32;   // tokens per wave iteration (two 16-token MFMA row blocks)
constexpr int kD = 128;
constexpr float kTau = 8.0f;  // lazy-rescale headroom in log2 units
constexpr int kMaxChunks = 2048;
// The workspace starts with the counter area: one slot of kCtrSlotWords u32 per (b, kv
// head), one 128-byte line each (no two counters share a line).  Word 0 counts the
// work-groups that have stored their partial (the tiled kernel's single-launch merge); it
// is zero between calls.  The chunk partials follow it, so the counters stay in place
// when a reused workspace serves calls with other split counts.
constexpr int kCtrSlotWords = 32;
constexpr int kMinChunk = 256;

struct KvDev {
  const uint8_t* codes;
  int64_t sb, sh, st;
  const void* scale;
  int64_t ssb, ssh, sst, ssg;
  int scale_f32;
  int n_out;
  const half_t* zp;
  const int32_t* oidx;
  const half_t* oval;
  int64_t osb, osh, ost;
  int layout;  // KVQ_LAYOUT_*
};

// The new token of a fused quantize-on-append (kvq_append_decode_attn): fp16 K / V rows
// [B, Hkv, 128] (strides in elements), the slot they go to, and the optional status words
// (int32 [2] each: NaN/Inf flag, clamped-element count).  kx == nullptr: no append.
struct FusedAppend {
  const half_t* kx;
  int64_t ksb, ksh;
  const half_t* vx;
  int64_t vsb, vsh;
  int64_t wpos;
  int32_t* kstatus;
  int32_t* vstatus;
  // INT8 sides: the append's static scale tables [H, G] (elements; fp32 when *_f32)
  const void* kst;
  const void* vst;
  int kst_f32, vst_f32;
  int64_t kst_sh, kst_sg, vst_sh, vst_sg;
};

struct DecodeArgs {
  const half_t* q;
  int64_t q_sb, q_sh;
  const half_t* inv_tau;
  KvDev k, v;
  const int32_t* ctx;  // context length per batch row, or null: every row has ctx_uniform
  int ctx_uniform;
  int B, Hq, Hkv, n_rep, gs;
  int vgs;          // the group size of per-token INT8 / INT4 V scales (gs unless set apart)
  int64_t cap;
  float sm_log2e;
  int chunk, n_chunks;
  int strided;      // work-group c takes 32-token tiles c*nw + w + i*n_chunks*nw (wave w)
                    // instead of the contiguous tokens [c*chunk, (c+1)*chunk)
  int nw;           // waves per work-group of the split-K kernel
  float* part_acc;  // [B, Hq, n_chunks, 128]
  float2* part_ml;  // [B, Hq, n_chunks]
  uint32_t* counters;  // [B, Hkv] slots of kCtrSlotWords u32, zero between calls (below)
  int fused;           // 1: the split-K kernel merges the partials itself (combine_unit)
  int share;           // tiled kernel, 1-D grid per kv head (x): rows of equal context
                       // length take u_chunks work-groups each (the uniform split); a ragged
                       // batch shares share_c work-groups out by context length.  n_chunks
                       // is then the partial pitch per row
  int u_chunks, share_c;
  half_t* out;
  int64_t o_sb, o_sh;
  FusedAppend app;
  // fp16 residual window: res_n tokens per (b, kv head) at res_k / res_v + b * rsb + h * rsh
  // (elements, dense 128-element token rows), merged by the merging work-group
  const half_t* res_k;
  const half_t* res_v;
  int64_t rsb, rsh;
  int res_n;
  // The fused append of the row formats (per-token INT8 / INT4 scales, the KIVI family, fp16
  // sides): the writer wave quantises its (b, kv head) row of each side with the append
  // kernel's quant_row_x (app.kx != nullptr marks the call; app.wpos is the slot)
  AppendDev ark, arv;
};

// context length of batch row b, clamped to [0, capacity]
// b uniform: the length is read through the scalar cache (a constant-address load), whose
// wait does not include the vector loads issued before it (a vector load here would make
// the wave wait for the q-side loads before it requests its first cache tiles).  Nothing
// in a launch writes the lengths.
__device__ __forceinline__ int64_t row_context(const DecodeArgs& a, int b) {
  using cint = const __attribute__((address_space(4))) int32_t;
  const int64_t c = a.ctx != nullptr ? (int64_t)((cint*)a.ctx)[b] : (int64_t)a.ctx_uniform;
  return c < 0 ? 0 : (c > a.cap ? a.cap : c);
}

__device__ __forceinline__ uint32_t splat_h2(half_t s) { return as_u32(half2v{s, s}); }
__device__ __forceinline__ uint32_t pair_h2(half_t lo, half_t hi) { return as_u32(half2v{lo, hi}); }
// q' = fp16(q * inv_tau): fp16 x fp16 product rounded once, as torch's Half mul
__device__ __forceinline__ half_t qscale(half_t x, half_t tau, bool has_tau) {
  return has_tau ? (half_t)((float)x * (float)tau) : x;
}
// two fp32 -> packed fp16, rounding toward zero (v_cvt_pkrtz_f16_f32)
__device__ __forceinline__ half2v pk_rtz(float a, float b) {
  return __builtin_bit_cast(half2v, __builtin_amdgcn_cvt_pkrtz(a, b));
}
// (x - off) * s on a half2: exact code recovery, then one fp16 rounding of the product
__device__ __forceinline__ uint32_t deq_pair(uint32_t x, half_t off, uint32_t s2) {
  const half2v o = {off, off};
  return as_u32((as_h2(x) - o) * as_h2(s2));
}
// b * sb + h * sh for b, h >= 0 (a (b, head) slab's offset): zero-extended 32 x 64-bit
// products, three scalar multiplies each where the sign-extended form takes four and a shift
// (the same bits for b, h >= 0, whatever the strides' signs)
__device__ __forceinline__ int64_t slab_off(int64_t sb, int64_t sh, int b, int h) {
  return (int64_t)((uint64_t)(uint32_t)b * (uint64_t)sb + (uint64_t)(uint32_t)h * (uint64_t)sh);
}
__device__ __forceinline__ const half_t* q_row(const DecodeArgs& a, int b, int hq) {
  return a.q + slab_off(a.q_sb, a.q_sh, b, hq);
}
// q'[32 lg + i] for i < 32 (the lane group's quantisation group) with four 16-byte
// loads issued together; q' = fp16(q * inv_tau) when inv_tau is given
__device__ __forceinline__ void load_q_group(const half_t* qr, int lg, half_t tau, bool has_tau,
                                             half_t out[32]) {
  const u32x4* p = reinterpret_cast<const u32x4*>(qr + 32 * lg);
  u32x4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = p[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const half2v h = as_h2(w[k]);
      out[8 * i + 2 * k] = qscale(h.x, tau, has_tau);
      out[8 * i + 2 * k + 1] = qscale(h.y, tau, has_tau);
    }
  }
}

// Online-softmax update of one 32-token tile.  x0 / x1 are the fp32 logits of tokens
// 4 lg + r and 16 + 4 lg + r (r < 4) for head lane % 16, already masked to -inf where
// invalid.  The running max m is raised only when a tile's max exceeds it by more than
// kTau (decided wave-wide with a ballot), in which case l and acc are rescaled.
// The fp32 probabilities p are returned as the PV B operands hi = fp16(p) (rounded toward
// zero) and lo = fp16(p - hi) (p - hi is exact in fp32), in k-slot order [4lg, 4lg+1,
// 4lg+2, 4lg+3, 16+4lg, .., 16+4lg+3]; l accumulates hi + lo.  The PV MFMAs multiply the
// V operand by both, so each weight is carried to about 2^-21 of itself: one fp16 weight
// alone perturbs the softmax weights by up to 2^-10, which for large V entries (|v - out|
// of 100 and more) moves an output by more than 2e-3.
// ex: optional two more running sums of the format (rescaled with l and acc)
__device__ __forceinline__ void split_pair(float a, float b, uint32_t& hi, uint32_t& lo) {
  const half2v h = pk_rtz(a, b);
  hi = as_u32(h);
  lo = as_u32(pk_rtz(a - (float)h.x, b - (float)h.y));
}

__device__ __forceinline__ void softmax_tile(float4v x0, float4v x1, float sm, float& m, float& l,
                                             float4v acc[8], half8v& ph, half8v& pl,
                                             float* ex = nullptr) {
  const float lmax = max8f(x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]) * sm;
  if (__ballot(lmax > m + kTau)) {
    // raise the running max of every head to its current wave-wide maximum
    const float mn = fmaxf(m, wave_max_xor_groups(lmax));
    const float alpha = fast_exp2(m - mn);
    m = mn;
    l *= alpha;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= alpha;
    if (ex) {
      ex[0] *= alpha;
      ex[1] *= alpha;
    }
  }
  const float nm = -m;
  uint32_t h[4], o[4];
  split_pair(fast_exp2(fmaf(x0[0], sm, nm)), fast_exp2(fmaf(x0[1], sm, nm)), h[0], o[0]);
  split_pair(fast_exp2(fmaf(x0[2], sm, nm)), fast_exp2(fmaf(x0[3], sm, nm)), h[1], o[1]);
  split_pair(fast_exp2(fmaf(x1[0], sm, nm)), fast_exp2(fmaf(x1[1], sm, nm)), h[2], o[2]);
  split_pair(fast_exp2(fmaf(x1[2], sm, nm)), fast_exp2(fmaf(x1[3], sm, nm)), h[3], o[3]);
  const half2v ones = {(half_t)1.0f, (half_t)1.0f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    l = __builtin_amdgcn_fdot2(as_h2(h[i]), ones, l, false);
    l = __builtin_amdgcn_fdot2(as_h2(o[i]), ones, l, false);
  }
  ph = pack8(h[0], h[1], h[2], h[3]);
  pl = pack8(o[0], o[1], o[2], o[3]);
}

// DPP row_ror:8 within each row of 16 lanes (lane c reads lane (c + 8) % 16), written only
// to the lanes of bank_mask (bank = 4 lanes; 0xC = lanes 8..15, 0x3 = lanes 0..7 of each
// row); the other lanes keep `old`.
template <int BANKS>
__device__ __forceinline__ uint32_t dpp_ror8(uint32_t old, uint32_t src) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)src, 0x128, 0xF, BANKS, false);
}
template <int BANKS>
__device__ __forceinline__ float dpp_ror8f(float old, float src) {
  return __builtin_bit_cast(float, dpp_ror8<BANKS>(__builtin_bit_cast(uint32_t, old),
                                                   __builtin_bit_cast(uint32_t, src)));
}

// softmax_tile for at most 8 heads (n_rep <= 8): head h's logits of row block 1 are moved
// from lane h into the padding lane h + 8, so each lane exponentiates 4 values instead of
// 8.  m is kept equal in lanes h and h + 8; l holds the block-0 part of head h's sum in
// lane h and the block-1 part in lane h + 8 (merge_and_store adds them).  The returned PV
// operands are valid in lanes h < 8; lanes 8..15 carry finite values of padding columns.
__device__ __forceinline__ void softmax_tile8(float4v x0, float4v x1, float sm, float& m,
                                              float& l, float4v acc[8], half8v& ph, half8v& pl,
                                              float* ex = nullptr) {
  float y[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) y[r] = dpp_ror8f<0xC>(x0[r], x1[r]);
  const float lmax = max3f(max3f(y[0], y[1], y[2]), y[3], y[3]) * sm;
  if (__ballot(lmax > m + kTau)) {
    const float hm = fmaxf(lmax, dpp_ror8f<0xF>(lmax, lmax));  // both halves of the head
    const float mn = fmaxf(m, wave_max_xor_groups(hm));
    const float alpha = fast_exp2(m - mn);
    m = mn;
    l *= alpha;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= alpha;
    if (ex) {
      ex[0] *= alpha;
      ex[1] *= alpha;
    }
  }
  const float nm = -m;
  uint32_t a0, a1, b0, b1;
  split_pair(fast_exp2(fmaf(y[0], sm, nm)), fast_exp2(fmaf(y[1], sm, nm)), a0, b0);
  split_pair(fast_exp2(fmaf(y[2], sm, nm)), fast_exp2(fmaf(y[3], sm, nm)), a1, b1);
  const half2v ones = {(half_t)1.0f, (half_t)1.0f};
  l = __builtin_amdgcn_fdot2(as_h2(a0), ones, l, false);
  l = __builtin_amdgcn_fdot2(as_h2(b0), ones, l, false);
  l = __builtin_amdgcn_fdot2(as_h2(a1), ones, l, false);
  l = __builtin_amdgcn_fdot2(as_h2(b1), ones, l, false);
  ph = pack8(a0, a1, dpp_ror8<0x3>(a0, a0), dpp_ror8<0x3>(a1, a1));
  pl = pack8(b0, b1, dpp_ror8<0x3>(b0, b0), dpp_ror8<0x3>(b1, b1));
}

// softmax_tile8 whose probabilities enter the PV MFMA as one operand: column h < 8 (lane h)
// carries the hi halves of head h's probabilities and the padding column h + 8 (lane h + 8)
// the lo halves, in the same k-slot order ([row block 0, row block 1] as softmax_tile8's
// ph), so one MFMA accumulates hi x V in column h and lo x V in column h + 8; fold_lo adds
// the two columns once after the loop.  Both lanes of a head hold its m, so a rescale
// applies to both columns.  Each lane passes its partner (lane ^ 8 within the 16-lane row)
// the half the partner lacks: lane h < 8 its block-0 lo, lane h + 8 its block-1 hi.
__device__ __forceinline__ void softmax_tile8c(float4v x0, float4v x1, float sm, float& m,
                                               float& l, float4v acc[8], half8v& pc, bool lo8) {
  float y[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) y[r] = dpp_ror8f<0xC>(x0[r], x1[r]);
  const float lmax = max3f(max3f(y[0], y[1], y[2]), y[3], y[3]) * sm;
  if (__ballot(lmax > m + kTau)) {
    const float hm = fmaxf(lmax, dpp_ror8f<0xF>(lmax, lmax));  // both halves of the head
    const float mn = fmaxf(m, wave_max_xor_groups(hm));
    const float alpha = fast_exp2(m - mn);
    m = mn;
    l *= alpha;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= alpha;
  }
  const float nm = -m;
  uint32_t a0, a1, b0, b1;
  split_pair(fast_exp2(fmaf(y[0], sm, nm)), fast_exp2(fmaf(y[1], sm, nm)), a0, b0);
  split_pair(fast_exp2(fmaf(y[2], sm, nm)), fast_exp2(fmaf(y[3], sm, nm)), a1, b1);
  const half2v ones = {(half_t)1.0f, (half_t)1.0f};
  l = __builtin_amdgcn_fdot2(as_h2(a0), ones, l, false);
  l = __builtin_amdgcn_fdot2(as_h2(b0), ones, l, false);
  l = __builtin_amdgcn_fdot2(as_h2(a1), ones, l, false);
  l = __builtin_amdgcn_fdot2(as_h2(b1), ones, l, false);
  const uint32_t s0 = lo8 ? b0 : a0, s1 = lo8 ? b1 : a1;
  const uint32_t r0 = dpp_ror8<0xF>(s0, s0), r1 = dpp_ror8<0xF>(s1, s1);
  pc = lo8 ? pack8(a0, a1, r0, r1) : pack8(r0, r1, b0, b1);
}

// after a loop of softmax_tile8c steps: column h (lanes h < 8) += column h + 8
__device__ __forceinline__ void fold_lo(float4v acc[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[i][r] += dpp_ror8f<0x3>(0.0f, acc[i][r]);
}

// masks logits of tokens >= t1 (tile starts at tt) to -inf
__device__ __forceinline__ void mask_tile(float4v& x0, float4v& x1, int tt, int t1, int lg) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (tt + 4 * lg + r >= t1) x0[r] = kNegInf;
    if (tt + 16 + 4 * lg + r >= t1) x1[r] = kNegInf;
  }
}

// Merges the (m, l, acc) states of the NW waves of a work-group through LDS and
// writes one partial (M, L, acc[128]) per valid head of this chunk.  acc[mb][r] of lane
// (head, lg) holds channel d = 32 lg + 8 r + mb.
template <int NW>
struct MergeLdsT {
  float m[NW][16];
  float l[NW][16];
  float acc[NW][16][kD + 1];
};
using MergeLds = MergeLdsT<kWaves>;

// partial stores; WT = write-through at device scope, so a work-group of the same launch
// on another XCD can read them once the store has completed (no L2 write-back needed)
template <bool WT>
__device__ __forceinline__ void store_partial(float* p, float v) {
  if constexpr (WT) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}

template <bool PACK8 = false, bool WT = false, int NW = kWaves>
__device__ __forceinline__ void merge_and_store(const DecodeArgs& a, MergeLdsT<NW>& sh, int wave,
                                                int col, int lg, float m, float l,
                                                const float4v acc[8], int b, int hkv, int chunk) {
  if constexpr (PACK8) l += dpp_ror8f<0xF>(l, l);  // add the block-1 part from lane h + 8
  l = wave_sum_xor_groups(l);
  if (lg == 0) {
    sh.m[wave][col] = m;
    sh.l[wave][col] = l;
  }
#pragma unroll
  for (int mb = 0; mb < 8; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) sh.acc[wave][col][32 * lg + 8 * r + mb] = acc[mb][r];
  __syncthreads();
  for (int idx = threadIdx.x; idx < a.n_rep * kD; idx += NW * 64) {
    const int h = idx >> 7, d = idx & (kD - 1);
    float M = sh.m[0][h];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, sh.m[w][h]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float e = fast_exp2(sh.m[w][h] - M);
      num = fmaf(e, sh.acc[w][h][d], num);
      den = fmaf(e, sh.l[w][h], den);
    }
    const int hq = hkv * a.n_rep + h;
    const int64_t pi = ((int64_t)b * a.Hq + hq) * a.n_chunks + chunk;
    store_partial<WT>(a.part_acc + pi * kD + d, num);
    if (d == 0) {
      store_partial<WT>(&a.part_ml[pi].x, M);
      store_partial<WT>(&a.part_ml[pi].y, den);
    }
  }
}

// number of work-groups (partials) with at least one token for a context of ctx tokens
__host__ __device__ __forceinline__ int valid_chunks(const DecodeArgs& a, int64_t ctx) {
  if (a.strided) {
    const int64_t tiles = (ctx + kTile - 1) / kTile;
    const int64_t n = (tiles + a.nw - 1) / a.nw;
    return (int)(n < a.n_chunks ? n : a.n_chunks);
  }
  return (int)((ctx + a.chunk - 1) / a.chunk);
}

// Merges the first nvalid chunk partials of (b, query head hq) for output channel d and
// writes the fp16 output, applying the asymmetric V epilogue when v_affine: the codes
// entered the PV MFMA as the fp16 subnormals 16 n 2^-24 (even channel) and n 2^-24 (odd),
// so out = s (acc / l * 2^20 or 2^24 - 8) + z.
// Every partial of a batch of kCombineBatch chunks is requested before any is used.
constexpr int kCombineBatch = 32;
// the tiled kernel merges its chunk partials in the same launch (its last work-group per
// (b, kv head) reads them) when there are at most this many chunks per (b, kv head)
constexpr int kUnitChunks = 64;

__device__ __forceinline__ void combine_one(const DecodeArgs& a, int b, int hq, int d, int nvalid,
                                            int v_affine) {
  half_t* o = a.out + (int64_t)b * a.o_sb + (int64_t)hq * a.o_sh;
  if (nvalid <= 0) {
    o[d] = (half_t)0.0f;
    return;
  }
  const int64_t base = ((int64_t)b * a.Hq + hq) * a.n_chunks;
  const float* pa = a.part_acc + base * kD + d;
  const float2* pm = a.part_ml + base;
  float M = kNegInf, num = 0.f, den = 0.f;
  for (int c0 = 0; c0 < nvalid; c0 += kCombineBatch) {
    const int n = nvalid - c0 < kCombineBatch ? nvalid - c0 : kCombineBatch;
    float av[kCombineBatch];
    float2 mv[kCombineBatch];
#pragma unroll
    for (int c = 0; c < kCombineBatch; ++c) {
      av[c] = 0.f;
      mv[c] = float2{kNegInf, 0.f};
      if (c < n) {
        av[c] = pa[(int64_t)(c0 + c) * kD];
        mv[c] = pm[c0 + c];
      }
    }
    float Mb = M;
#pragma unroll
    for (int c = 0; c < kCombineBatch; ++c)
      if (c < n) Mb = fmaxf(Mb, mv[c].x);
    const float r = fast_exp2(M - Mb);  // 0 on the first batch (M = -inf)
    num *= r;
    den *= r;
    M = Mb;
#pragma unroll
    for (int c = 0; c < kCombineBatch; ++c) {
      if (c < n) {
        const float e = fast_exp2(mv[c].x - M);
        num = fmaf(e, av[c], num);
        den = fmaf(e, mv[c].y, den);
      }
    }
  }
  float r = num / den;
  if (v_affine) {
    const int hkv = hq / a.n_rep, g = d >> 5;
    const float s = (float)reinterpret_cast<const half_t*>(a.v.scale)[hkv * a.v.ssh + g * a.v.ssg];
    const float z = (float)a.v.zp[hkv * a.v.ssh + g * a.v.ssg];
    r = fmaf(s, fmaf(r, (d & 1) ? 16777216.0f : 1048576.0f, -8.0f), z);
  }
  o[d] = (half_t)r;
}

// ---- host side (decode_attn.hip)
int fail(int code, const std::string& msg);

// ---- tiled kernels (decode_tiled.h; dispatch in decode_tiled.hip): 8-wave work-groups,
// interleaved 32-token tiles, single-launch merge.  Format families:
enum TiledFam {
  kTiledNone = 0,
  kTiledA4A4,   // INT4_ASYM K, INT4_ASYM V in the TILE32 layout
  kTiledA4A4o,  // the same with 4 fp16 outlier K channels
  kTiledI8A4,   // INT8_SYM K (static scale), INT4_ASYM V in the TILE32 layout
  kTiledI8I8,   // INT8_SYM K and V (static scales, groups of 32), token rows
  kTiledI8I8g,  // the same with any other group size (8, 16, 64, 128)
  kTiledT8,     // INT8_SYM K and V with per-token fp16 scales, groups of 32 .. 128, rows
  kTiledT8g16,  // the same with groups of 16
  kTiledT4,     // INT4_SYM K and V with per-token fp32 scales, groups of 32 .. 128, rows
  kTiledT4g16,  // the same with groups of 16
  kTiledT8Kv,   // INT8_SYM K with per-token fp16 scales, INT4_KIVI V (per-token fp32), rows
  kTiledT8Kvg16,  // the same with K groups of 16
  kTiledKivi,   // INT4_KIVI K (per-channel) and V (per-token), token rows
  // the KIVI family's other (K, V) pairs: 4 = INT4_KIVI, 8 = INT8_KIVI, F = FP16
  kTiledKv48, kTiledKv4F, kTiledKv84, kTiledKv88, kTiledKv8F, kTiledKvF4, kTiledKvF8, kTiledKvFF,
  kTiledT8F,    // INT8_SYM K with per-token fp16 scales, FP16 V
  kTiledT8Fg16,  // the same with K groups of 16
  // INT4 asymmetric K per token (INT4_KIVI with per-token parameters), with V INT4_KIVI,
  // INT8_SYM with per-token fp16 scales, or FP16 (the reference's MixedKVCache at K 4 bits)
  kTiledKtKv, kTiledKtT8, kTiledKtF,
  kTiledFT8,    // FP16 K, INT8_SYM V with per-token fp16 scales (MixedKVCache (16, 8))
  // kTiledT4 / kTiledT4g16 whose V scale rows are dense and 16-byte aligned: V tiles read with
  // 16-byte loads and gathered through LDS (VTokT<true, true>)
  kTiledT4s, kTiledT4g16s,
  // kTiledKivi / kTiledT8Kv / kTiledT8Kvg16 with 16-byte aligned V code rows: the V rows read
  // with 16-byte loads and gathered through LDS (VKiviRowTS)
  kTiledKivis, kTiledT8Kvs, kTiledT8Kvg16s,
};
// a tiled kernel and the formats of the fused row append built into it (-1: none)
struct TiledFn {
  const void* fn;        // the grid split's instantiation
  const void* fn_share;  // the shared split's (a.share)
  int kfmt, vfmt;
};
// the instantiations, one lookup per translation unit (fn nullptr: not one of its families)
TiledFn tiled_kernel_a4(int fam, bool pack8);
TiledFn tiled_kernel_tok(int fam, bool pack8);
TiledFn tiled_kernel_kv4(int fam, bool pack8);
TiledFn tiled_kernel_kv16(int fam, bool pack8);
TiledFn tiled_kernel_kt(int fam, bool pack8);
// kernel of family fam for n_rep query heads per kv head (fn nullptr if none)
TiledFn tiled_kernel(int fam, int n_rep);
hipError_t launch_tiled(const DecodeArgs& a, const TiledFn& k, dim3 grid, hipStream_t s);

}  // namespace kvq

// Split-K quantized decode attention for gfx950 (CDNA4).
//
// One work-group = 4 wavefronts = one (batch b, kv head, chunk of tokens).  All
// n_rep query heads that share the kv head are processed together (GQA): the
// heads are the N dimension (padded to 16) of v_mfma_f32_16x16x32_f16 and the
// tokens are M, so every code byte is read from HBM exactly once.
//
//   S^T[t, h]   = K[t, :] . q'[h, :]           A = dequantised K tile, B = q'^T
//   out^T[d, h] = sum_t V^T[d, t] * P^T[t, h]  A = dequantised V^T,    B = P^T
//
// The D layout of the first MFMA (lane = (h, 4 tokens)) is exactly the B layout
// the second one needs, so the softmax probabilities never leave registers.
// Each wave keeps an online-softmax state (m, l, acc) for its tokens; the four
// waves merge through LDS and write one partial (m, l, acc[128]) per head and
// chunk; kvq_combine merges the chunks (flash-decoding) and applies the V
// epilogue.  Reference semantics: src/kernels/triton_decode_attn_int8.py:126-303
// (online softmax, masking) and src/engine/patch_model.py:281-377 (fp16 dequant
// product code * scale, fp32 softmax, fp16 output).
#include "kvq_common.h"
#include "kvq.h"

#include <string>

namespace kvq {

constexpr int kWaves = 4;
constexpr int kTile = 32;  // tokens per wave iteration (two 16-token MFMA row blocks)
constexpr int kD = 128;

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
};

struct DecodeArgs {
  const half_t* q;
  int64_t q_sb, q_sh;
  const half_t* inv_tau;
  KvDev k, v;
  const int32_t* ctx;
  int B, Hq, Hkv, n_rep, gs;
  int64_t cap;
  float sm_log2e;
  int chunk, n_chunks;
  float* part_acc;  // [B, Hq, n_chunks, 128]
  float2* part_ml;  // [B, Hq, n_chunks]
  half_t* out;
  int64_t o_sb, o_sh;
};

__device__ __forceinline__ half_t ld_scale(const KvDev& kv, int64_t off) {
  if (kv.scale_f32) return (half_t)(reinterpret_cast<const float*>(kv.scale)[off]);
  return reinterpret_cast<const half_t*>(kv.scale)[off];
}
__device__ __forceinline__ uint32_t splat_h2(half_t s) {
  half2v v = {s, s};
  return as_u32(v);
}
__device__ __forceinline__ uint32_t pair_h2(half_t lo, half_t hi) {
  half2v v = {lo, hi};
  return as_u32(v);
}
// q' = fp16(q * inv_tau): fp16 x fp16 product rounded once, as torch's Half mul
__device__ __forceinline__ half_t qscale(half_t x, half_t tau, bool has_tau) {
  return has_tau ? (half_t)((float)x * (float)tau) : x;
}
// exact dequant of a half2 of codes (64 + n form): (n - 8) * s, rounded to fp16
__device__ __forceinline__ uint32_t deq_sym4(uint32_t u64pn, uint32_t s2) {
  const half2v off = {(half_t)72.0f, (half_t)72.0f};
  half2v c = as_h2(u64pn) - off;  // exact small integers
  return as_u32(c * as_h2(s2));
}
// int8 pair (already xor 0x80 and placed in the low byte of each half) -> (c * s)
__device__ __forceinline__ uint32_t deq_int8_pair(uint32_t perm_bytes, uint32_t s2) {
  const half2v off = {(half_t)1152.0f, (half_t)1152.0f};
  half2v c = as_h2(perm_bytes | kMagic1024) - off;
  return as_u32(c * as_h2(s2));
}

// two fp32 -> packed fp16, rounding toward zero (v_cvt_pkrtz_f16_f32)
__device__ __forceinline__ half2v pk_rtz(float a, float b) {
  return __builtin_bit_cast(half2v, __builtin_amdgcn_cvt_pkrtz(a, b));
}

// ---------------------------------------------------------------- K formats

// INT4 asymmetric, static scale/zero-point per (kv head, group of 32), optional fp16
// outlier channels.  One MFMA per quantisation group so the group scale is applied
// to the fp32 MFMA result (no fp16 rounding of q * s):
//   logit = sum_g s_g * C_g + sum_g Q_g (zp_g - 72 s_g) + sum_j q[o_j] k16[o_j]
// with C_g = sum_{d in g} q'_d (64 + n_d), Q_g = sum_{d in g} q'_d (outliers excluded).
struct KAsym4 {
  half8v qb[4];
  half4v qo;
  float sj[4];
  float bias;
  float sm;
  bool has_out;
  struct Raw {
    uint32_t w[4];
    u32x2 o;
  };

  __device__ void setup(const DecodeArgs& a, int b, int hkv, int col, int lg) {
    const bool valid = col < a.n_rep;
    const int hq = hkv * a.n_rep + (valid ? col : 0);
    const bool has_tau = a.inv_tau != nullptr;
    const half_t tau = has_tau ? a.inv_tau[hq] : (half_t)1.0f;
    const half_t* qrow = a.q + (int64_t)b * a.q_sb + (int64_t)hq * a.q_sh;
    has_out = a.k.n_out > 0;
    sm = a.sm_log2e;
    int oc[4] = {-1, -1, -1, -1};
    for (int i = 0; i < a.k.n_out; ++i) oc[i] = min(max(a.k.oidx[hkv * a.k.n_out + i], 0), kD - 1);
    float Q[4];
    for (int j = 0; j < 4; ++j) {
      half_t v8[8];
      float part = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 32 * j + 8 * lg + kNibSlotElem(e);
        half_t x = valid ? qscale(qrow[d], tau, has_tau) : (half_t)0.0f;
        if (d == oc[0] || d == oc[1] || d == oc[2] || d == oc[3]) x = (half_t)0.0f;
        v8[e] = x;
        part += (float)x;
      }
      qb[j] = half8v{v8[0], v8[1], v8[2], v8[3], v8[4], v8[5], v8[6], v8[7]};
      Q[j] = wave_sum_xor_groups(part);
    }
    half_t o4[4] = {(half_t)0.0f, (half_t)0.0f, (half_t)0.0f, (half_t)0.0f};
    if (lg == 0 && valid)
      for (int i = 0; i < a.k.n_out; ++i) o4[i] = qscale(qrow[oc[i]], tau, has_tau);
    qo = half4v{o4[0], o4[1], o4[2], o4[3]};
    const half_t* sc = reinterpret_cast<const half_t*>(a.k.scale);
    float bsum = 0.f;
    for (int j = 0; j < 4; ++j) {
      const float s = (float)sc[hkv * a.k.ssh + j * a.k.ssg];
      const float z = (float)a.k.zp[hkv * a.k.ssh + j * a.k.ssg];
      sj[j] = s * a.sm_log2e;
      bsum += Q[j] * (z - 72.0f * s);
    }
    bias = valid ? bsum : 0.f;
  }

  __device__ __forceinline__ void load(const DecodeArgs& a, int b, int hkv, int t, int lg,
                                       Raw& r) const {
    const uint8_t* p = a.k.codes + (int64_t)b * a.k.sb + (int64_t)hkv * a.k.sh +
                       (int64_t)t * a.k.st + 4 * lg;
#pragma unroll
    for (int j = 0; j < 4; ++j) r.w[j] = *reinterpret_cast<const uint32_t*>(p + 16 * j);
    r.o = u32x2{0u, 0u};
    if (has_out && lg == 0) {
      const half_t* o = a.k.oval + (int64_t)b * a.k.osb + (int64_t)hkv * a.k.osh +
                        (int64_t)t * a.k.ost;
      r.o = *reinterpret_cast<const u32x2*>(o);
    }
  }

  __device__ __forceinline__ float4v logits(const Raw& r) const {
    float4v co = {bias, bias, bias, bias};
    if (has_out) co = mfma16x16x16(pack4(r.o.x, r.o.y), qo, co);
    float4v x = co * sm;
    const float4v z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t u[4];
      unpack_dword_64pn(r.w[j], u);
      const float4v c = mfma16x16x32(pack8(u[0], u[1], u[2], u[3]), qb[j], z);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = fmaf(sj[j], c[i], x[i]);
    }
    return x;
  }
};

// INT8 or INT4-symmetric codes with a per-(token, group) scale.  K is dequantised
// exactly like the reference torch path, khat = fp16(code * fp16(scale)), then one
// MFMA accumulator covers all 128 channels.
template <bool I4>
struct KTok {
  half8v qb[4];
  float sm;
  struct Raw {
    uint32_t w[I4 ? 4 : 8];
    uint32_t s[4];
  };

  __device__ void setup(const DecodeArgs& a, int b, int hkv, int col, int lg) {
    const bool valid = col < a.n_rep;
    const int hq = hkv * a.n_rep + (valid ? col : 0);
    const bool has_tau = a.inv_tau != nullptr;
    const half_t tau = has_tau ? a.inv_tau[hq] : (half_t)1.0f;
    const half_t* qrow = a.q + (int64_t)b * a.q_sb + (int64_t)hq * a.q_sh;
    sm = a.sm_log2e;
    for (int j = 0; j < 4; ++j) {
      half_t v8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 32 * lg + 8 * j + (I4 ? kNibSlotElem(e) : e);
        v8[e] = valid ? qscale(qrow[d], tau, has_tau) : (half_t)0.0f;
      }
      qb[j] = half8v{v8[0], v8[1], v8[2], v8[3], v8[4], v8[5], v8[6], v8[7]};
    }
  }

  __device__ __forceinline__ void load(const DecodeArgs& a, int b, int hkv, int t, int lg,
                                       Raw& r) const {
    const uint8_t* p = a.k.codes + (int64_t)b * a.k.sb + (int64_t)hkv * a.k.sh +
                       (int64_t)t * a.k.st;
    if constexpr (I4) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(p + 16 * lg);
      r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
    } else {
      const u32x4 v0 = *reinterpret_cast<const u32x4*>(p + 32 * lg);
      const u32x4 v1 = *reinterpret_cast<const u32x4*>(p + 32 * lg + 16);
      r.w[0] = v0.x; r.w[1] = v0.y; r.w[2] = v0.z; r.w[3] = v0.w;
      r.w[4] = v1.x; r.w[5] = v1.y; r.w[6] = v1.z; r.w[7] = v1.w;
    }
    const int64_t sbase = (int64_t)b * a.k.ssb + (int64_t)hkv * a.k.ssh + (int64_t)t * a.k.sst;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gi = (32 * lg + 8 * j) / a.gs;
      r.s[j] = splat_h2(ld_scale(a.k, sbase + (int64_t)gi * a.k.ssg));
    }
  }

  __device__ __forceinline__ float4v logits(const Raw& r) const {
    float4v c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t u[4];
      if constexpr (I4) {
        unpack_dword_64pn(r.w[j], u);
#pragma unroll
        for (int i = 0; i < 4; ++i) u[i] = deq_sym4(u[i], r.s[j]);
      } else {
        const uint32_t w0 = r.w[2 * j] ^ 0x80808080u;
        const uint32_t w1 = r.w[2 * j + 1] ^ 0x80808080u;
        u[0] = deq_int8_pair(perm_b32(0u, w0, 0x0c010c00u), r.s[j]);
        u[1] = deq_int8_pair(perm_b32(0u, w0, 0x0c030c02u), r.s[j]);
        u[2] = deq_int8_pair(perm_b32(0u, w1, 0x0c010c00u), r.s[j]);
        u[3] = deq_int8_pair(perm_b32(0u, w1, 0x0c030c02u), r.s[j]);
      }
      c = mfma16x16x32(pack8(u[0], u[1], u[2], u[3]), qb[j], c);
    }
    return c * sm;
  }
};

// ---------------------------------------------------------------- V formats
//
// V^T operand: lane (c = lane % 16, lg = lane / 16) supplies d-row c and the 8 tokens
// T(lg) = {4lg..4lg+3, 16+4lg..16+4lg+3} of the tile (the tokens whose
// probabilities the same lane group holds after the QK MFMA).  It reads 8 channels
// d = 8c..8c+7 of each token; MFMA mb uses channel 8c + mb, so acc[mb][r] holds
// out^T[d = 32*lg + 8*r + mb, h = lane % 16].

__device__ __forceinline__ int tile_token(int lg, int e) {
  return e < 4 ? 4 * lg + e : 16 + 4 * lg + (e - 4);
}
__device__ __forceinline__ uint32_t sel_byte_pair(int k) {
  // [lo.byte_k, 0, hi.byte_k, 0]
  return (uint32_t)k | 0x0c00u | ((uint32_t)(4 + k) << 16) | 0x0c000000u;
}

// INT4 asymmetric static: accumulate sum_t p16 * (64 + n); the combine applies
// out = s_g * (acc / l - 72) + zp_g.
struct VAsym4 {
  struct Raw {
    uint32_t w[8];
  };
  __device__ void setup(const DecodeArgs&, int, int, int, int) {}
  __device__ __forceinline__ void load(const DecodeArgs& a, int b, int hkv, int tt, int t1,
                                       int col, int lg, Raw& r) const {
    const uint8_t* base = a.v.codes + (int64_t)b * a.v.sb + (int64_t)hkv * a.v.sh + 4 * col;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = min(tt + tile_token(lg, e), t1 - 1);
      r.w[e] = *reinterpret_cast<const uint32_t*>(base + (int64_t)t * a.v.st);
    }
  }
  __device__ __forceinline__ void mma(const Raw& r, half8v pb, float4v acc[8]) const {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t sel = sel_byte_pair(k);
      uint32_t R[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) R[p] = perm_b32(r.w[2 * p + 1], r.w[2 * p], sel);
      acc[2 * k] = mfma16x16x32(
          pack8(nib_hi_pair(R[0]), nib_hi_pair(R[1]), nib_hi_pair(R[2]), nib_hi_pair(R[3])),
          pb, acc[2 * k]);
      acc[2 * k + 1] = mfma16x16x32(pack8(nib_hi_pair(R[0] << 4), nib_hi_pair(R[1] << 4),
                                          nib_hi_pair(R[2] << 4), nib_hi_pair(R[3] << 4)),
                                    pb, acc[2 * k + 1]);
    }
  }
};

// INT8 / INT4-symmetric codes with per-(token, group) scale: vhat = fp16(code * scale).
template <bool I4>
struct VTok {
  struct Raw {
    uint32_t w[8][I4 ? 1 : 2];
    uint32_t s[4];
  };
  __device__ void setup(const DecodeArgs&, int, int, int, int) {}
  __device__ __forceinline__ void load(const DecodeArgs& a, int b, int hkv, int tt, int t1,
                                       int col, int lg, Raw& r) const {
    const uint8_t* base = a.v.codes + (int64_t)b * a.v.sb + (int64_t)hkv * a.v.sh +
                          (I4 ? 4 : 8) * col;
    const int gi = (8 * col) / a.gs;
    const int64_t sbase = (int64_t)b * a.v.ssb + (int64_t)hkv * a.v.ssh + (int64_t)gi * a.v.ssg;
    half_t sv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = min(tt + tile_token(lg, e), t1 - 1);
      if constexpr (I4) {
        r.w[e][0] = *reinterpret_cast<const uint32_t*>(base + (int64_t)t * a.v.st);
      } else {
        const u32x2 v = *reinterpret_cast<const u32x2*>(base + (int64_t)t * a.v.st);
        r.w[e][0] = v.x;
        r.w[e][1] = v.y;
      }
      sv[e] = ld_scale(a.v, sbase + (int64_t)t * a.v.sst);
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) r.s[p] = pair_h2(sv[2 * p], sv[2 * p + 1]);
  }
  __device__ __forceinline__ void mma(const Raw& r, half8v pb, float4v acc[8]) const {
    if constexpr (I4) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t sel = sel_byte_pair(k);
        uint32_t R[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) R[p] = perm_b32(r.w[2 * p + 1][0], r.w[2 * p][0], sel);
        acc[2 * k] = mfma16x16x32(
            pack8(deq_sym4(nib_hi_pair(R[0]), r.s[0]), deq_sym4(nib_hi_pair(R[1]), r.s[1]),
                  deq_sym4(nib_hi_pair(R[2]), r.s[2]), deq_sym4(nib_hi_pair(R[3]), r.s[3])),
            pb, acc[2 * k]);
        acc[2 * k + 1] = mfma16x16x32(pack8(deq_sym4(nib_hi_pair(R[0] << 4), r.s[0]),
                                            deq_sym4(nib_hi_pair(R[1] << 4), r.s[1]),
                                            deq_sym4(nib_hi_pair(R[2] << 4), r.s[2]),
                                            deq_sym4(nib_hi_pair(R[3] << 4), r.s[3])),
                                      pb, acc[2 * k + 1]);
      }
    } else {
      uint32_t wx[8][2];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        wx[e][0] = r.w[e][0] ^ 0x80808080u;
        wx[e][1] = r.w[e][1] ^ 0x80808080u;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t sel = sel_byte_pair(k & 3);
        uint32_t u[4];
#pragma unroll
        for (int p = 0; p < 4; ++p)
          u[p] = deq_int8_pair(perm_b32(wx[2 * p + 1][k >> 2], wx[2 * p][k >> 2], sel), r.s[p]);
        acc[k] = mfma16x16x32(pack8(u[0], u[1], u[2], u[3]), pb, acc[k]);
      }
    }
  }
};

// ---------------------------------------------------------------- main kernel

template <class KF, class VF>
__global__ __launch_bounds__(kWaves * 64) void decode_splitk_kernel(DecodeArgs a) {
  const int chunk = blockIdx.x, hkv = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, lg = lane >> 4;

  int64_t ctx64 = a.ctx[b];
  ctx64 = ctx64 < 0 ? 0 : (ctx64 > a.cap ? a.cap : ctx64);
  const int ctx = (int)ctx64;
  const int t0 = chunk * a.chunk;
  if (t0 >= ctx) return;  // uniform over the work-group
  const int t1 = min(t0 + a.chunk, ctx);

  KF kf;
  kf.setup(a, b, hkv, col, lg);
  VF vf;
  vf.setup(a, b, hkv, col, lg);

  float4v acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = float4v{0.f, 0.f, 0.f, 0.f};
  float m = kNegInf, l = 0.f;
  const half2v ones = {(half_t)1.0f, (half_t)1.0f};

  int tt = t0 + kTile * wave;
  typename KF::Raw kr0, kr1;
  typename VF::Raw vr;
  if (tt < t1) {
    kf.load(a, b, hkv, min(tt + col, t1 - 1), lg, kr0);
    kf.load(a, b, hkv, min(tt + 16 + col, t1 - 1), lg, kr1);
    vf.load(a, b, hkv, tt, t1, col, lg, vr);
  }
  for (; tt < t1; tt += kTile * kWaves) {
    // prefetch the next tile of this wave
    const int tn = tt + kTile * kWaves;
    typename KF::Raw nk0, nk1;
    typename VF::Raw nv;
    if (tn < t1) {
      kf.load(a, b, hkv, min(tn + col, t1 - 1), lg, nk0);
      kf.load(a, b, hkv, min(tn + 16 + col, t1 - 1), lg, nk1);
      vf.load(a, b, hkv, tn, t1, col, lg, nv);
    }

    float4v x0 = kf.logits(kr0);
    float4v x1 = kf.logits(kr1);
    if (tt + kTile > t1) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (tt + 4 * lg + r >= t1) x0[r] = kNegInf;
        if (tt + 16 + 4 * lg + r >= t1) x1[r] = kNegInf;
      }
    }
    float mx = fmaxf(fmaxf(fmaxf(x0[0], x0[1]), fmaxf(x0[2], x0[3])),
                     fmaxf(fmaxf(x1[0], x1[1]), fmaxf(x1[2], x1[3])));
    mx = wave_max_xor_groups(mx);
    const float mn = fmaxf(m, mx);
    const float alpha = fast_exp2(m - mn);
    m = mn;
    float p[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = fast_exp2(x0[r] - m);
      p[4 + r] = fast_exp2(x1[r] - m);
    }
    const half2v pp0 = pk_rtz(p[0], p[1]);
    const half2v pp1 = pk_rtz(p[2], p[3]);
    const half2v pp2 = pk_rtz(p[4], p[5]);
    const half2v pp3 = pk_rtz(p[6], p[7]);
    // l accumulates exactly the fp16 probabilities the PV MFMA consumes
    float ls = __builtin_amdgcn_fdot2(pp0, ones, 0.f, false);
    ls = __builtin_amdgcn_fdot2(pp1, ones, ls, false);
    ls = __builtin_amdgcn_fdot2(pp2, ones, ls, false);
    ls = __builtin_amdgcn_fdot2(pp3, ones, ls, false);
    l = fmaf(l, alpha, ls);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= alpha;
    const half8v pb = pack8(as_u32(pp0), as_u32(pp1), as_u32(pp2), as_u32(pp3));
    vf.mma(vr, pb, acc);

    kr0 = nk0;
    kr1 = nk1;
    vr = nv;
  }

  l = wave_sum_xor_groups(l);

  // ---- merge the 4 waves of the work-group through LDS
  __shared__ float sm_m[kWaves][16];
  __shared__ float sm_l[kWaves][16];
  __shared__ float sm_acc[kWaves][16][kD + 1];
  if (lg == 0) {
    sm_m[wave][col] = m;
    sm_l[wave][col] = l;
  }
#pragma unroll
  for (int mb = 0; mb < 8; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm_acc[wave][col][32 * lg + 8 * r + mb] = acc[mb][r];
  __syncthreads();

  for (int idx = threadIdx.x; idx < a.n_rep * kD; idx += kWaves * 64) {
    const int h = idx >> 7, d = idx & (kD - 1);
    float M = sm_m[0][h];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, sm_m[w][h]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float e = fast_exp2(sm_m[w][h] - M);
      num = fmaf(e, sm_acc[w][h][d], num);
      den = fmaf(e, sm_l[w][h], den);
    }
    const int hq = hkv * a.n_rep + h;
    const int64_t pi = ((int64_t)b * a.Hq + hq) * a.n_chunks + chunk;
    a.part_acc[pi * kD + d] = num;
    if (d == 0) a.part_ml[pi] = float2{M, den};
  }
}

// Combine the chunk partials of one (b, query head) and apply the V epilogue.
__global__ __launch_bounds__(kD) void combine_kernel(DecodeArgs a, int v_affine) {
  const int hq = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  int64_t ctx64 = a.ctx[b];
  ctx64 = ctx64 < 0 ? 0 : (ctx64 > a.cap ? a.cap : ctx64);
  const int nvalid = (int)((ctx64 + a.chunk - 1) / a.chunk);
  half_t* o = a.out + (int64_t)b * a.o_sb + (int64_t)hq * a.o_sh;
  if (nvalid == 0) {
    o[d] = (half_t)0.0f;
    return;
  }
  const int64_t base = ((int64_t)b * a.Hq + hq) * a.n_chunks;
  float M = kNegInf;
  for (int c = 0; c < nvalid; ++c) M = fmaxf(M, a.part_ml[base + c].x);
  float num = 0.f, den = 0.f;
  for (int c = 0; c < nvalid; ++c) {
    const float2 ml = a.part_ml[base + c];
    const float e = fast_exp2(ml.x - M);
    num = fmaf(e, a.part_acc[(base + c) * kD + d], num);
    den = fmaf(e, ml.y, den);
  }
  float r = num / den;
  if (v_affine) {
    const int hkv = hq / a.n_rep, g = d >> 5;
    const half_t* sc = reinterpret_cast<const half_t*>(a.v.scale);
    const float s = (float)sc[hkv * a.v.ssh + g * a.v.ssg];
    const float z = (float)a.v.zp[hkv * a.v.ssh + g * a.v.ssg];
    r = fmaf(s, r - 72.0f, z);
  }
  o[d] = (half_t)r;
}

// ---------------------------------------------------------------- host side

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

static bool aligned(const void* p, int n) { return ((uintptr_t)p % n) == 0; }

int32_t choose_chunk(const kvq_decode_params* p) {
  if (p->chunk_tokens > 0) return p->chunk_tokens;
  const int64_t units = (int64_t)p->batch * p->kv_heads;
  const int64_t target_wgs = 1024;  // 4 work-groups per CU on 256 CUs
  int64_t c = (p->capacity * units + target_wgs - 1) / target_wgs;
  c = ((c + 127) / 128) * 128;
  if (c < 256) c = 256;
  if (c > 8192) c = 8192;
  return (int32_t)c;
}

static KvDev to_dev(const kvq_kv_view& v) {
  KvDev d;
  d.codes = reinterpret_cast<const uint8_t*>(v.codes);
  d.sb = v.stride_b; d.sh = v.stride_h; d.st = v.stride_t;
  d.scale = v.scale;
  d.ssb = v.scale_stride_b; d.ssh = v.scale_stride_h; d.sst = v.scale_stride_t;
  d.ssg = v.scale_stride_g;
  d.scale_f32 = v.scale_dtype == KVQ_DTYPE_F32;
  d.n_out = v.n_outlier;
  d.zp = reinterpret_cast<const half_t*>(v.zero_point);
  d.oidx = v.outlier_idx;
  d.oval = reinterpret_cast<const half_t*>(v.outlier_val);
  d.osb = v.outlier_stride_b; d.osh = v.outlier_stride_h; d.ost = v.outlier_stride_t;
  return d;
}

static int check_view(const kvq_kv_view& v, int fmt, bool is_k, const char* name, int gs) {
  std::string n(name);
  if (!v.codes) return fail(KVQ_ERR_INVALID, n + ": codes is NULL");
  if (!v.scale) return fail(KVQ_ERR_INVALID, n + ": scale is NULL");
  const int row_bytes = fmt == KVQ_FMT_INT8_SYM ? kD : kD / 2;
  if (v.stride_t < row_bytes && v.stride_t != 0)
    return fail(KVQ_ERR_INVALID, n + ": token stride smaller than a code row");
  const int need = (fmt == KVQ_FMT_INT4_SYM && is_k) ? 16 : (fmt == KVQ_FMT_INT8_SYM ? (is_k ? 16 : 8) : 4);
  if (!aligned(v.codes, need) || v.stride_b % need || v.stride_h % need || v.stride_t % need)
    return fail(KVQ_ERR_UNSUPPORTED,
                n + ": code rows must be " + std::to_string(need) + "-byte aligned");
  if (v.scale_dtype != KVQ_DTYPE_F16 && v.scale_dtype != KVQ_DTYPE_F32)
    return fail(KVQ_ERR_INVALID, n + ": scale_dtype must be F16 or F32");
  if (fmt == KVQ_FMT_INT4_ASYM) {
    if (gs != 32) return fail(KVQ_ERR_UNSUPPORTED, n + ": INT4_ASYM needs group_size 32");
    if (v.scale_dtype != KVQ_DTYPE_F16)
      return fail(KVQ_ERR_UNSUPPORTED, n + ": INT4_ASYM needs fp16 static scale");
    if (!v.zero_point) return fail(KVQ_ERR_INVALID, n + ": INT4_ASYM needs zero_point");
    if (v.n_outlier != 0) {
      if (!is_k) return fail(KVQ_ERR_UNSUPPORTED, n + ": outlier channels are K only");
      if (v.n_outlier != 4)
        return fail(KVQ_ERR_UNSUPPORTED, n + ": n_outlier must be 0 or 4");
      if (!v.outlier_idx || !v.outlier_val)
        return fail(KVQ_ERR_INVALID, n + ": outlier pointers are NULL");
      if (!aligned(v.outlier_val, 8) || v.outlier_stride_b % 4 || v.outlier_stride_h % 4 ||
          v.outlier_stride_t % 4)
        return fail(KVQ_ERR_UNSUPPORTED, n + ": outlier rows must be 8-byte aligned");
    }
  } else if (v.n_outlier != 0) {
    return fail(KVQ_ERR_UNSUPPORTED, n + ": outlier channels need INT4_ASYM");
  }
  return KVQ_OK;
}

template <class KF, class VF>
static void launch(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((decode_splitk_kernel<KF, VF>), grid, dim3(kWaves * 64), 0, s, a);
}

}  // namespace kvq

using namespace kvq;

extern "C" int32_t kvq_decode_chunk_tokens(const kvq_decode_params* p) {
  return p ? choose_chunk(p) : 0;
}

extern "C" int64_t kvq_decode_workspace_bytes(const kvq_decode_params* p) {
  if (!p) return 0;
  const int64_t chunk = choose_chunk(p);
  const int64_t nch = (p->capacity + chunk - 1) / chunk;
  const int64_t rows = (int64_t)p->batch * p->q_heads * (nch > 0 ? nch : 1);
  return rows * (kD * 4 + 8) + 256;
}

extern "C" int kvq_decode_attn(const kvq_decode_params* p, kvq_stream_t stream) {
  if (!p) return fail(KVQ_ERR_INVALID, "params is NULL");
  if (p->head_dim != kD) return fail(KVQ_ERR_UNSUPPORTED, "head_dim must be 128");
  if (p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0)
    return fail(KVQ_ERR_INVALID, "batch/q_heads/kv_heads must be positive");
  if (p->q_heads % p->kv_heads)
    return fail(KVQ_ERR_INVALID, "q_heads must be a multiple of kv_heads");
  const int n_rep = p->q_heads / p->kv_heads;
  if (n_rep > 16) return fail(KVQ_ERR_UNSUPPORTED, "q_heads / kv_heads must be <= 16");
  const int gs = p->group_size;
  if (gs != 8 && gs != 16 && gs != 32 && gs != 64 && gs != 128)
    return fail(KVQ_ERR_UNSUPPORTED, "group_size must be 8, 16, 32, 64 or 128");
  if (p->capacity < 0 || p->capacity > (int64_t)1 << 30)
    return fail(KVQ_ERR_INVALID, "capacity out of range");
  if (!p->q || !p->out || !p->context_lens)
    return fail(KVQ_ERR_INVALID, "q/out/context_lens is NULL");
  if (!aligned(p->q, 16) || p->q_stride_b % 8 || p->q_stride_h % 8)
    return fail(KVQ_ERR_UNSUPPORTED, "q rows must be 16-byte aligned");
  const int kf = p->k_format, vf = p->v_format;
  const bool combo_ok = (kf == KVQ_FMT_INT8_SYM && vf == KVQ_FMT_INT8_SYM) ||
                        (kf == KVQ_FMT_INT4_SYM && vf == KVQ_FMT_INT4_SYM) ||
                        (kf == KVQ_FMT_INT4_ASYM && vf == KVQ_FMT_INT4_ASYM) ||
                        (kf == KVQ_FMT_INT8_SYM && vf == KVQ_FMT_INT4_ASYM);
  if (!combo_ok) return fail(KVQ_ERR_UNSUPPORTED, "unsupported (k_format, v_format) pair");
  int rc = check_view(p->k, kf, true, "k", gs);
  if (rc) return rc;
  rc = check_view(p->v, vf, false, "v", gs);
  if (rc) return rc;

  const int32_t chunk = choose_chunk(p);
  if (chunk <= 0 || chunk % (kTile * kWaves))
    return fail(KVQ_ERR_INVALID, "chunk_tokens must be a positive multiple of 128");
  const int64_t nch64 = p->capacity > 0 ? (p->capacity + chunk - 1) / chunk : 1;
  if (nch64 > 65535) return fail(KVQ_ERR_UNSUPPORTED, "too many chunks");
  const int64_t need = kvq_decode_workspace_bytes(p);
  if (!p->workspace || p->workspace_bytes < need)
    return fail(KVQ_ERR_INVALID, "workspace too small: need " + std::to_string(need) + " bytes");
  if (!aligned(p->workspace, 16)) return fail(KVQ_ERR_INVALID, "workspace must be 16-byte aligned");

  DecodeArgs a;
  a.q = reinterpret_cast<const half_t*>(p->q);
  a.q_sb = p->q_stride_b; a.q_sh = p->q_stride_h;
  a.inv_tau = reinterpret_cast<const half_t*>(p->inv_tau);
  a.k = to_dev(p->k);
  a.v = to_dev(p->v);
  a.ctx = p->context_lens;
  a.B = p->batch; a.Hq = p->q_heads; a.Hkv = p->kv_heads; a.n_rep = n_rep; a.gs = gs;
  a.cap = p->capacity;
  a.sm_log2e = p->sm_scale * kLog2e;
  a.chunk = chunk;
  a.n_chunks = (int)nch64;
  const int64_t rows = (int64_t)p->batch * p->q_heads * nch64;
  a.part_acc = reinterpret_cast<float*>(p->workspace);
  a.part_ml = reinterpret_cast<float2*>(reinterpret_cast<char*>(p->workspace) + rows * kD * 4);
  a.out = reinterpret_cast<half_t*>(p->out);
  a.o_sb = p->out_stride_b; a.o_sh = p->out_stride_h;

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (p->capacity > 0) {
    const dim3 grid((unsigned)nch64, (unsigned)p->kv_heads, (unsigned)p->batch);
    if (kf == KVQ_FMT_INT8_SYM && vf == KVQ_FMT_INT8_SYM)
      launch<KTok<false>, VTok<false>>(a, grid, s);
    else if (kf == KVQ_FMT_INT4_SYM)
      launch<KTok<true>, VTok<true>>(a, grid, s);
    else if (kf == KVQ_FMT_INT4_ASYM)
      launch<KAsym4, VAsym4>(a, grid, s);
    else
      launch<KTok<false>, VAsym4>(a, grid, s);
  }
  hipLaunchKernelGGL(combine_kernel, dim3(p->q_heads, p->batch), dim3(kD), 0, s, a,
                     vf == KVQ_FMT_INT4_ASYM ? 1 : 0);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(KVQ_ERR_LAUNCH, std::string("launch: ") + hipGetErrorString(e));
  return KVQ_OK;
}

extern "C" const char* kvq_last_error(void) { return g_last_error.c_str(); }
extern "C" int32_t kvq_abi_version(void) { return 1; }

// Split-K quantized decode attention for gfx950 (CDNA4).
//
// One work-group = 4 wavefronts = one (batch b, kv head, chunk of tokens).  All
// n_rep query heads that share the kv head are processed together (GQA): the
// heads are the N dimension (padded to 16) of v_mfma_f32_16x16x32_f16 and the
// tokens are M, so every code byte is read from HBM exactly once.
//
//   S^T[t, h]   = K[t, :] . q'[h, :]           A = K tile (codes as fp16), B = q'^T
//   out^T[d, h] = sum_t V^T[d, t] * P^T[t, h]  A = V^T (codes as fp16),    B = P^T
//
// The D layout of the first MFMA (lane = (h, 4 tokens)) is exactly the B layout
// the second one needs, so probabilities never leave registers.  Each wave streams
// 32-token tiles with a ring of DEPTH tiles in registers (DEPTH-1 in flight while
// one is computed) and keeps an online-softmax state (m, l, acc).  The running max
// is raised lazily: p = 2^(x - m) may reach 2^kTau before the accumulators are
// rescaled.  The four waves merge through LDS into one partial (m, l, acc[128])
// per head and chunk; combine_kernel merges the chunks (flash-decoding) and applies
// the V epilogue.
//
// Reference semantics: src/kernels/triton_decode_attn_int8.py:126-303 (online
// softmax, masking, zero-context rows) and src/engine/patch_model.py:281-377
// (dequant product code * scale in fp16, fp32 softmax, fp16 output).
#include "decode_common.h"

#include <cstdlib>
#include <map>
#include <mutex>
#include <string>
#include <utility>

namespace kvq {

// ---------------------------------------------------------------- K formats
//
// A operand of the QK MFMA: lane (row = lane % 16, lg = lane / 16) of row block s
// (0/1) supplies token tt + 16 s + row.  For INT4 it reads the 16 bytes [16 lg, 16 lg
// + 16) of that token's 64-byte code row = channels [32 lg, 32 lg + 32) = quantisation
// group lg; dword j feeds MFMA j with channels 32 lg + 8 j + kNibSlotElem(e).

// INT4 asymmetric, static scale s / zero-point z per (kv head, group of 32), optional
// fp16 outlier channels.  With x = 64 + n = c + 72 the logit is
//   sum_d q_d (s_g c_d + z_g) = sum_d (q_d s_g) x_d + sum_d q_d (z_g - 72 s_g)
// q_d s_g (exact in fp32) is split into fp16 hi + lo; both go through the MFMA, so the
// product is not rounded to fp16.  The constant term is the accumulator's initial value;
// outlier channels (q zeroed in the main MFMAs) are added by one more MFMA whose A and B
// operands hold the 4 outlier values / q' entries in lane group 0 and zeros elsewhere.
template <bool OUT>
struct KAsym4 {
  static constexpr bool has_out = OUT;
  half8v qh[4], ql[4];
  half8v qo;  // q' of the outlier channels in k-slots 0..3 of lane group 0, zero elsewhere
  float bias;
  const uint8_t* kb;
  const half_t* ob;
  int64_t st, ost;
  uint32_t koff[2], ooff[2];
  int row, lg;
  struct Raw {
    u32x4 w[2];
    u32x2 o[2];
  };

  __device__ void setup(const DecodeArgs& a, int b, int hkv, int col, int lg_) {
    row = col;
    lg = lg_;
    const bool valid = col < a.n_rep;
    const int hq = hkv * a.n_rep + (valid ? col : 0);
    const bool has_tau = a.inv_tau != nullptr;
    const half_t tau = has_tau ? a.inv_tau[hq] : (half_t)1.0f;
    const half_t* qr = q_row(a, b, hq);
    // all loads are unconditional and issued together (no branch per element)
    int oc[4] = {-1, -1, -1, -1};
    if constexpr (OUT) {
      const int4 o = *reinterpret_cast<const int4*>(a.k.oidx + hkv * 4);
      oc[0] = min(max(o.x, 0), kD - 1);
      oc[1] = min(max(o.y, 0), kD - 1);
      oc[2] = min(max(o.z, 0), kD - 1);
      oc[3] = min(max(o.w, 0), kD - 1);
    }
    half_t qv[32];
    load_q_group(qr, lg, tau, has_tau, qv);
    half_t qoe[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) qoe[i] = qscale(qr[OUT ? oc[i] : 0], tau, has_tau);
    const half_t* sc = reinterpret_cast<const half_t*>(a.k.scale);
    const float s = (float)sc[hkv * a.k.ssh + lg * a.k.ssg];
    const float z = (float)a.k.zp[hkv * a.k.ssh + lg * a.k.ssg];
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      half_t vh[8], vl[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int dl = 8 * j + kNibSlotElem(e);
        const int d = 32 * lg + dl;
        const bool use = valid && d != oc[0] && d != oc[1] && d != oc[2] && d != oc[3];
        const float qd = use ? (float)qv[dl] : 0.f;
        const float P = qd * s;  // exact: 11-bit x 11-bit significands
        const half_t hi = (half_t)P;
        const half_t lo = (half_t)(P - (float)hi);
        vh[e] = hi;
        vl[e] = lo;
        part += qd * z - 72.0f * ((float)hi + (float)lo);
      }
      qh[j] = half8v{vh[0], vh[1], vh[2], vh[3], vh[4], vh[5], vh[6], vh[7]};
      ql[j] = half8v{vl[0], vl[1], vl[2], vl[3], vl[4], vl[5], vl[6], vl[7]};
    }
    bias = wave_sum_xor_groups(part);
    const bool own = lg == 0 && valid && OUT;
    const half_t h0 = (half_t)0.0f;
    qo = half8v{own ? qoe[0] : h0, own ? qoe[1] : h0, own ? qoe[2] : h0, own ? qoe[3] : h0,
                h0, h0, h0, h0};
    kb = a.k.codes + (int64_t)b * a.k.sb + (int64_t)hkv * a.k.sh;
    st = a.k.st;
    koff[0] = (uint32_t)(row * st + 16 * lg);
    koff[1] = (uint32_t)((row + 16) * st + 16 * lg);
    ob = a.k.oval + (int64_t)b * a.k.osb + (int64_t)hkv * a.k.osh;
    ost = a.k.ost;
    ooff[0] = (uint32_t)(row * ost);
    ooff[1] = (uint32_t)((row + 16) * ost);
  }

  __device__ __forceinline__ void load_full(int tt, Raw& r) const {
    const uint8_t* p = kb + (int64_t)tt * st;
    r.w[0] = ld_stream<u32x4>(p + koff[0]);
    r.w[1] = ld_stream<u32x4>(p + koff[1]);
    if constexpr (OUT) {
      r.o[0] = r.o[1] = u32x2{0u, 0u};
      if (lg == 0) {
        const half_t* o = ob + (int64_t)tt * ost;
        r.o[0] = ld_stream<u32x2>(o + ooff[0]);
        r.o[1] = ld_stream<u32x2>(o + ooff[1]);
      }
    }
  }
  __device__ __forceinline__ void load_clamped(int tt, int t1, Raw& r) const {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int t = min(tt + 16 * s + row, t1 - 1);
      r.w[s] = ld_stream<u32x4>(kb + (int64_t)t * st + 16 * lg);
      if constexpr (OUT) {
        r.o[s] = u32x2{0u, 0u};
        if (lg == 0) r.o[s] = ld_stream<u32x2>(ob + (int64_t)t * ost);
      }
    }
  }

  __device__ __forceinline__ float4v qk(const Raw& r, int s, const NibConsts& nc) const {
    float4v c = {bias, bias, bias, bias};
    // Same MFMA shape as the chain below, so the accumulator chain never changes shape.
    if constexpr (OUT) c = mfma16x16x32(pack8(r.o[s].x, r.o[s].y, 0u, 0u), qo, c);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t u[4];
      unpack_dword_64pn(r.w[s][j], nc, u);
      const half8v A = pack8(u[0], u[1], u[2], u[3]);
      c = mfma16x16x32(A, qh[j], c);
      c = mfma16x16x32(A, ql[j], c);
    }
    return c;
  }
};

// INT8 or INT4-symmetric codes with a per-(token, group) scale.  K is dequantised
// like the reference torch path, khat = fp16(code * fp16(scale)), then one MFMA
// accumulator covers all 128 channels.
template <bool I4, bool SF32>
struct KTok {
  half8v qb[4];
  const uint8_t* kb;
  int64_t st;
  const void* sp;
  int64_t sst, ssg;
  uint32_t koff[2];
  int row, lg, gsh[4];
  struct Raw {
    uint32_t w[2][I4 ? 4 : 8];
    uint32_t s[2][4];
  };

  __device__ void setup(const DecodeArgs& a, int b, int hkv, int col, int lg_) {
    row = col;
    lg = lg_;
    const bool valid = col < a.n_rep;
    const int hq = hkv * a.n_rep + (valid ? col : 0);
    const bool has_tau = a.inv_tau != nullptr;
    const half_t tau = has_tau ? a.inv_tau[hq] : (half_t)1.0f;
    const half_t* qr = q_row(a, b, hq);
    half_t qv[32];
    load_q_group(qr, lg, tau, has_tau, qv);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      half_t v8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int dl = 8 * j + (I4 ? kNibSlotElem(e) : e);
        v8[e] = valid ? qv[dl] : (half_t)0.0f;
      }
      qb[j] = half8v{v8[0], v8[1], v8[2], v8[3], v8[4], v8[5], v8[6], v8[7]};
      gsh[j] = (32 * lg + 8 * j) / a.gs;
    }
    kb = a.k.codes + (int64_t)b * a.k.sb + (int64_t)hkv * a.k.sh;
    st = a.k.st;
    const int span = I4 ? 16 : 32;
    koff[0] = (uint32_t)(row * st + span * lg);
    koff[1] = (uint32_t)((row + 16) * st + span * lg);
    sp = reinterpret_cast<const char*>(a.k.scale) +
         ((int64_t)b * a.k.ssb + (int64_t)hkv * a.k.ssh) * (SF32 ? 4 : 2);
    sst = a.k.sst;
    ssg = a.k.ssg;
  }

  __device__ __forceinline__ half_t scale_at(int t, int gi) const {
    const int64_t off = (int64_t)t * sst + (int64_t)gi * ssg;
    if constexpr (SF32) return (half_t)(reinterpret_cast<const float*>(sp)[off]);
    return reinterpret_cast<const half_t*>(sp)[off];
  }

  __device__ __forceinline__ void load_full(int tt, Raw& r) const { load_impl<true>(tt, 0, r); }
  __device__ __forceinline__ void load_clamped(int tt, int t1, Raw& r) const {
    load_impl<false>(tt, t1, r);
  }
  template <bool FULL>
  __device__ __forceinline__ void load_impl(int tt, int t1, Raw& r) const {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int t = FULL ? tt + 16 * s + row : min(tt + 16 * s + row, t1 - 1);
      const uint8_t* p = FULL ? kb + (int64_t)tt * st + koff[s]
                              : kb + (int64_t)t * st + (I4 ? 16 : 32) * lg;
      const u32x4 v0 = ld_stream<u32x4>(p);
      r.w[s][0] = v0.x; r.w[s][1] = v0.y; r.w[s][2] = v0.z; r.w[s][3] = v0.w;
      if constexpr (!I4) {
        const u32x4 v1 = ld_stream<u32x4>(p + 16);
        r.w[s][4] = v1.x; r.w[s][5] = v1.y; r.w[s][6] = v1.z; r.w[s][7] = v1.w;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) r.s[s][j] = splat_h2(scale_at(t, gsh[j]));
    }
  }

  __device__ __forceinline__ float4v qk(const Raw& r, int s, const NibConsts& nc) const {
    float4v c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t u[4];
      if constexpr (I4) {
        unpack_dword_64pn(r.w[s][j], nc, u);
#pragma unroll
        for (int i = 0; i < 4; ++i) u[i] = deq_pair(u[i], (half_t)72.0f, r.s[s][j]);
      } else {
        const uint32_t w0 = r.w[s][2 * j] ^ 0x80808080u;
        const uint32_t w1 = r.w[s][2 * j + 1] ^ 0x80808080u;
        u[0] = deq_pair(perm_b32(0u, w0, 0x0c010c00u) | nc.c1024, (half_t)1152.0f, r.s[s][j]);
        u[1] = deq_pair(perm_b32(0u, w0, 0x0c030c02u) | nc.c1024, (half_t)1152.0f, r.s[s][j]);
        u[2] = deq_pair(perm_b32(0u, w1, 0x0c010c00u) | nc.c1024, (half_t)1152.0f, r.s[s][j]);
        u[3] = deq_pair(perm_b32(0u, w1, 0x0c030c02u) | nc.c1024, (half_t)1152.0f, r.s[s][j]);
      }
      c = mfma16x16x32(pack8(u[0], u[1], u[2], u[3]), qb[j], c);
    }
    return c;
  }
};

// ---------------------------------------------------------------- V formats
//
// V^T operand: lane (c = lane % 16, lg = lane / 16) supplies d-row c and the 8 tokens
// T(lg) = {4lg..4lg+3, 16+4lg..16+4lg+3} of the tile, which are the tokens whose
// probabilities the same lane group holds after the QK MFMA.  It reads channels
// 8c..8c+7 of each token, and MFMA mb uses channel 8c + mb, so acc[mb][r] holds
// out^T[d = 32 lg + 8 r + mb, h = lane % 16].  Byte k of two tokens is gathered into
// one dword with v_perm_b32; its high nibbles (even channels) become 64 + n and its
// low nibbles (odd channels) 1024 + n.

__device__ __forceinline__ int tile_token_uniform(int e) { return e < 4 ? e : e + 12; }
__device__ __forceinline__ uint32_t sel_byte_pair(int k) {
  // [lo.byte_k, 0, hi.byte_k, 0]
  return (uint32_t)k | 0x0c00u | ((uint32_t)(4 + k) << 16) | 0x0c000000u;
}

// INT4 asymmetric static: accumulates sum_t p16 * x with x = 64 + n (even d) or 1024 + n
// (odd d); combine_kernel applies out_d = s_g * (acc_d / l - off_d) + z_g, off_d = 72 or 1032.
struct VAsym4 {
  const uint8_t* vb;
  int64_t st;
  uint32_t voff;
  int col, lg;
  struct Raw {
    uint32_t w[8];
  };
  __device__ void setup(const DecodeArgs& a, int b, int hkv, int col_, int lg_) {
    col = col_;
    lg = lg_;
    vb = a.v.codes + (int64_t)b * a.v.sb + (int64_t)hkv * a.v.sh;
    st = a.v.st;
    voff = (uint32_t)(4 * lg * st + 4 * col);
  }
  __device__ __forceinline__ void load_full(int tt, Raw& r) const {
    const uint8_t* p = vb + (int64_t)tt * st + voff;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      r.w[e] = ld_stream<uint32_t>(p + (int64_t)tile_token_uniform(e) * st);
  }
  __device__ __forceinline__ void load_clamped(int tt, int t1, Raw& r) const {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = min(tt + 4 * lg + tile_token_uniform(e), t1 - 1);
      r.w[e] = ld_stream<uint32_t>(vb + (int64_t)t * st + 4 * col);
    }
  }
  // codes as the exact fp16 subnormals 16 n 2^-24 (even channel, high nibble) and n 2^-24
  // (odd channel), each multiplied by both probability operands (softmax_tile); the
  // combine applies out = s (acc / l * 2^20 or 2^24 - 8) + z
  __device__ __forceinline__ void mma(const Raw& r, half8v pb, half8v pl, float4v acc[8],
                                      const NibConsts& nc) const {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t sel = sel_byte_pair(k);
      uint32_t R[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) R[p] = perm_b32(r.w[2 * p + 1], r.w[2 * p], sel);
      const half8v ah = pack8(R[0] & nc.m_hi, R[1] & nc.m_hi, R[2] & nc.m_hi, R[3] & nc.m_hi);
      const half8v al = pack8(R[0] & nc.m_lo, R[1] & nc.m_lo, R[2] & nc.m_lo, R[3] & nc.m_lo);
      acc[2 * k] = mfma16x16x32(ah, pb, acc[2 * k]);
      acc[2 * k + 1] = mfma16x16x32(al, pb, acc[2 * k + 1]);
      acc[2 * k] = mfma16x16x32(ah, pl, acc[2 * k]);
      acc[2 * k + 1] = mfma16x16x32(al, pl, acc[2 * k + 1]);
    }
  }
};

// INT8 / INT4-symmetric codes with per-(token, group) scale: vhat = fp16(code * scale).
template <bool I4, bool SF32>
struct VTok {
  const uint8_t* vb;
  int64_t st;
  const void* sp;
  int64_t sst;
  int col, lg;
  struct Raw {
    uint32_t w[8][I4 ? 1 : 2];
    uint32_t s[4];
  };
  __device__ void setup(const DecodeArgs& a, int b, int hkv, int col_, int lg_) {
    col = col_;
    lg = lg_;
    vb = a.v.codes + (int64_t)b * a.v.sb + (int64_t)hkv * a.v.sh + (I4 ? 4 : 8) * col;
    st = a.v.st;
    const int gi = (8 * col) / a.gs;
    sp = reinterpret_cast<const char*>(a.v.scale) +
         ((int64_t)b * a.v.ssb + (int64_t)hkv * a.v.ssh + (int64_t)gi * a.v.ssg) * (SF32 ? 4 : 2);
    sst = a.v.sst;
  }
  __device__ __forceinline__ void load_full(int tt, Raw& r) const { load_impl<true>(tt, 0, r); }
  __device__ __forceinline__ void load_clamped(int tt, int t1, Raw& r) const {
    load_impl<false>(tt, t1, r);
  }
  template <bool FULL>
  __device__ __forceinline__ void load_impl(int tt, int t1, Raw& r) const {
    half_t sv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      int t = tt + 4 * lg + tile_token_uniform(e);
      if (!FULL) t = min(t, t1 - 1);
      const uint8_t* p = vb + (int64_t)t * st;
      if constexpr (I4) {
        r.w[e][0] = ld_stream<uint32_t>(p);
      } else {
        const u32x2 v = ld_stream<u32x2>(p);
        r.w[e][0] = v.x;
        r.w[e][1] = v.y;
      }
      const int64_t so = (int64_t)t * sst;
      if constexpr (SF32) sv[e] = (half_t)(reinterpret_cast<const float*>(sp)[so]);
      else sv[e] = reinterpret_cast<const half_t*>(sp)[so];
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) r.s[p] = pair_h2(sv[2 * p], sv[2 * p + 1]);
  }
  // vhat = fp16(code * scale) times both probability operands (softmax_tile)
  __device__ __forceinline__ void mma(const Raw& r, half8v pb, half8v pl, float4v acc[8],
                                      const NibConsts& nc) const {
    if constexpr (I4) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t sel = sel_byte_pair(k);
        uint32_t R[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) R[p] = perm_b32(r.w[2 * p + 1][0], r.w[2 * p][0], sel);
        uint32_t h[4], o[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          h[p] = deq_pair(and_or(R[p], nc.m_hi, nc.c64), (half_t)72.0f, r.s[p]);
          o[p] = deq_pair(and_or(R[p], nc.m_lo, nc.c1024), (half_t)1032.0f, r.s[p]);
        }
        const half8v ah = pack8(h[0], h[1], h[2], h[3]), ao = pack8(o[0], o[1], o[2], o[3]);
        acc[2 * k] = mfma16x16x32(ah, pb, acc[2 * k]);
        acc[2 * k + 1] = mfma16x16x32(ao, pb, acc[2 * k + 1]);
        acc[2 * k] = mfma16x16x32(ah, pl, acc[2 * k]);
        acc[2 * k + 1] = mfma16x16x32(ao, pl, acc[2 * k + 1]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t sel = sel_byte_pair(k & 3);
        uint32_t u[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t hi = r.w[2 * p + 1][k >> 2] ^ 0x80808080u;
          const uint32_t lo = r.w[2 * p][k >> 2] ^ 0x80808080u;
          u[p] = deq_pair(perm_b32(hi, lo, sel) | nc.c1024, (half_t)1152.0f, r.s[p]);
        }
        const half8v au = pack8(u[0], u[1], u[2], u[3]);
        acc[k] = mfma16x16x32(au, pb, acc[k]);
        acc[k] = mfma16x16x32(au, pl, acc[k]);
      }
    }
  }
};

// ---------------------------------------------------------------- main kernel

template <class KF, class VF, int DEPTH>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2)))
void decode_splitk_kernel(DecodeArgs a) {
  const int chunk = blockIdx.x, hkv = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  // wave index is uniform per wave; say so, so tile addressing stays in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, lg = lane >> 4;

  const int64_t ctx64 = row_context(a, b);
  const int ctx = (int)ctx64;
  const int t0 = chunk * a.chunk;
  if (t0 >= ctx) return;  // uniform over the work-group
  const int t1 = min(t0 + a.chunk, ctx);

  NibConsts nc;
  nc.init();
  KF kf;
  kf.setup(a, b, hkv, col, lg);
  VF vf;
  vf.setup(a, b, hkv, col, lg);

  float4v acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = float4v{0.f, 0.f, 0.f, 0.f};
  float m = kNegInf, l = 0.f;
  const float sm = a.sm_log2e;
  constexpr int kStep = kTile * kWaves;
  const int tw = t0 + kTile * wave;

  // Softmax + PV of one tile whose QK logits (x0: tokens 4lg+r, x1: 16+4lg+r) are known.
  auto finish = [&](float4v x0, float4v x1, const typename VF::Raw& vt, int tt, bool masked) {
    if (masked) mask_tile(x0, x1, tt, t1, lg);
    half8v pb, pl;
    softmax_tile(x0, x1, sm, m, l, acc, pb, pl);
    vf.mma(vt, pb, pl, acc, nc);
  };

  // Full tiles of this wave are tw + i * kStep for i < nfull; the (at most one) partial
  // tile after them is peeled off with clamped loads and masking.  QK runs one tile
  // ahead of softmax/PV, so the next tile's MFMA chain overlaps this tile's VALU work.
  // K tile i + DEPTH and V tile i + DEPTH - 1 are fetched during iteration i.
  const int nfull = (t1 - tw >= kTile) ? (t1 - tw - kTile) / kStep + 1 : 0;
  if (nfull > 0) {
    typename KF::Raw kr[DEPTH];
    typename VF::Raw vr[DEPTH];
#pragma unroll
    for (int s = 0; s < DEPTH; ++s)
      if (s < nfull) kf.load_full(tw + s * kStep, kr[s]);
#pragma unroll
    for (int s = 0; s < DEPTH - 1; ++s)
      if (s < nfull) vf.load_full(tw + s * kStep, vr[s]);
    float4v xa0 = kf.qk(kr[0], 0, nc), xa1 = kf.qk(kr[0], 1, nc);
    for (int i0 = 0; i0 < nfull; i0 += DEPTH) {
#pragma unroll
      for (int s = 0; s < DEPTH; ++s) {
        const int i = i0 + s;
        if (i >= nfull) break;
        if (i + DEPTH - 1 < nfull) vf.load_full(tw + (i + DEPTH - 1) * kStep, vr[(s + DEPTH - 1) % DEPTH]);
        float4v xb0 = xa0, xb1 = xa1;
        if (i + 1 < nfull) {
          xb0 = kf.qk(kr[(s + 1) % DEPTH], 0, nc);
          xb1 = kf.qk(kr[(s + 1) % DEPTH], 1, nc);
        }
        if (i + DEPTH < nfull) kf.load_full(tw + (i + DEPTH) * kStep, kr[s]);
        finish(xa0, xa1, vr[s], tw + i * kStep, false);
        xa0 = xb0;
        xa1 = xb1;
      }
    }
  }
  const int ttail = tw + nfull * kStep;
  if (ttail < t1) {
    typename KF::Raw kt;
    typename VF::Raw vt;
    kf.load_clamped(ttail, t1, kt);
    vf.load_clamped(ttail, t1, vt);
    finish(kf.qk(kt, 0, nc), kf.qk(kt, 1, nc), vt, ttail, true);
  }

  __shared__ MergeLds msh;
  merge_and_store(a, msh, wave, col, lg, m, l, acc, b, hkv, chunk);
}

// Combine the chunk partials of one (b, query head) and apply the V epilogue (the
// row-layout kernels; the tiled kernels combine in their last work-group).
__global__ __launch_bounds__(kD) void combine_kernel(DecodeArgs a, int v_affine) {
  const int hq = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int64_t ctx64 = row_context(a, b);
  combine_one(a, b, hq, d, valid_chunks(a, ctx64), v_affine);
}

// ---------------------------------------------------------------- host side

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

static bool aligned(const void* p, int n) { return ((uintptr_t)p % n) == 0; }

// Register-ring depth = tiles per wave in flight + 1.  Default: the deepest ring (4, 3
// or 2) whose kernel needs no scratch (no register spills); KVQ_RING_DEPTH=2|3|4
// overrides it.
template <class KF, class VF>
static const void* kernel_ptr(int depth) {
  if (depth == 2) return reinterpret_cast<const void*>(&decode_splitk_kernel<KF, VF, 2>);
  if (depth == 3) return reinterpret_cast<const void*>(&decode_splitk_kernel<KF, VF, 3>);
  return reinterpret_cast<const void*>(&decode_splitk_kernel<KF, VF, 4>);
}

template <class KF, class VF>
static int ring_depth() {
  static int d = [] {
    const char* e = getenv("KVQ_RING_DEPTH");
    if (e) {
      const int v = atoi(e);
      if (v >= 2 && v <= 4) return v;
    }
    for (int cand = 4; cand >= 2; --cand) {
      hipFuncAttributes at;
      if (hipFuncGetAttributes(&at, kernel_ptr<KF, VF>(cand)) == hipSuccess && at.localSizeBytes == 0)
        return cand;
    }
    (void)hipGetLastError();
    return 2;
  }();
  return d;
}

template <class KF, class VF>
static const void* selected_kernel() {
  return kernel_ptr<KF, VF>(ring_depth<KF, VF>());
}

// (k_format, v_format, scale dtype) -> kernel family; 0 means unsupported
enum Family { kNone = 0, kI8I8_16, kI8I8_32, kI4I4_16, kI4I4_32, kA4A4, kA4A4o, kI8A4_16, kI8A4_32,
              kKivi, kI8Kv, kMixedT8 };

// the KIVI family's formats: per-channel K / per-token V asymmetric codes, or fp16 values
static bool kivi_fmt(int f) {
  return f == KVQ_FMT_INT4_KIVI || f == KVQ_FMT_INT8_KIVI || f == KVQ_FMT_FP16;
}
// bytes of one token's row of a format
static int row_bytes_of(int f) {
  return f == KVQ_FMT_FP16 ? 2 * kD : (f == KVQ_FMT_INT8_SYM || f == KVQ_FMT_INT8_KIVI) ? kD : kD / 2;
}

static Family family(int kf, int vf, int ksf32, int vsf32, int kout) {
  if (kf == KVQ_FMT_INT8_SYM && vf == KVQ_FMT_INT8_SYM && ksf32 == vsf32)
    return ksf32 ? kI8I8_32 : kI8I8_16;
  if (kf == KVQ_FMT_INT4_SYM && vf == KVQ_FMT_INT4_SYM && ksf32 == vsf32)
    return ksf32 ? kI4I4_32 : kI4I4_16;
  if (kf == KVQ_FMT_INT4_ASYM && vf == KVQ_FMT_INT4_ASYM) return kout ? kA4A4o : kA4A4;
  if (kf == KVQ_FMT_INT8_SYM && vf == KVQ_FMT_INT4_ASYM) return ksf32 ? kI8A4_32 : kI8A4_16;
  if (kivi_fmt(kf) && kivi_fmt(vf)) return kKivi;  // tiled kernel only
  if (kf == KVQ_FMT_INT8_SYM && (vf == KVQ_FMT_INT4_KIVI || vf == KVQ_FMT_FP16))
    return kI8Kv;  // tiled kernel only
  // the reference's MixedKVCache (K INT4 per token, or fp16 K) with INT8 V: tiled kernel only
  if ((kf == KVQ_FMT_INT4_KIVI || kf == KVQ_FMT_FP16) && vf == KVQ_FMT_INT8_SYM && !vsf32)
    return kMixedT8;
  return kNone;
}

static const void* select_kernel(Family f) {
  switch (f) {
    case kI8I8_16: return selected_kernel<KTok<false, false>, VTok<false, false>>();
    case kI8I8_32: return selected_kernel<KTok<false, true>, VTok<false, true>>();
    case kI4I4_16: return selected_kernel<KTok<true, false>, VTok<true, false>>();
    case kI4I4_32: return selected_kernel<KTok<true, true>, VTok<true, true>>();
    case kA4A4: return selected_kernel<KAsym4<false>, VAsym4>();
    case kA4A4o: return selected_kernel<KAsym4<true>, VAsym4>();
    case kI8A4_16: return selected_kernel<KTok<false, false>, VAsym4>();
    case kI8A4_32: return selected_kernel<KTok<false, true>, VAsym4>();
    default: return nullptr;
  }
}

// work-groups of the selected kernel that fit on the device at once
static int64_t resident_slots(const void* fn, int threads) {
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, int64_t> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1024;
  std::lock_guard<std::mutex> g(mu);
  auto key = std::make_pair(fn, dev * 4096 + threads);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      per_cu <= 0 || cus <= 0) {
    (void)hipGetLastError();
    return 1024;
  }
  const int64_t slots = (int64_t)per_cu * cus;
  cache[key] = slots;
  return slots;
}

// The tiled kernel family that serves p, or kTiledNone (a row-layout kernel then does):
// INT4_ASYM K with TILE32 V, or INT8 K with a static scale (a view with stride 0 over b and t)
// and dense 128-byte rows, with TILE32 INT4_ASYM V or static-scale INT8 V in dense rows.
// A per-token scale view is static when it does not vary over b and t (stride 0, or a
// dimension of size 1, whose stride is never used).
static bool static_over_bt(const kvq_kv_view& v, const kvq_decode_params* p) {
  return (v.scale_stride_b == 0 || p->batch == 1) && (v.scale_stride_t == 0 || p->capacity <= 1);
}

// Per-token scales on both sides in dense token rows (static stride-0 views too): INT8 with
// fp16 scales or INT4_SYM with fp32 scales (the dtypes the engines store), groups of 16 or
// more, the groups of a token contiguous.  INT8 K with groups of 16 reads two fp16 scales in
// one 4-byte load, so its scale rows must be 4-byte aligned.
// INT8 K with per-token fp16 scales may also pair with per-token asymmetric INT4 V in the
// KIVI layout (the reference's MixedKVCache: K INT8 symmetric per group, V INT4 asymmetric
// per token).
// the group size of the V side's per-token scales (kvq_decode_params.v_group_size, ABI 6)
static int v_group(const kvq_decode_params* p) {
  return p->v_group_size > 0 ? p->v_group_size : p->group_size;
}

// a per-token INT4_KIVI K view (the reference's MixedKVCache K at 4 bits): fp32 parameters
// [B, H, T], tokens contiguous, no channel stride
static bool kivi_k_per_token(const kvq_kv_view& v) {
  return v.scale_stride_t == 1 && v.scale_stride_g == 0;
}

// the longest fp16 residual window: the merging work-group attends it with VALU dot products
// (16 tokens per batch), so its time grows with the window (about 1 us per 256 tokens)
constexpr int kMaxResidual = 65536;

// code rows whose every (b, head) slab starts 16-byte aligned: the V tiles can be read with
// 16-byte loads (the staged V operand types)
static bool rows16_aligned(const kvq_kv_view& v) {
  return ((uintptr_t)v.codes % 16) == 0 && v.stride_b % 16 == 0 && v.stride_h % 16 == 0;
}

static int tok_family(const kvq_decode_params* p) {
  if (p->v.layout != KVQ_LAYOUT_ROWS) return kTiledNone;
  const bool kivi_v = p->k_format == KVQ_FMT_INT8_SYM &&
                      (p->v_format == KVQ_FMT_INT4_KIVI || p->v_format == KVQ_FMT_FP16);
  if (p->k_format != p->v_format && !kivi_v) return kTiledNone;
  const bool i4 = p->k_format == KVQ_FMT_INT4_SYM;
  if (!i4 && p->k_format != KVQ_FMT_INT8_SYM) return kTiledNone;
  const int gs = p->group_size, vgs = v_group(p);
  if (gs < 16 || vgs < 16) return kTiledNone;
  if (vgs != gs && (i4 || p->v_format != KVQ_FMT_INT8_SYM)) return kTiledNone;
  const int64_t row = i4 ? kD / 2 : kD;
  const int dt = i4 ? KVQ_DTYPE_F32 : KVQ_DTYPE_F16;
  const int64_t es = i4 ? 4 : 2;
  // w: elements per aligned scale load (INT8 K with groups of 16 reads two fp16 at once)
  auto ok = [&](const kvq_kv_view& v, int g, int64_t w) {
    return v.stride_t == row && v.scale_dtype == dt && v.scale != nullptr &&
           (v.scale_stride_g == 1 || g == kD) && ((uintptr_t)v.scale % (w * es)) == 0 &&
           v.scale_stride_b % w == 0 && v.scale_stride_h % w == 0 && v.scale_stride_t % w == 0 &&
           v.scale_stride_b >= 0 && v.scale_stride_h >= 0 && v.scale_stride_t >= 0;
  };
  const int64_t wk = (!i4 && gs == 16) ? 2 : 1;
  if (kivi_v) {
    if (!ok(p->k, gs, wk)) return kTiledNone;
    if (p->v_format == KVQ_FMT_FP16)  // fp16 V in dense 256-byte rows
      return p->v.stride_t == 2 * kD ? (gs == 16 ? kTiledT8Fg16 : kTiledT8F) : kTiledNone;
    // V codes in dense 64-byte rows, fp32 scale / zero-point per token (checked by check_view)
    if (p->v.stride_t != kD / 2 || p->v.scale_stride_t != 1) return kTiledNone;
    if (rows16_aligned(p->v)) return gs == 16 ? kTiledT8Kvg16s : kTiledT8Kvs;
    return gs == 16 ? kTiledT8Kvg16 : kTiledT8Kv;
  }
  if (!ok(p->k, gs, wk) || !ok(p->v, vgs, i4 ? 1 : 1)) return kTiledNone;
  if (i4) {
    // groups of 16 or 32 in dense V scale rows (128 / gs fp32 per token, contiguous, rows
    // 16-byte aligned) and 16-byte aligned code rows: the tile is read with 16-byte loads and
    // gathered in LDS
    const kvq_kv_view& v = p->v;
    const int64_t ng = kD / vgs;
    const bool staged = vgs <= 32 && v.scale_stride_t == ng && v.scale_stride_g == 1 &&
                        ((uintptr_t)v.scale % 16) == 0 && (v.scale_stride_b * 4) % 16 == 0 &&
                        (v.scale_stride_h * 4) % 16 == 0 && rows16_aligned(v);
    if (staged) return gs == 16 ? kTiledT4g16s : kTiledT4s;
    return gs == 16 ? kTiledT4g16 : kTiledT4;
  }
  return gs == 16 ? kTiledT8g16 : kTiledT8;
}

// INT8_SYM V with per-token fp16 scales in dense rows (groups of 16 or more, contiguous) on
// the tiled kernel's VTokT, next to a K of another format
static bool tok8_v_ok(const kvq_decode_params* p) {
  const kvq_kv_view& v = p->v;
  const int vgs = v_group(p);
  return p->v_format == KVQ_FMT_INT8_SYM && v.layout == KVQ_LAYOUT_ROWS && v.stride_t == kD &&
         v.scale != nullptr && v.scale_dtype == KVQ_DTYPE_F16 && vgs >= 16 &&
         (v.scale_stride_g == 1 || vgs == kD) && v.scale_stride_b >= 0 && v.scale_stride_h >= 0 &&
         v.scale_stride_t >= 0;
}

static int tiled_family(const kvq_decode_params* p) {
  const bool vt = p->v.layout == KVQ_LAYOUT_TILE32;
  // the reference's MixedKVCache pairs with a per-token INT4 K, or fp16 K with INT8 V
  if (p->k_format == KVQ_FMT_INT4_KIVI && kivi_k_per_token(p->k)) {
    if (vt || p->k.stride_t != kD / 2) return kTiledNone;
    if (p->v_format == KVQ_FMT_INT4_KIVI)
      return (p->v.stride_t == kD / 2 && p->v.scale_stride_t == 1) ? kTiledKtKv : kTiledNone;
    if (p->v_format == KVQ_FMT_FP16) return p->v.stride_t == 2 * kD ? kTiledKtF : kTiledNone;
    return tok8_v_ok(p) ? kTiledKtT8 : kTiledNone;
  }
  if (p->k_format == KVQ_FMT_FP16 && p->v_format == KVQ_FMT_INT8_SYM)
    return (!vt && p->k.stride_t == 2 * kD && tok8_v_ok(p)) ? kTiledFT8 : kTiledNone;
  if (kivi_fmt(p->k_format)) {
    if (!kivi_fmt(p->v_format) || vt || p->k.stride_t != row_bytes_of(p->k_format) ||
        p->v.stride_t != row_bytes_of(p->v_format))
      return kTiledNone;
    const auto idx = [](int f) { return f == KVQ_FMT_INT4_KIVI ? 0 : f == KVQ_FMT_INT8_KIVI ? 1 : 2; };
    static const int fams[3][3] = {{kTiledKivi, kTiledKv48, kTiledKv4F},
                                   {kTiledKv84, kTiledKv88, kTiledKv8F},
                                   {kTiledKvF4, kTiledKvF8, kTiledKvFF}};
    const int fam = fams[idx(p->k_format)][idx(p->v_format)];
    return (fam == kTiledKivi && rows16_aligned(p->v)) ? kTiledKivis : fam;
  }
  if (p->k_format == KVQ_FMT_INT4_ASYM)
    return (p->v_format == KVQ_FMT_INT4_ASYM && vt) ? (p->k.n_outlier > 0 ? kTiledA4A4o : kTiledA4A4)
                                                     : kTiledNone;
  // static INT8 K with any group size (8 .. 128, checked by the caller); INT4_ASYM V
  // needs groups of 32, and the call has one group size for both sides
  const bool k8 = p->k_format == KVQ_FMT_INT8_SYM && static_over_bt(p->k, p) && p->k.stride_t == kD;
  if (k8 && p->v_format == KVQ_FMT_INT4_ASYM && vt)
    return p->group_size == kTile ? kTiledI8A4 : kTiledNone;
  if (k8 && p->v_format == KVQ_FMT_INT8_SYM && !vt && static_over_bt(p->v, p) && p->v.stride_t == kD)
    return p->group_size == kTile ? kTiledI8I8 : kTiledI8I8g;
  return tok_family(p);
}

// the split-K kernel kvq_decode_attn launches for p (nullptr if unsupported)
static const void* kernel_for(const kvq_decode_params* p) {
  const int fam = tiled_family(p);
  if (fam != kTiledNone) return tiled_kernel(fam, p->q_heads / p->kv_heads).fn;
  if (p->v.layout == KVQ_LAYOUT_TILE32) return nullptr;
  return select_kernel(family(p->k_format, p->v_format, p->k.scale_dtype == KVQ_DTYPE_F32,
                              p->v.scale_dtype == KVQ_DTYPE_F32, p->k.n_outlier > 0));
}

// waves per work-group of the split-K kernel kvq_decode_attn launches for p
static int waves_for(const kvq_decode_params* p) {
  return tiled_family(p) != kTiledNone ? kTiledWaves : kWaves;
}

// Tokens per work-group: fill every resident work-group slot exactly once when the
// context is long enough (one wave of work-groups, no tail), in multiples of the
// waves x 32 tokens one pass of the work-group covers, never below kMinChunk.  The tiled
// kernels cap it at kTiledMaxTiles tiles per wave: with many (b, kv head) units or ragged
// contexts that gives more, shorter work-groups, which the dispatcher spreads over the CUs
// (work-groups past a short context exit at once).  Measured on MI355X: 16 tiles per wave
// is the best split at configs 2, 3 (uniform 32k contexts) and 4 (ragged 4k-64k).
constexpr int kTiledMaxTiles = 16;
int32_t choose_chunk(const kvq_decode_params* p) {
  if (p->chunk_tokens > 0) return p->chunk_tokens;
  const int64_t units = (int64_t)p->batch * p->kv_heads;
  const void* fn = kernel_for(p);
  const int nw = waves_for(p);
  const int64_t slots = fn ? resident_slots(fn, nw * 64) : 1024;
  int64_t per_unit = slots / (units > 0 ? units : 1);
  if (per_unit < 1) per_unit = 1;
  int64_t c = (p->capacity + per_unit - 1) / per_unit;
  c = ((c + kTile * nw - 1) / (kTile * nw)) * (kTile * nw);
  if (tiled_family(p) != kTiledNone && c > (int64_t)kTiledMaxTiles * nw * kTile)
    c = (int64_t)kTiledMaxTiles * nw * kTile;
  if (c < kMinChunk) c = kMinChunk;
  const int64_t min_for_cap = (p->capacity + kMaxChunks - 1) / kMaxChunks;
  if (c < min_for_cap) c = ((min_for_cap + kTile - 1) / kTile) * kTile;
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
  d.layout = v.layout;
  return d;
}

static int check_view(const kvq_kv_view& v, int fmt, bool is_k, const char* name, int gs) {
  std::string n(name);
  if (!v.codes) return fail(KVQ_ERR_INVALID, n + ": codes is NULL");
  if (v.layout != KVQ_LAYOUT_ROWS && v.layout != KVQ_LAYOUT_TILE32)
    return fail(KVQ_ERR_INVALID, n + ": unknown layout");
  if (v.layout == KVQ_LAYOUT_TILE32) {
    if (is_k || fmt != KVQ_FMT_INT4_ASYM)
      return fail(KVQ_ERR_UNSUPPORTED, n + ": the TILE32 layout is for INT4_ASYM V only");
    if (v.stride_t != kD / 2)
      return fail(KVQ_ERR_INVALID, n + ": TILE32 needs stride_t == 64");
  }
  if (!v.scale && fmt != KVQ_FMT_FP16) return fail(KVQ_ERR_INVALID, n + ": scale is NULL");
  const int row_bytes = row_bytes_of(fmt);
  if (v.stride_t < row_bytes)
    return fail(KVQ_ERR_INVALID, n + ": token stride smaller than a code row");
  // lane byte offsets within a 32-token tile are 32-bit
  if (v.stride_t > ((int64_t)1 << 24) || v.outlier_stride_t > ((int64_t)1 << 22))
    return fail(KVQ_ERR_UNSUPPORTED, n + ": token stride too large");
  const int need = (is_k || fmt == KVQ_FMT_FP16) ? 16 : (row_bytes == kD ? 8 : 4);
  if (!aligned(v.codes, need) || v.stride_b % need || v.stride_h % need || v.stride_t % need)
    return fail(KVQ_ERR_UNSUPPORTED,
                n + ": code rows must be " + std::to_string(need) + "-byte aligned");
  if (fmt == KVQ_FMT_FP16) {
    if (v.layout != KVQ_LAYOUT_ROWS || v.stride_t != 2 * kD)
      return fail(KVQ_ERR_UNSUPPORTED, n + ": FP16 needs dense 256-byte token rows");
    if (v.n_outlier != 0) return fail(KVQ_ERR_UNSUPPORTED, n + ": outlier channels need INT4_ASYM");
    return KVQ_OK;
  }
  if (v.scale_dtype != KVQ_DTYPE_F16 && v.scale_dtype != KVQ_DTYPE_F32)
    return fail(KVQ_ERR_INVALID, n + ": scale_dtype must be F16 or F32");
  if (fmt == KVQ_FMT_INT4_KIVI || fmt == KVQ_FMT_INT8_KIVI) {
    if (v.layout != KVQ_LAYOUT_ROWS)
      return fail(KVQ_ERR_UNSUPPORTED, n + ": KIVI codes are in token rows");
    if (v.stride_t != row_bytes)
      return fail(KVQ_ERR_UNSUPPORTED, n + ": KIVI needs dense token rows (64 bytes INT4, 128 INT8)");
    if (v.scale_dtype != KVQ_DTYPE_F32 || !v.zero_point)
      return fail(KVQ_ERR_INVALID, n + ": KIVI needs fp32 scale and zero_point");
    if (v.n_outlier != 0) return fail(KVQ_ERR_UNSUPPORTED, n + ": outlier channels need INT4_ASYM");
    if (is_k && fmt == KVQ_FMT_INT4_KIVI && kivi_k_per_token(v)) {
      // per-token K: 4 tokens' parameters are read as one 16-byte vector
      if (!aligned(v.scale, 16) || !aligned(v.zero_point, 16) || v.scale_stride_b % 4 ||
          v.scale_stride_h % 4)
        return fail(KVQ_ERR_UNSUPPORTED, n + ": per-token K parameter rows must be 16-byte aligned");
    } else if (is_k) {
      // the 8 channels of a lane are read as two 16-byte vectors
      if (v.scale_stride_g != 1)
        return fail(KVQ_ERR_UNSUPPORTED, n + ": KIVI K parameters need contiguous channels");
      if (!aligned(v.scale, 16) || !aligned(v.zero_point, 16) || v.scale_stride_b % 4 ||
          v.scale_stride_h % 4)
        return fail(KVQ_ERR_UNSUPPORTED, n + ": KIVI K parameter rows must be 16-byte aligned");
    } else {
      if (v.scale_stride_t != 1)
        return fail(KVQ_ERR_UNSUPPORTED, n + ": KIVI V parameters need contiguous tokens");
      if (!aligned(v.scale, 4) || !aligned(v.zero_point, 4))
        return fail(KVQ_ERR_UNSUPPORTED, n + ": KIVI V parameters must be 4-byte aligned");
    }
    return KVQ_OK;
  }
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
  const int d = ring_depth<KF, VF>();
  if (d == 2)
    hipLaunchKernelGGL((decode_splitk_kernel<KF, VF, 2>), grid, dim3(kWaves * 64), 0, s, a);
  else if (d == 3)
    hipLaunchKernelGGL((decode_splitk_kernel<KF, VF, 3>), grid, dim3(kWaves * 64), 0, s, a);
  else
    hipLaunchKernelGGL((decode_splitk_kernel<KF, VF, 4>), grid, dim3(kWaves * 64), 0, s, a);
}

static int64_t n_chunks_for(const kvq_decode_params* p, int32_t chunk) {
  return p->capacity > 0 ? (p->capacity + chunk - 1) / chunk : 1;
}

// How a call is split.  Uniform split: every row gets u = capacity / chunk work-groups
// (grid (u, Hkv, B)).  With the tiled kernels, context lengths given per row (2..64 rows),
// no explicit chunk_tokens and u <= kUnitChunks, the grid is one dimension per kv head
// instead: rows of equal length still take u work-groups each, in the same chunks (so
// their bits are those of the uniform split), while a ragged batch shares the waves of
// share_c work-groups of the kv head, about one work-group per resident slot, out by
// length: row b gets a run of about t_b / T waves (at least one work-group's worth; t_b
// its tiles, T the smallest per-wave load that fits; see share_waves in decode_tiled.h),
// so every wave streams about the same number of tiles in one round.  pitch: partial
// slots per (b, query head): a run touches at most one work-group more than its length
// in work-groups (it need not start at a work-group boundary).
struct Split {
  int32_t chunk;
  int64_t grid_x, pitch, u, share_c;
  bool share;
};
constexpr int kShareMaxRows = 64;
static Split plan_split(const kvq_decode_params* p) {
  Split sp;
  sp.chunk = choose_chunk(p);
  sp.u = sp.grid_x = sp.pitch = n_chunks_for(p, sp.chunk);
  sp.share_c = 0;
  sp.share = false;
  if (tiled_family(p) != kTiledNone && p->context_lens != nullptr && p->chunk_tokens <= 0 &&
      p->batch >= 2 && p->batch <= kShareMaxRows && p->capacity > 0 && sp.u <= kUnitChunks) {
    const void* fn = tiled_kernel(tiled_family(p), p->q_heads / p->kv_heads).fn_share;
    const int64_t slots = fn ? resident_slots(fn, kTiledWaves * 64) : 256;
    int64_t c = slots / p->kv_heads;
    if (c < p->batch) c = p->batch;
    if (c > (int64_t)kUnitChunks * p->batch) c = (int64_t)kUnitChunks * p->batch;
    // a row's partials: one per work-group whose part of the row's run holds a tile, so at
    // most one per kTiledWaves tiles plus one, at most c, at most kUnitChunks (the device
    // caps a run at kTiledWaves * (kUnitChunks - 1) waves)
    const int64_t row_max = ((p->capacity + kTile - 1) / kTile + kTiledWaves - 1) / kTiledWaves + 1;
    int64_t share_pitch = c < kUnitChunks ? c : kUnitChunks;
    if (share_pitch > row_max) share_pitch = row_max;
    sp.share_c = c;
    sp.grid_x = c > sp.u * p->batch ? c : sp.u * p->batch;
    sp.pitch = share_pitch > sp.u ? share_pitch : sp.u;
    sp.share = true;
  }
  return sp;
}

}  // namespace kvq

using namespace kvq;

extern "C" int32_t kvq_decode_chunk_tokens(const kvq_decode_params* p) {
  return p ? choose_chunk(p) : 0;
}

// workspace: the counter slots [B, Hkv] x 128 bytes of the tiled kernel's single-launch
// merge (256-byte aligned size), then partial acc [B, Hq, n_chunks, 128] f32 and partial
// (m, l) [B, Hq, n_chunks] float2.  The counters come first so that their place depends
// only on B x Hkv: a zero-filled workspace can serve calls with other split counts.
static int64_t counter_bytes(const kvq_decode_params* p) {
  return (((int64_t)p->batch * p->kv_heads * kCtrSlotWords * 4 + 255) / 256) * 256;
}

// the n counter slots at ctr set to zero (a fill kernel rather than a memset, so that a
// call can be captured into a HIP graph)
static __global__ void clear_counts_kernel(uint32_t* ctr, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n * kCtrSlotWords;
       i += (int64_t)gridDim.x * blockDim.x)
    ctr[i] = 0u;
}
static int clear_arrival_counts(uint32_t* ctr, int64_t n, hipStream_t s) {
  const int64_t words = n * kCtrSlotWords;
  const int64_t blocks = (words + 255) / 256 < 1024 ? (words + 255) / 256 : 1024;
  hipLaunchKernelGGL(clear_counts_kernel, dim3((unsigned)blocks), dim3(256), 0, s, ctr, n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? KVQ_OK : fail(KVQ_ERR_LAUNCH, std::string("launch: ") + hipGetErrorString(e));
}

extern "C" int64_t kvq_decode_workspace_bytes(const kvq_decode_params* p) {
  if (!p) return 0;
  const int64_t rows = (int64_t)p->batch * p->q_heads * plan_split(p).pitch;
  return counter_bytes(p) + rows * (kD * 4 + 8) + 256;
}

// kvq_decode_attn, and with app != nullptr kvq_append_decode_attn (tiled path only; the
// row formats pass their two append sides in rk / rv)
static int decode_impl(const kvq_decode_params* p, const FusedAppend* app, kvq_stream_t stream,
                       const AppendDev* rk = nullptr, const AppendDev* rv = nullptr,
                       int fam_override = -1, bool clear_counts = false) {
  if (!p) return fail(KVQ_ERR_INVALID, "params is NULL");
  if (p->head_dim != kD) return fail(KVQ_ERR_UNSUPPORTED, "head_dim must be 128");
  if (p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0)
    return fail(KVQ_ERR_INVALID, "batch/q_heads/kv_heads must be positive");
  if (p->batch > 65535 || p->kv_heads > 65535 || p->q_heads > 65535)
    return fail(KVQ_ERR_UNSUPPORTED, "batch/head counts above 65535");
  if (p->q_heads % p->kv_heads)
    return fail(KVQ_ERR_INVALID, "q_heads must be a multiple of kv_heads");
  const int n_rep = p->q_heads / p->kv_heads;
  if (n_rep > 16) return fail(KVQ_ERR_UNSUPPORTED, "q_heads / kv_heads must be <= 16");
  const int gs = p->group_size;
  if (gs != 8 && gs != 16 && gs != 32 && gs != 64 && gs != 128)
    return fail(KVQ_ERR_UNSUPPORTED, "group_size must be 8, 16, 32, 64 or 128");
  const int vgs = v_group(p);
  if (p->v_group_size < 0 || (vgs != 8 && vgs != 16 && vgs != 32 && vgs != 64 && vgs != 128))
    return fail(KVQ_ERR_UNSUPPORTED, "v_group_size must be 0, 8, 16, 32, 64 or 128");
  if (p->capacity < 0 || p->capacity > (int64_t)1 << 30)
    return fail(KVQ_ERR_INVALID, "capacity out of range");
  if (!p->q || !p->out) return fail(KVQ_ERR_INVALID, "q/out is NULL");
  if (!p->context_lens && p->context_len < 0)
    return fail(KVQ_ERR_INVALID, "context_len must be >= 0 when context_lens is NULL");
  if (!aligned(p->q, 16) || p->q_stride_b % 8 || p->q_stride_h % 8)
    return fail(KVQ_ERR_UNSUPPORTED, "q rows must be 16-byte aligned");
  const int kf = p->k_format, vf = p->v_format;
  const Family fam = family(kf, vf, p->k.scale_dtype == KVQ_DTYPE_F32, p->v.scale_dtype == KVQ_DTYPE_F32,
                            p->k.n_outlier > 0);
  if (fam == kNone)
    return fail(KVQ_ERR_UNSUPPORTED,
                "unsupported (k_format, v_format) pair or mixed K/V scale dtypes");
  const int tfam = fam_override >= 0 ? fam_override : tiled_family(p);
  const bool tiled = tfam != kTiledNone;
  if (p->v.layout == KVQ_LAYOUT_TILE32 && !tiled)
    return fail(KVQ_ERR_UNSUPPORTED,
                "TILE32 V needs INT4_ASYM K or INT8 K with a static group-32 scale in dense rows");
  if (fam == kKivi && !tiled)
    return fail(KVQ_ERR_UNSUPPORTED,
                "KIVI-family K and V (INT4_KIVI, INT8_KIVI, FP16) need dense token rows");
  if (fam == kMixedT8 && !tiled)
    return fail(KVQ_ERR_UNSUPPORTED,
                "INT8 V with a per-token INT4 K or an fp16 K needs dense rows (per-token K "
                "parameters [B, H, T], fp16 V scales in groups of 16 or more)");
  if (fam == kI8Kv && !tiled)
    return fail(KVQ_ERR_UNSUPPORTED,
                "INT8 K with INT4_KIVI or FP16 V needs dense K rows with fp16 per-token scales "
                "(groups of 16 or more, contiguous) and dense V rows");
  if (tiled && p->k_format == KVQ_FMT_INT4_ASYM &&
      (p->k.stride_t != kD / 2 || (p->k.n_outlier && p->k.outlier_stride_t != 4)))
    return fail(KVQ_ERR_UNSUPPORTED, "with TILE32 V, K rows and outlier rows must be dense");
  // buffer loads address each (b, head) slab with 32-bit byte offsets
  if (tiled && (p->capacity + kTile) * (p->k.stride_t > p->v.stride_t ? p->k.stride_t : p->v.stride_t) >=
                   ((int64_t)1 << 31))
    return fail(KVQ_ERR_UNSUPPORTED, "capacity too large for one (b, head) slab");
  int rc = check_view(p->k, kf, true, "k", gs);
  if (rc) return rc;
  rc = check_view(p->v, vf, false, "v", vgs);
  if (rc) return rc;
  if (vgs != gs && !tiled)
    return fail(KVQ_ERR_UNSUPPORTED, "a V group size apart from K's needs per-token INT8 V on the "
                                     "tiled kernel (dense rows, groups of 16 or more)");

  const Split sp = plan_split(p);
  const int32_t chunk = sp.chunk;
  if (chunk <= 0 || chunk % kTile)
    return fail(KVQ_ERR_INVALID, "chunk_tokens must be a positive multiple of 32");
  const int64_t nch64 = sp.pitch;
  if (nch64 > kMaxChunks) return fail(KVQ_ERR_UNSUPPORTED, "too many chunks (raise chunk_tokens)");
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
  a.ctx_uniform = p->context_len;
  a.B = p->batch; a.Hq = p->q_heads; a.Hkv = p->kv_heads; a.n_rep = n_rep; a.gs = gs; a.vgs = vgs;
  a.cap = p->capacity;
  a.sm_log2e = p->sm_scale * kLog2e;
  a.chunk = chunk;
  a.n_chunks = (int)nch64;
  a.share = sp.share ? 1 : 0;
  a.u_chunks = (int)sp.u;
  a.share_c = (int)sp.share_c;
  a.strided = tiled ? 1 : 0;
  a.nw = waves_for(p);
  const int64_t rows = (int64_t)p->batch * p->q_heads * nch64;
  char* ws = reinterpret_cast<char*>(p->workspace);
  a.counters = reinterpret_cast<uint32_t*>(ws);
  a.part_acc = reinterpret_cast<float*>(ws + counter_bytes(p));
  a.part_ml = reinterpret_cast<float2*>(ws + counter_bytes(p) + rows * kD * 4);

  a.out = reinterpret_cast<half_t*>(p->out);
  a.o_sb = p->out_stride_b; a.o_sh = p->out_stride_h;

  a.res_k = a.res_v = nullptr;
  a.rsb = a.rsh = 0;
  a.res_n = 0;
  if (p->res_tokens != 0) {
    if (p->res_tokens < 0 || p->res_tokens > kMaxResidual)
      return fail(KVQ_ERR_INVALID, "res_tokens must lie in [0, " + std::to_string(kMaxResidual) + "]");
    if (!tiled || !kivi_fmt(kf) || !kivi_fmt(vf))
      return fail(KVQ_ERR_UNSUPPORTED,
                  "the fp16 residual window needs KIVI-family formats (INT4_KIVI, INT8_KIVI, FP16)");
    if (nch64 > kUnitChunks)
      return fail(KVQ_ERR_UNSUPPORTED, "the fp16 residual window needs at most 64 work-groups per "
                                       "(b, kv head) (raise chunk_tokens)");
    if (!p->res_k || !p->res_v) return fail(KVQ_ERR_INVALID, "res_k / res_v is NULL");
    if (!aligned(p->res_k, 4) || !aligned(p->res_v, 4) || p->res_stride_b % 2 || p->res_stride_h % 2 ||
        p->res_stride_b < 0 || p->res_stride_h < 0)
      return fail(KVQ_ERR_UNSUPPORTED, "residual rows must be 4-byte aligned");
    a.res_k = reinterpret_cast<const half_t*>(p->res_k);
    a.res_v = reinterpret_cast<const half_t*>(p->res_v);
    a.rsb = p->res_stride_b;
    a.rsh = p->res_stride_h;
    a.res_n = p->res_tokens;
  }

  a.app = FusedAppend{};
  a.ark = rk ? *rk : AppendDev{};
  a.arv = rv ? *rv : AppendDev{};
  if (app) {
    if (!tiled) return fail(KVQ_ERR_UNSUPPORTED, "the fused append needs a tiled-kernel format");
    a.app = *app;
  }

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  a.fused = tiled && nch64 <= kUnitChunks;
  if (clear_counts) {  // kvq_decode_attn_noalloc, after every check above has passed
    const int rc2 = clear_arrival_counts(a.counters, (int64_t)p->batch * p->kv_heads, s);
    if (rc2) return rc2;
  }
  if (tiled) {
    const dim3 grid = sp.share ? dim3((unsigned)sp.grid_x, (unsigned)p->kv_heads, 1u)
                               : dim3((unsigned)nch64, (unsigned)p->kv_heads, (unsigned)p->batch);
    const TiledFn k = tiled_kernel(tfam, a.n_rep);
    // the kernel's writer quantizes the formats it was built for
    if (rk && k.fn && (rk->fmt != k.kfmt || rv->fmt != k.vfmt))
      return fail(KVQ_ERR_UNSUPPORTED, "the fused append's formats differ from the kernel's");
    const hipError_t e = launch_tiled(a, k, grid, s);
    if (e != hipSuccess) return fail(KVQ_ERR_LAUNCH, std::string("launch: ") + hipGetErrorString(e));
    if (a.fused) return KVQ_OK;  // one launch: the last work-group of each (b, kv head) merged
  } else if (p->capacity > 0) {
    const dim3 grid((unsigned)nch64, (unsigned)p->kv_heads, (unsigned)p->batch);
    switch (fam) {
      case kI8I8_16: launch<KTok<false, false>, VTok<false, false>>(a, grid, s); break;
      case kI8I8_32: launch<KTok<false, true>, VTok<false, true>>(a, grid, s); break;
      case kI4I4_16: launch<KTok<true, false>, VTok<true, false>>(a, grid, s); break;
      case kI4I4_32: launch<KTok<true, true>, VTok<true, true>>(a, grid, s); break;
      case kA4A4: launch<KAsym4<false>, VAsym4>(a, grid, s); break;
      case kA4A4o: launch<KAsym4<true>, VAsym4>(a, grid, s); break;
      case kI8A4_16: launch<KTok<false, false>, VAsym4>(a, grid, s); break;
      case kI8A4_32: launch<KTok<false, true>, VAsym4>(a, grid, s); break;
      default: break;
    }
  }
  hipLaunchKernelGGL(combine_kernel, dim3(p->q_heads, p->batch), dim3(kD), 0, s, a,
                     vf == KVQ_FMT_INT4_ASYM ? 1 : 0);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(KVQ_ERR_LAUNCH, std::string("launch: ") + hipGetErrorString(e));
  return KVQ_OK;
}

extern "C" int kvq_decode_attn(const kvq_decode_params* p, kvq_stream_t stream) {
  return decode_impl(p, nullptr, stream);
}

// ---------------------------------------------------------------- no-allocation variant
//
// kvq_decode_attn_noalloc runs kvq_decode_attn with its split-K workspace (the chunk
// partials and the single-launch merge's arrival counters) in `scratch`, a file-scope
// device array every GPU holds once for the life of the process, instead of a
// caller-provided buffer.  In host code `scratch` names a host-side stand-in, not device
// memory: its device address is looked up with hipGetSymbolAddress, once per device with
// that device current, and only that address is ever passed to kernels.
constexpr int64_t kNoallocScratchBytes = (int64_t)16 << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, or null

// device address of `scratch` on device dev (looked up on the first call for dev)
int scratch_ptr(int dev, void** out) {
  if (dev < 0 || dev >= kMaxDevices) return fail(KVQ_ERR_UNSUPPORTED, "device ordinal above 63");
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return fail(KVQ_ERR_LAUNCH, "hipGetDevice failed");
    if (cur != dev && hipSetDevice(dev) != hipSuccess)
      return fail(KVQ_ERR_LAUNCH, "hipSetDevice failed");
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || !ptr)
      return fail(KVQ_ERR_LAUNCH, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return KVQ_OK;
}
}  // namespace

extern "C" int kvq_decode_attn_noalloc(const kvq_decode_params* p, kvq_stream_t stream) {
  if (!p) return fail(KVQ_ERR_INVALID, "params is NULL");
  // shapes kvq_decode_attn would reject are rejected before anything is enqueued
  if (p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0 || p->batch > 65535 ||
      p->q_heads > 65535 || p->kv_heads > 65535 || p->capacity < 0 ||
      p->capacity > ((int64_t)1 << 30))
    return decode_impl(p, nullptr, stream);
  const int64_t need = kvq_decode_workspace_bytes(p);
  if (need > kNoallocScratchBytes)
    return fail(KVQ_ERR_UNSUPPORTED,
                "kvq_decode_attn_noalloc: the split-K workspace of this call needs " +
                    std::to_string(need) + " bytes, above the fixed " +
                    std::to_string(kNoallocScratchBytes) +
                    "-byte scratch; raise chunk_tokens or call kvq_decode_attn with a workspace");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int dev = -1;
  if (s != nullptr) {
    if (hipStreamGetDevice(s, &dev) != hipSuccess) return fail(KVQ_ERR_INVALID, "invalid stream");
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return fail(KVQ_ERR_LAUNCH, "hipGetDevice failed");
  }
  void* ws = nullptr;
  int rc = scratch_ptr(dev, &ws);
  if (rc) return rc;
  kvq_decode_params q = *p;
  q.workspace = ws;
  q.workspace_bytes = kNoallocScratchBytes;
  // The counter slots this call's merge uses (the first B x Hkv x 128 bytes of the
  // workspace) are cleared by a fill kernel, enqueued by decode_impl once every argument
  // check has passed: a rejected call enqueues nothing.  (The array keeps what the previous
  // call, of any shape, left there.)
  return decode_impl(&q, nullptr, stream, nullptr, nullptr, -1, true);
}

// One new token per (b, kv head) appended to the cache p attends over, in the same launch.
// The append parameters must describe exactly that cache: the same code, outlier and
// static-table buffers with the same strides (so the kernel writes what it later reads).
static int check_fused_side(const kvq_append_params* x, const kvq_kv_view& v, int fmt,
                            const kvq_decode_params* p, bool is_k) {
  const std::string n(is_k ? "k_new" : "v_new");
  if (!x) return fail(KVQ_ERR_INVALID, n + " is NULL");
  if (x->format != fmt)
    return fail(KVQ_ERR_UNSUPPORTED, n + ": format differs from the decode call's");
  if (x->seq_new != 1) return fail(KVQ_ERR_UNSUPPORTED, n + ": the fused append takes one token");
  if (x->batch != p->batch || x->heads != p->kv_heads || x->head_dim != kD ||
      x->group_size != p->group_size)
    return fail(KVQ_ERR_INVALID, n + ": shape does not match the decode call");
  if (!x->x || ((uintptr_t)x->x % 4) || (x->x_stride_b % 2) || (x->x_stride_h % 2))
    return fail(KVQ_ERR_INVALID, n + ": x is NULL or its rows are not 4-byte aligned");
  if (x->write_pos < 0 || x->write_pos >= p->capacity)
    return fail(KVQ_ERR_INVALID, n + ": write_pos outside the cache capacity");
  if (x->codes != v.codes || x->codes_stride_b != v.stride_b || x->codes_stride_h != v.stride_h)
    return fail(KVQ_ERR_UNSUPPORTED, n + ": codes must be the buffer the decode call reads");
  if (x->codes_layout != v.layout || (v.layout == KVQ_LAYOUT_ROWS && x->codes_stride_t != v.stride_t))
    return fail(KVQ_ERR_UNSUPPORTED, n + ": codes layout differs from the decode call's");
  if (x->adaptive || x->mixed_rescue || x->rescue_quantile > 0.f || x->rescue_all || x->scale_out)
    return fail(KVQ_ERR_UNSUPPORTED, n + ": the fused append takes static scales only");
  if (!x->static_scale) return fail(KVQ_ERR_UNSUPPORTED, n + ": the fused append needs a static scale");
  if (fmt == KVQ_FMT_INT8_SYM) {
    // the append quantizes with its own table (as kvq_quant_append would); no side-band
    if (x->static_scale_dtype != KVQ_DTYPE_F16 && x->static_scale_dtype != KVQ_DTYPE_F32)
      return fail(KVQ_ERR_INVALID, n + ": static_scale_dtype must be F16 or F32");
    if (x->n_outlier) return fail(KVQ_ERR_UNSUPPORTED, n + ": outlier channels need INT4_ASYM");
    return KVQ_OK;
  }
  if (x->static_scale != v.scale || x->static_zp != v.zero_point ||
      x->static_scale_dtype != KVQ_DTYPE_F16 || x->static_stride_h != v.scale_stride_h ||
      x->static_stride_g != v.scale_stride_g)
    return fail(KVQ_ERR_UNSUPPORTED, n + ": static tables differ from the decode call's");
  if (x->n_outlier != v.n_outlier)
    return fail(KVQ_ERR_UNSUPPORTED, n + ": outlier channels differ from the decode call's");
  if (x->n_outlier &&
      (x->outlier_idx != v.outlier_idx || x->outlier_out != v.outlier_val ||
       x->oo_stride_b != v.outlier_stride_b || x->oo_stride_h != v.outlier_stride_h ||
       x->oo_stride_t != v.outlier_stride_t))
    return fail(KVQ_ERR_UNSUPPORTED, n + ": outlier buffers differ from the decode call's");
  return KVQ_OK;
}

// One side of the row formats' fused append (per-token INT8 / INT4 scales, the KIVI family,
// fp16 sides): the writer quantises it with the append kernel's arithmetic, into the
// buffers the decode call reads.
static int check_row_side(const kvq_append_params* x, const kvq_kv_view& v, int fmt,
                          const kvq_decode_params* p, bool is_k) {
  const std::string n(is_k ? "k_new" : "v_new");
  if (!x) return fail(KVQ_ERR_INVALID, n + " is NULL");
  if (x->format != fmt)
    return fail(KVQ_ERR_UNSUPPORTED, n + ": format differs from the decode call's");
  if (x->seq_new != 1) return fail(KVQ_ERR_UNSUPPORTED, n + ": the fused append takes one token");
  if (x->batch != p->batch || x->heads != p->kv_heads || x->head_dim != kD ||
      ((fmt == KVQ_FMT_INT8_SYM || fmt == KVQ_FMT_INT4_SYM) &&
       x->group_size != (is_k ? p->group_size : v_group(p))))
    return fail(KVQ_ERR_INVALID, n + ": shape does not match the decode call");
  if (x->write_pos < 0 || x->write_pos >= p->capacity)
    return fail(KVQ_ERR_INVALID, n + ": write_pos outside the cache capacity");
  if (x->codes != v.codes || x->codes_stride_b != v.stride_b || x->codes_stride_h != v.stride_h ||
      x->codes_stride_t != v.stride_t || x->codes_layout != v.layout)
    return fail(KVQ_ERR_UNSUPPORTED, n + ": codes must be the buffer the decode call reads");
  // the group rescue's threshold spans every row of the append: the writer wave finds it
  // itself from at most kRescueRows new rows when the walk from the top reaches it
  if (x->rescue_quantile > 0.f && !x->rescue_all && x->static_scale && fmt == KVQ_FMT_INT4_SYM &&
      (x->batch * x->heads > kRescueRows ||
       !rescue_walk_ok(x->rescue_quantile,
                       x->group_size > 0 ? x->batch * x->heads * (kD / x->group_size) : 0)))
    return fail(KVQ_ERR_UNSUPPORTED, n + ": the group rescue's threshold is beyond the writer "
                                         "wave (more than 32 rows, or ranks far from the top of "
                                         "the append's scales): use kvq_quant_append, then "
                                         "kvq_decode_attn");
  if (x->scale_out &&
      (x->scale_out != v.scale || x->scale_out_dtype != v.scale_dtype ||
       x->so_stride_b != v.scale_stride_b || x->so_stride_h != v.scale_stride_h ||
       x->so_stride_t != v.scale_stride_t ||
       ((fmt == KVQ_FMT_INT8_SYM || fmt == KVQ_FMT_INT4_SYM) && x->so_stride_g != v.scale_stride_g)))
    return fail(KVQ_ERR_UNSUPPORTED, n + ": scale_out must be the scales the decode call reads");
  if (kivi_fmt(fmt) && fmt != KVQ_FMT_FP16) {
    const bool ok = x->static_scale ? (x->static_scale == v.scale && x->static_zp == v.zero_point)
                                    : x->zp_out == v.zero_point;
    if (!ok)
      return fail(KVQ_ERR_UNSUPPORTED, n + ": KIVI parameters must be the ones the decode call reads");
  }
  return KVQ_OK;
}

extern "C" int kvq_append_decode_attn(const kvq_decode_params* p, const kvq_append_params* k_new,
                                      const kvq_append_params* v_new, kvq_stream_t stream) {
  if (!p) return fail(KVQ_ERR_INVALID, "params is NULL");
  int fam = tiled_family(p);
  bool spec = fam == kTiledA4A4 || fam == kTiledA4A4o || fam == kTiledI8A4 ||
              fam == kTiledI8I8 || fam == kTiledI8I8g;
  // per-token scale views of one row and one token look static to tiled_family; an append
  // that computes its scales (no static table, a scale policy or scale_out) takes the
  // per-token family's writer instead
  const auto table_append = [](const kvq_append_params* x) {
    return x && x->static_scale && !x->adaptive && !x->mixed_rescue && x->rescue_quantile <= 0.f &&
           !x->rescue_all && !x->scale_out;
  };
  if ((fam == kTiledI8I8 || fam == kTiledI8I8g) && !(table_append(k_new) && table_append(v_new))) {
    const int tf = tok_family(p);
    if (tf != kTiledNone) {
      fam = tf;
      spec = false;
    }
  }
  if (fam == kTiledNone)
    return fail(KVQ_ERR_UNSUPPORTED,
                "the fused append needs a tiled-kernel format: INT4_ASYM K with TILE32 V, "
                "static-scale INT8 K with TILE32 INT4_ASYM V or static-scale INT8 V rows, "
                "per-token INT8 / INT4 scales in dense rows (groups of 16 or more), or the "
                "KIVI family");
  if (!spec) {  // the row formats: the writer runs the append kernel's row quantizer
    int rc = check_row_side(k_new, p->k, p->k_format, p, true);
    if (rc) return rc;
    rc = check_row_side(v_new, p->v, p->v_format, p, false);
    if (rc) return rc;
    if (k_new->write_pos != v_new->write_pos)
      return fail(KVQ_ERR_INVALID, "k_new and v_new must share write_pos");
    AppendDev dk, dv;
    if ((rc = fill_dev(k_new, dk, "k_new"))) return rc;
    if ((rc = fill_dev(v_new, dv, "v_new"))) return rc;
    FusedAppend f{};
    f.kx = reinterpret_cast<const half_t*>(k_new->x);  // marks the fused call
    f.wpos = k_new->write_pos;
    return decode_impl(p, &f, stream, &dk, &dv, fam);
  }
  int rc = check_fused_side(k_new, p->k, p->k_format, p, true);
  if (rc) return rc;
  rc = check_fused_side(v_new, p->v, p->v_format, p, false);
  if (rc) return rc;
  if (k_new->write_pos != v_new->write_pos)
    return fail(KVQ_ERR_INVALID, "k_new and v_new must share write_pos");
  FusedAppend f{};
  f.kx = reinterpret_cast<const half_t*>(k_new->x);
  f.ksb = k_new->x_stride_b;
  f.ksh = k_new->x_stride_h;
  f.vx = reinterpret_cast<const half_t*>(v_new->x);
  f.vsb = v_new->x_stride_b;
  f.vsh = v_new->x_stride_h;
  f.wpos = k_new->write_pos;
  f.kstatus = k_new->status;
  f.vstatus = v_new->status;
  f.kst = k_new->static_scale;
  f.kst_f32 = k_new->static_scale_dtype == KVQ_DTYPE_F32;
  f.kst_sh = k_new->static_stride_h;
  f.kst_sg = k_new->static_stride_g;
  f.vst = v_new->static_scale;
  f.vst_f32 = v_new->static_scale_dtype == KVQ_DTYPE_F32;
  f.vst_sh = v_new->static_stride_h;
  f.vst_sg = v_new->static_stride_g;
  return decode_impl(p, &f, stream);
}

extern "C" const char* kvq_last_error(void) { return g_last_error.c_str(); }
extern "C" int32_t kvq_abi_version(void) { return 6; }

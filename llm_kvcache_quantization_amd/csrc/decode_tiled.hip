// Split-K decode attention for gfx950 over INT4_ASYM K (optional fp16 outlier
// channels) and INT4_ASYM V stored in the TILE32 layout.
//
// The work decomposition is that of decode_attn.hip: one work-group = 4 waves = one
// (batch b, kv head, chunk of tokens), the GQA heads of the kv head are the N = 16
// columns of v_mfma_f32_16x16x32_f16 and each wave walks 32-token tiles.  What is
// different is how the bytes get into registers and how cheaply they become fp16:
//
//  * K rows are dense (64 bytes per token) and so is the outlier side-band (8 bytes).
//  * Every cache read is a buffer load.  The (b, kv head) slab of each stream is a
//    wave-uniform buffer resource whose size bounds the reads (bytes past it read as
//    zero), the per-tile offset is a scalar and the per-lane offset is loop-invariant,
//    so the loop does no 64-bit address arithmetic on the vector ALU.
//  * V in the TILE32 layout stores, for each tile, the 32 bytes lane L needs for its PV
//    operand contiguously at L * 32: two dwordx4 loads per lane, fully coalesced.
//    Within a lane's 32 bytes, dword 2 p + k holds bytes (2k, 2k+1) of the lane's 4-byte
//    column slice for the two tokens of k-slot pair p.
//  * The 4 fp16 outlier channels of the 32 tokens of a tile (256 bytes) are fetched by
//    one dword load of the whole wave: lane (row, g) takes the channel pair g & 1 of
//    token 16 (g >> 1) + row, which is where the outlier MFMA of row block g >> 1
//    needs it.
//  * A packed dword becomes 8 fp16 operands with 5 ops: v_and_or_b32 with the masks
//    0x00F000F0 (high nibbles of bytes 0 and 2 -> 64 + n) and 0x000F000F (low nibbles
//    -> 1024 + n), then the same on the dword shifted right by 8 (bytes 1 and 3).
//    The two offsets are exact in fp16 and are removed in the bias (K) or the
//    epilogue (V): channel offsets 72 = 64 + 8 and 1032 = 1024 + 8.
//  * The q-dependent operands (q * s split into fp16 hi + lo, the bias) are built once
//    per work-group: wave j builds those of channel slice 8j..8j+7 of each group and
//    shares them through LDS.
//  * K and V tiles are fetched LOOK steps ahead of their use (register rings of
//    LOOK + 1 tiles); QK of tile i + 1 is issued before softmax / PV of tile i.  The
//    first tiles are requested before the q set-up.
//  * The n_chunks work-groups of a (b, kv head) interleave tile by tile, so the device
//    streams each slab front to back.  With at most kUnitChunks of them and n_rep <= 8
//    the last of them to finish merges their partials (no second launch; the arrival
//    counters live in the workspace, which must be zero-filled before its first use and
//    which every call leaves zero); otherwise combine_kernel does.
#include "decode_common.h"

#include <cstdlib>

namespace kvq {
namespace {

using rsrc_t = __amdgpu_buffer_rsrc_t;
constexpr int kBufNT = 2;               // cache-policy bits of the buffer loads: nt (streaming)
constexpr int kRsrcWord3 = 0x00020000;  // buffer descriptor word 3 for raw loads on gfx9 parts
constexpr int kRowK = kD / 2;           // bytes per token of packed K (dense rows)
constexpr int kRowO = 4 * 2;            // bytes per token of the fp16 outlier side-band
// a voffset past every slab (slabs are below 2^31 bytes): such a buffer load returns 0
constexpr uint32_t kOutOfRange = 0x80000000u;

// Raw buffer loads return 0 when voffset + the instruction offset is at or past the
// descriptor's byte size; soffset is added to the address but not range checked.  Every
// offset that may run past a buffer's end therefore goes into voffset.
__device__ __forceinline__ rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kRsrcWord3);
}
__device__ __forceinline__ u32x4 bload4(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(
      u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, kBufNT));
}
__device__ __forceinline__ uint32_t bload1(rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, kBufNT);
}

// Fused combine: the last work-group of a (b, kv head) to finish merges the partials of
// its n_rep heads, which the other work-groups of the launch stored write-through, and
// writes the output rows with combine_one's arithmetic.  Needs n_rep <= 8 and n_chunks <=
// kUnitChunks.  Thread t takes head h = t / 32 and channels 4 (t % 32) .. +3; the 32
// threads of a head are one half of a wave.  Every load is issued first: (m, l) of chunks
// t % 32 (+ 32) and one 16-byte acc load per chunk (kUnitBatch in flight), bypassing the
// non-coherent cache levels (sc1, as device-scope atomic loads).  The max and the
// denominator are reduced across the half-wave; the chunk weights reach the other lanes
// of the head through LDS.  Loads of chunks past nvalid (or heads past n_rep) use an
// offset past the descriptor's end and read 0.
constexpr int kBufSC1 = 16;  // cache-policy bits: sc1 (device-coherent load)
constexpr int kUnitBatch = 32;

struct UnitLds {
  float e[8][kUnitChunks];  // chunk weights exp2(m_c - M) of head h
};

// max / sum over the 32 lanes of a half-wave (lanes l and l ^ 1, ^ 2, .., ^ 16)
__device__ __forceinline__ float halfwave_max(float x) {
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  return x;
}
__device__ __forceinline__ float halfwave_sum(float x) {
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) x += __shfl_xor(x, o, 64);
  return x;
}

__device__ __forceinline__ void combine_unit(const DecodeArgs& a, UnitLds& sh, int b, int hkv,
                                             int nvalid) {
  static_assert(kUnitChunks == 64 && kUnitChunks % kUnitBatch == 0, "chunk tiling");
  const int t = threadIdx.x;
  const int h = t >> 5, dg = t & 31;
  const bool hv = h < a.n_rep;
  const int64_t row0 = ((int64_t)b * a.Hq + hkv * a.n_rep) * a.n_chunks;
  const rsrc_t r = buffer_rsrc(a.part_acc + row0 * kD, (uint32_t)(a.n_rep * a.n_chunks * kD * 4));
  const rsrc_t rml = buffer_rsrc(a.part_ml + row0, (uint32_t)(a.n_rep * a.n_chunks * 8));
  const uint32_t vbase = (uint32_t)((h * a.n_chunks * kD + 4 * dg) * 4);
  u32x4 av[kUnitBatch];
  auto issue = [&](int c0) {
#pragma unroll
    for (int c = 0; c < kUnitBatch; ++c) {
      const uint32_t voff =
          (hv && c0 + c < nvalid) ? vbase + (uint32_t)((c0 + c) * kD * 4) : kOutOfRange;
      av[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, kBufSC1));
    }
  };
  // (m, l) of chunks dg and dg + 32 of head h (m = -inf, l = 0 past nvalid)
  float m2[2], l2[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int c = dg + 32 * k;
    const bool ok = hv && c < nvalid;
    const uint32_t off = ok ? (uint32_t)((h * a.n_chunks + c) * 8) : kOutOfRange;
    const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rml, (int)off, 0, kBufSC1));
    m2[k] = ok ? __builtin_bit_cast(float, (uint32_t)v.x) : kNegInf;
    l2[k] = __builtin_bit_cast(float, (uint32_t)v.y);  // 0 when out of range
  }
  issue(0);
  const float M = halfwave_max(fmaxf(m2[0], m2[1]));
  float e2[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) e2[k] = m2[k] == kNegInf ? 0.f : fast_exp2(m2[k] - M);
  const float den = halfwave_sum(fmaf(e2[0], l2[0], e2[1] * l2[1]));
  sh.e[h][dg] = e2[0];
  sh.e[h][dg + 32] = e2[1];
  // the weights of head h were written by this half-wave: a wave-level LDS wait suffices
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  float num[4] = {0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < nvalid; c0 += kUnitBatch) {
    if (c0 > 0) issue(c0);
#pragma unroll
    for (int c = 0; c < kUnitBatch; ++c) {
      const float e = sh.e[h][c0 + c];  // 0 past nvalid
      // (uint32_t) makes the vector element an rvalue: this clang's __builtin_bit_cast of
      // an ext_vector element lvalue reads element 0 whatever the index
#pragma unroll
      for (int j = 0; j < 4; ++j)
        num[j] = fmaf(e, __builtin_bit_cast(float, (uint32_t)av[c][j]), num[j]);
    }
  }
  if (!hv) return;
  const int g = dg >> 3;  // quantisation group of channels 4 dg .. 4 dg + 3
  const float s = (float)reinterpret_cast<const half_t*>(a.v.scale)[hkv * a.v.ssh + g * a.v.ssg];
  const float z = (float)a.v.zp[hkv * a.v.ssh + g * a.v.ssg];
  half4v o;
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = (half_t)fmaf(s, num[j] / den - ((j & 1) ? 1032.0f : 72.0f), z);
  *reinterpret_cast<half4v*>(a.out + (int64_t)b * a.o_sb + (int64_t)(hkv * a.n_rep + h) * a.o_sh +
                             4 * dg) = o;
}

// 8 packed codes -> 8 fp16 operands in k-slot order [e0, e4, e1, e5, e2, e6, e3, e7]
// (e = element within the dword; byte k holds e = 2k in its high nibble), valued
// 64 + n for even e and 1024 + n for odd e.
__device__ __forceinline__ half8v unpack5(uint32_t w, const NibConsts& nc) {
  const uint32_t w8 = w >> 8;
  return pack8(and_or(w, nc.m_hi, nc.c64), and_or(w, nc.m_lo, nc.c1024),
               and_or(w8, nc.m_hi, nc.c64), and_or(w8, nc.m_lo, nc.c1024));
}
__host__ __device__ constexpr int slot_elem(int k) { return (k & 1) * 4 + (k >> 1); }
__host__ __device__ constexpr float slot_offset(int k) {  // operand offset + code offset 8
  return ((k >> 1) & 1) ? 1032.0f : 72.0f;
}

// LDS through which the 4 waves share the q-dependent K operands, and the scaled q rows
// from which the outlier operand is gathered
struct QShareLds {
  u32x4 qh[4][64];
  u32x4 ql[4][64];
  float bias[4][16];
  half_t qv[16][kD];  // q' of head column c (zero for padding columns)
};

// The q-side inputs of one lane: q[32 lg + 8 wave .. + 7] of head column lane % 16, its
// inverse temperature and the K scale / zero-point of group lg.  They are fetched before
// the first cache loads, so waiting for them does not wait for those (vmcnt counts loads
// in issue order).
struct QIn {
  u32x4 q;
  half_t tau, s, z;
  int4 oc;
};

// INT4 asymmetric K with static scale s / zero-point z per (kv head, group of 32).  With
// x = off + n and code c = n - 8 the logit is
//   sum_d q_d (s c_d + z) = sum_d (q_d s) x_d + sum_d q_d (z - (off_d + 8) s),
// q_d s is split exactly into fp16 hi + lo (both go through the MFMA) and the constant
// term is the accumulator's initial value.  Outlier channels (q zeroed in the main
// MFMAs) are added by one MFMA of the same shape whose operands are the 4 fp16
// outlier values and q' of those channels in the first two k-slots of each lane group.
template <bool OUT>
struct KAsymT {
  half8v qh[4];
  half8v qo;
  float bias;
  rsrc_t rk, ro;
  uint32_t vk, vo;
  bool olo;  // lane group 0 or 1 (row block 0 of the outlier operand)
  struct Raw {
    u32x4 w[2];
    uint32_t o;
  };

  // buffer resources and lane offsets (no dependence on q: runs before the first loads)
  __device__ void setup_addr(const DecodeArgs& a, int b, int hkv, int lane) {
    const int col = lane & 15, lg = lane >> 4;
    olo = lg < 2;
    const uint8_t* kb = a.k.codes + (int64_t)b * a.k.sb + (int64_t)hkv * a.k.sh;
    rk = buffer_rsrc(kb, (uint32_t)(a.cap * kRowK));
    vk = (uint32_t)(col * kRowK + 16 * lg);
    if constexpr (OUT) {
      const half_t* ob = a.k.oval + (int64_t)b * a.k.osb + (int64_t)hkv * a.k.osh;
      ro = buffer_rsrc(ob, (uint32_t)(a.cap * kRowO));
      vo = (uint32_t)((16 * (lg >> 1) + col) * kRowO + (lg & 1) * 4);
    }
  }

  // issues the loads of the q-side inputs (padding columns read head 0's row)
  __device__ void fetch_q(const DecodeArgs& a, int b, int hkv, int lane, int wave, QIn& in) const {
    const int col = lane & 15, lg = lane >> 4;
    const int hq = hkv * a.n_rep + (col < a.n_rep ? col : 0);
    in.q = *reinterpret_cast<const u32x4*>(q_row(a, b, hq) + 32 * lg + 8 * wave);
    in.tau = a.inv_tau != nullptr ? a.inv_tau[hq] : (half_t)1.0f;
    in.s = reinterpret_cast<const half_t*>(a.k.scale)[hkv * a.k.ssh + lg * a.k.ssg];
    in.z = a.k.zp[hkv * a.k.ssh + lg * a.k.ssg];
    in.oc = int4{-1, -1, -1, -1};
    if constexpr (OUT) {
      const int4 o = *reinterpret_cast<const int4*>(a.k.oidx + hkv * 4);
      in.oc = int4{min(max(o.x, 0), kD - 1), min(max(o.y, 0), kD - 1), min(max(o.z, 0), kD - 1),
                   min(max(o.w, 0), kD - 1)};
    }
  }

  // q-dependent operands of this wave's channel slice, shared through LDS
  __device__ void setup_q(const DecodeArgs& a, const QIn& in, int lane, int wave, QShareLds& sh) {
    const int col = lane & 15, lg = lane >> 4;
    const bool valid = col < a.n_rep;
    const bool has_tau = a.inv_tau != nullptr;
    // this wave builds the operands of channels 32 lg + 8 j + e, j = wave
    const int j = wave;
    const uint32_t qw[4] = {in.q.x, in.q.y, in.q.z, in.q.w};
    const float s = (float)in.s;
    const float z = (float)in.z;
    float part = 0.f;
    half_t vh[8], vl[8], qs[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const half2v h2 = as_h2(qw[e >> 1]);
      qs[e] = valid ? qscale((e & 1) ? h2.y : h2.x, in.tau, has_tau) : (half_t)0.0f;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = slot_elem(k);
      const int d = 32 * lg + 8 * j + e;
      const bool use = d != in.oc.x && d != in.oc.y && d != in.oc.z && d != in.oc.w;
      const float qd = use ? (float)qs[e] : 0.f;
      const float P = qd * s;  // exact: 11-bit x 11-bit significands
      const half_t hi = (half_t)P;
      const half_t lo = (half_t)(P - (float)hi);
      vh[k] = hi;
      vl[k] = lo;
      part += qd * z - slot_offset(k) * ((float)hi + (float)lo);
    }
    sh.qh[j][lane] = __builtin_bit_cast(u32x4, half8v{vh[0], vh[1], vh[2], vh[3], vh[4], vh[5], vh[6], vh[7]});
    sh.ql[j][lane] = __builtin_bit_cast(u32x4, half8v{vl[0], vl[1], vl[2], vl[3], vl[4], vl[5], vl[6], vl[7]});
    *reinterpret_cast<u32x4*>(&sh.qv[col][32 * lg + 8 * j]) =
        __builtin_bit_cast(u32x4, half8v{qs[0], qs[1], qs[2], qs[3], qs[4], qs[5], qs[6], qs[7]});
    part = wave_sum_xor_groups(part);
    if (lg == 0) sh.bias[j][col] = part;
  }

  // after the work-group barrier: pick up the operands all four waves built
  __device__ void finish_setup(const QShareLds& sh, const QIn& in, int lane) {
#pragma unroll
    for (int j = 0; j < 4; ++j) qh[j] = __builtin_bit_cast(half8v, sh.qh[j][lane]);
    const int col = lane & 15;
    bias = (sh.bias[0][col] + sh.bias[1][col]) + (sh.bias[2][col] + sh.bias[3][col]);
    const half_t h0 = (half_t)0.0f;
    qo = half8v{h0, h0, h0, h0, h0, h0, h0, h0};
    if constexpr (OUT) {
      // lane group lg supplies outlier channels 2 (lg & 1) and 2 (lg & 1) + 1
      const bool odd = ((lane >> 4) & 1) != 0;
      qo = half8v{sh.qv[col][odd ? in.oc.z : in.oc.x], sh.qv[col][odd ? in.oc.w : in.oc.y],
                  h0, h0, h0, h0, h0, h0};
    }
  }

  // rows of a partial last tile past the capacity read 0 (tok in voffset, range checked);
  // with !valid (wave-uniform) every load is out of range: it reads 0 and touches no memory
  __device__ __forceinline__ void load(int tok, bool valid, Raw& r) const {
    const uint32_t v = vk + (valid ? (uint32_t)tok * kRowK : kOutOfRange);
    r.w[0] = bload4(rk, v, 0);
    r.w[1] = bload4(rk, v + 16 * kRowK, 0);
    if constexpr (OUT) r.o = bload1(ro, vo + (valid ? (uint32_t)tok * kRowO : kOutOfRange), 0);
  }

  // logits of the tile's two 16-token row blocks (x0: tokens 4 lg + r, x1: 16 + 4 lg + r).
  // The lo halves of q * s are read from LDS at every tile (16 VGPRs fewer); qlo is the
  // lane's byte offset into them, made opaque by the caller so the reads stay in the loop.
  __device__ __forceinline__ void qk(const Raw& r, const QShareLds& sh, uint32_t qlo,
                                     const NibConsts& nc, float4v& x0, float4v& x1) const {
    float4v c0 = {bias, bias, bias, bias};
    float4v c1 = c0;
    if constexpr (OUT) {
      c0 = mfma16x16x32(pack8(olo ? r.o : 0u, 0u, 0u, 0u), qo, c0);
      c1 = mfma16x16x32(pack8(olo ? 0u : r.o, 0u, 0u, 0u), qo, c1);
    }
    const char* qlb = reinterpret_cast<const char*>(&sh.ql[0][0]) + qlo;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half8v lo = __builtin_bit_cast(half8v, *reinterpret_cast<const u32x4*>(qlb + j * 64 * 16));
      const half8v A0 = unpack5(r.w[0][j], nc);
      const half8v A1 = unpack5(r.w[1][j], nc);
      c0 = mfma16x16x32(A0, qh[j], c0);
      c1 = mfma16x16x32(A1, qh[j], c1);
      c0 = mfma16x16x32(A0, lo, c0);
      c1 = mfma16x16x32(A1, lo, c1);
    }
    x0 = c0;
    x1 = c1;
  }
};

// INT4 asymmetric V in the TILE32 layout.  acc[c] (c < 8) accumulates sum_t p16 * x for
// channel 8 col + c of the lane's d-row col, x = 64 + n (even c) or 1024 + n (odd c);
// combine_kernel applies out = s (acc / l - off) + z with off = 72 or 1032.
struct VAsymT {
  rsrc_t rv;
  uint32_t vv;
  struct Raw {
    u32x4 w[2];
  };

  __device__ void setup(const DecodeArgs& a, int b, int hkv, int lane) {
    const uint8_t* vb = a.v.codes + (int64_t)b * a.v.sb + (int64_t)hkv * a.v.sh;
    rv = buffer_rsrc(vb, (uint32_t)(((a.cap + kTile - 1) / kTile) * kTile * (kD / 2)));
    vv = (uint32_t)lane * 32u;
  }
  // whole tiles only: the descriptor spans ceil(capacity / 32) tiles; with !valid
  // (wave-uniform) voffset is out of range, so the loads read 0 and touch no memory
  __device__ __forceinline__ void load(int tok, bool valid, Raw& r) const {
    const uint32_t soff = valid ? (uint32_t)tok * (kD / 2) : 0u;  // tile index * 2048
    const uint32_t v = vv + (valid ? 0u : kOutOfRange);
    r.w[0] = bload4(rv, v, soff);
    r.w[1] = bload4(rv, v + 16u, soff);
  }
  __device__ __forceinline__ void mma(const Raw& r, half8v pb, float4v acc[8],
                                      const NibConsts& nc) const {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      // dword 2p + k of the lane: bytes (2k, 2k+1) of the two tokens of k-slot pair p
      const uint32_t a0 = k ? r.w[0].y : r.w[0].x, a1 = k ? r.w[0].w : r.w[0].z;
      const uint32_t a2 = k ? r.w[1].y : r.w[1].x, a3 = k ? r.w[1].w : r.w[1].z;
      const uint32_t s0 = a0 >> 8, s1 = a1 >> 8, s2 = a2 >> 8, s3 = a3 >> 8;
      acc[4 * k] = mfma16x16x32(pack8(and_or(a0, nc.m_hi, nc.c64), and_or(a1, nc.m_hi, nc.c64),
                                      and_or(a2, nc.m_hi, nc.c64), and_or(a3, nc.m_hi, nc.c64)),
                                pb, acc[4 * k]);
      acc[4 * k + 1] =
          mfma16x16x32(pack8(and_or(a0, nc.m_lo, nc.c1024), and_or(a1, nc.m_lo, nc.c1024),
                             and_or(a2, nc.m_lo, nc.c1024), and_or(a3, nc.m_lo, nc.c1024)),
                       pb, acc[4 * k + 1]);
      acc[4 * k + 2] = mfma16x16x32(pack8(and_or(s0, nc.m_hi, nc.c64), and_or(s1, nc.m_hi, nc.c64),
                                          and_or(s2, nc.m_hi, nc.c64), and_or(s3, nc.m_hi, nc.c64)),
                                    pb, acc[4 * k + 2]);
      acc[4 * k + 3] =
          mfma16x16x32(pack8(and_or(s0, nc.m_lo, nc.c1024), and_or(s1, nc.m_lo, nc.c1024),
                             and_or(s2, nc.m_lo, nc.c1024), and_or(s3, nc.m_lo, nc.c1024)),
                       pb, acc[4 * k + 3]);
    }
  }
};

// Fused quantize-on-append of the new token of (b, kv head): one wave, two values per
// lane, the arithmetic of the append kernel (asym_pack_pair with the decode's static
// tables).  K goes to row wpos, V to its TILE32 bytes, the outlier channels verbatim.
// NaN / Inf set status[0], clamped elements are added to status[1] (per side).
template <bool OUT>
__device__ __forceinline__ void append_token(const DecodeArgs& a, int b, int hkv, int lane) {
  const FusedAppend& f = a.app;
  const int64_t t = f.wpos;
  const int g = lane >> 4;  // group of channels 2 lane, 2 lane + 1
  const half_t* xk = f.kx + (int64_t)b * f.ksb + (int64_t)hkv * f.ksh;
  const half_t* xv = f.vx + (int64_t)b * f.vsb + (int64_t)hkv * f.vsh;
  const half2v k2 = *reinterpret_cast<const half2v*>(xk + 2 * lane);
  const half2v v2 = *reinterpret_cast<const half2v*>(xv + 2 * lane);
  const half_t* ks = reinterpret_cast<const half_t*>(a.k.scale);
  const half_t* vs = reinterpret_cast<const half_t*>(a.v.scale);
  int kclip = 0, vclip = 0;
  const uint8_t kb = asym_pack_pair((float)k2.x, (float)k2.y, (float)ks[hkv * a.k.ssh + g * a.k.ssg],
                                    (float)a.k.zp[hkv * a.k.ssh + g * a.k.ssg], kclip);
  const uint8_t vb = asym_pack_pair((float)v2.x, (float)v2.y, (float)vs[hkv * a.v.ssh + g * a.v.ssg],
                                    (float)a.v.zp[hkv * a.v.ssh + g * a.v.ssg], vclip);
  uint8_t* kc = const_cast<uint8_t*>(a.k.codes) + (int64_t)b * a.k.sb + (int64_t)hkv * a.k.sh;
  uint8_t* vc = const_cast<uint8_t*>(a.v.codes) + (int64_t)b * a.v.sb + (int64_t)hkv * a.v.sh;
  kc[t * a.k.st + lane] = kb;
  vc[tile32_offset(t, lane)] = vb;
  if constexpr (OUT) {
    if (lane < 4) {
      const int ch = min(max(a.k.oidx[hkv * 4 + lane], 0), kD - 1);
      half_t* orow = const_cast<half_t*>(a.k.oval) + (int64_t)b * a.k.osb + (int64_t)hkv * a.k.osh +
                     t * a.k.ost;
      orow[lane] = xk[ch];
    }
  }
  const bool kbad = !(__builtin_isfinite((float)k2.x) && __builtin_isfinite((float)k2.y));
  const bool vbad = !(__builtin_isfinite((float)v2.x) && __builtin_isfinite((float)v2.y));
  const bool any_kbad = __ballot(kbad) != 0, any_vbad = __ballot(vbad) != 0;
  kclip = wave_sum_int(kclip);
  vclip = wave_sum_int(vclip);
  if (lane == 0) {
    if (f.kstatus) {
      if (any_kbad) atomicOr(&f.kstatus[0], 1);
      if (kclip) atomicAdd(&f.kstatus[1], kclip);
    }
    if (f.vstatus) {
      if (any_vbad) atomicOr(&f.vstatus[0], 1);
      if (vclip) atomicAdd(&f.vstatus[1], vclip);
    }
  }
}

template <bool OUT, int LOOK, bool PACK8, int WPE = 3>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(WPE)))
void decode_tiled_kernel(DecodeArgs a) {
  const int chunk = blockIdx.x, hkv = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, lg = lane >> 4;

  // Fused quantize-on-append: the wave whose schedule holds the new token's tile (below)
  // writes it before it issues any load, so its loads of that tile, later in program
  // order and to the same addresses, read the new codes.  (The tile may lie past the
  // context, and that wave's work-group may then have nothing else to do.)
  if (a.app.kx != nullptr &&
      chunk * kWaves + wave == (int)((a.app.wpos / kTile) % (a.n_chunks * kWaves)))
    append_token<OUT>(a, b, hkv, lane);

  int64_t ctx64 = a.ctx[b];
  ctx64 = ctx64 < 0 ? 0 : (ctx64 > a.cap ? a.cap : ctx64);
  const int ctx = (int)ctx64;
  // The n_chunks work-groups of a (b, kv head) interleave: at step i the waves of all of
  // them read one contiguous run of n_chunks * kWaves tiles, so the device streams each
  // slab front to back.  Wave w of work-group c takes tiles c*kWaves + w + i*stride.
  const int ntot = (ctx + kTile - 1) / kTile;
  if (ntot == 0) {  // empty context: the first work-group writes zero rows
    if (chunk == 0 && a.fused)
      for (int idx = threadIdx.x; idx < a.n_rep * kD; idx += kWaves * 64)
        a.out[(int64_t)b * a.o_sb + (int64_t)(hkv * a.n_rep + (idx >> 7)) * a.o_sh +
              (idx & (kD - 1))] = (half_t)0.0f;
    return;
  }
  if (chunk * kWaves >= ntot) return;  // no tile for this work-group (uniform)

  __shared__ QShareLds qsh;
  __shared__ MergeLds msh;
  KAsymT<OUT> kf;
  // the q-side inputs are requested first: the wait for them then does not include the
  // cache tiles requested next
  QIn qin;
  kf.fetch_q(a, b, hkv, lane, wave, qin);
  kf.setup_addr(a, b, hkv, lane);
  VAsymT vf;
  vf.setup(a, b, hkv, lane);

  // Tile schedule: the n_chunks work-groups of a (b, kv head) interleave, so at step i the
  // waves of all of them read one contiguous run of n_chunks * kWaves tiles and the device
  // streams each slab front to back.  Wave w of work-group c takes tiles c * kWaves + w +
  // i * stride (tile = 32 tokens; only the context's last tile, ntot - 1, may be partial).
  // The schedule is static, so results do not depend on timing.
  const int first = chunk * kWaves + wave;
  const int stride = a.n_chunks * kWaves;
  const bool partial = (ctx & (kTile - 1)) != 0;
  // tile[j] = tile of step i + j (j <= LOOK + 1)
  int tile[LOOK + 2];
#pragma unroll
  for (int j = 0; j <= LOOK; ++j) tile[j] = first + j * stride;
  constexpr int R = LOOK + 1;                 // ring slots per stream
  constexpr int U = (R % 2 == 0) ? R : 2 * R;  // unroll: ring slot and x buffer are static
  typename KAsymT<OUT>::Raw kr[R];
  VAsymT::Raw vr[R];
  // K tiles of steps 0..LOOK and V tiles of steps 0..LOOK-1 are requested before the q
  // set-up, so the memory system is busy from the start of the kernel.  Every ring load is
  // issued unconditionally (out of range for a tile past the context): conditional loads
  // would make the compiler's vmcnt waits conservative at the joins, i.e. wait for the
  // tiles just requested.
#ifdef KVQ_EXP_QWAIT
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#else
  asm volatile("" ::: "memory");
#endif
#pragma unroll
  for (int s = 0; s <= LOOK; ++s) {
    kf.load(kTile * tile[s], tile[s] < ntot, kr[s]);
    if (s < LOOK) vf.load(kTile * tile[s], tile[s] < ntot, vr[s]);
  }
  kf.setup_q(a, qin, lane, wave, qsh);
  NibConsts nc;
  nc.init();
  __syncthreads();
  kf.finish_setup(qsh, qin, lane);

  float4v acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = float4v{0.f, 0.f, 0.f, 0.f};
  float m = kNegInf, l = 0.f;
  const float sm = a.sm_log2e;
  if (tile[0] < ntot) {
    float4v x[2][2];
    kf.qk(kr[0], qsh, (uint32_t)lane * 16u, nc, x[0][0], x[0][1]);
    while (tile[0] < ntot) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        // step i (i % U == u): the tiles of this wave form a prefix of its schedule
        if (tile[0] >= ntot) break;
        tile[LOOK + 1] = tile[LOOK] + stride;
        // fetch K of step i + LOOK + 1 (into the slot K of step i used) and V of step
        // i + LOOK (into the slot V of step i - 1 used), QK of step i + 1, then softmax
        // and PV of step i
        kf.load(kTile * tile[LOOK + 1], tile[LOOK + 1] < ntot, kr[u % R]);
        vf.load(kTile * tile[LOOK], tile[LOOK] < ntot, vr[(u + LOOK) % R]);
        if (tile[1] < ntot) {
          uint32_t qlo = (uint32_t)lane * 16u;
          asm volatile("" : "+v"(qlo));
          kf.qk(kr[(u + 1) % R], qsh, qlo, nc, x[(u + 1) & 1][0], x[(u + 1) & 1][1]);
        }
        float4v x0 = x[u & 1][0], x1 = x[u & 1][1];
        if (partial && tile[0] == ntot - 1) mask_tile(x0, x1, kTile * tile[0], ctx, lg);
        half8v pb;
        if constexpr (PACK8) pb = softmax_tile8(x0, x1, sm, m, l, acc);
        else pb = softmax_tile(x0, x1, sm, m, l, acc);
        vf.mma(vr[u % R], pb, acc, nc);
#pragma unroll
        for (int j = 0; j <= LOOK; ++j) tile[j] = tile[j + 1];
      }
    }
  }
  merge_and_store<PACK8, true>(a, msh, wave, col, lg, m, l, acc, b, hkv, chunk);

  // Fused combine.  The partials were stored write-through; once every store of the
  // work-group has completed, one thread counts the work-group in.  The last of the
  // (b, kv head)'s work-groups merges all partials and resets the counter.
  if (!a.fused) return;  // combine_kernel merges
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __shared__ int is_last;
  __shared__ UnitLds ush;
  const int nvalid = valid_chunks(a, ctx);
  uint32_t* counter = a.counters + ((int64_t)b * a.Hkv + hkv) * kCtrSlotWords;
  if (threadIdx.x == 0)
    is_last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              (uint32_t)(nvalid - 1);
  __syncthreads();
  if (!is_last) return;
  combine_unit(a, ush, b, hkv, nvalid);
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool OUT, bool PACK8>
const void* tiled_ptr(int look) {
  if (look == 2) return reinterpret_cast<const void*>(&decode_tiled_kernel<OUT, 2, PACK8>);
  return reinterpret_cast<const void*>(&decode_tiled_kernel<OUT, 1, PACK8>);
}

// Tiles of lookahead: 1 (measured fastest at the headline shape: both variants keep 3
// waves per SIMD, and the deeper ring spills), or KVQ_TILED_LOOK=1|2.
int tiled_look() {
  static int d = [] {
    const char* e = getenv("KVQ_TILED_LOOK");
    const int v = e ? atoi(e) : 1;
    return (v == 1 || v == 2) ? v : 1;
  }();
  return d;
}

template <bool OUT, bool PACK8>
void launch_one(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  const dim3 block(kWaves * 64);
  if (tiled_look() == 2)
    hipLaunchKernelGGL((decode_tiled_kernel<OUT, 2, PACK8>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((decode_tiled_kernel<OUT, 1, PACK8>), grid, block, 0, s, a);
}

}  // namespace

// the kernels for n_rep <= 8 pack the second row block's softmax into the padding lanes
const void* tiled_kernel(int kf, int kout, int n_rep) {
  if (kf != KVQ_FMT_INT4_ASYM) return nullptr;
  const bool p8 = n_rep <= 8;
  if (kout) return p8 ? tiled_ptr<true, true>(tiled_look()) : tiled_ptr<true, false>(tiled_look());
  return p8 ? tiled_ptr<false, true>(tiled_look()) : tiled_ptr<false, false>(tiled_look());
}

void launch_tiled(const DecodeArgs& a, int kf, int kout, dim3 grid, hipStream_t s) {
  (void)kf;
  const bool p8 = a.n_rep <= 8;
  if (kout) {
    if (p8) launch_one<true, true>(a, grid, s);
    else launch_one<true, false>(a, grid, s);
  } else {
    if (p8) launch_one<false, true>(a, grid, s);
    else launch_one<false, false>(a, grid, s);
  }
}

}  // namespace kvq

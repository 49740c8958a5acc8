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
// kUnitChunks.  Thread t takes head t / 32 and channels 4 (t % 32) .. +3: one 16-byte
// load per chunk, all issued at once, bypassing the non-coherent cache levels (sc1, as
// device-scope atomic loads).  The (m, l) pairs go through LDS.  Loads of chunks past
// nvalid (or heads past n_rep) use an offset past the descriptor's end and read 0.
constexpr int kBufSC1 = 16;  // cache-policy bits: sc1 (device-coherent load)

struct UnitLds {
  float2 ml[8][32];
};

__device__ __forceinline__ void combine_unit(const DecodeArgs& a, UnitLds& sh, int b, int hkv,
                                             int nvalid) {
  const int t = threadIdx.x;
  const int h = t >> 5, dg = t & 31;
  const bool hv = h < a.n_rep;
  const int64_t row0 = ((int64_t)b * a.Hq + hkv * a.n_rep) * a.n_chunks;
  const rsrc_t r = buffer_rsrc(a.part_acc + row0 * kD, (uint32_t)(a.n_rep * a.n_chunks * kD * 4));
  const uint32_t vbase = (uint32_t)((h * a.n_chunks * kD + 4 * dg) * 4);
  u32x4 av[kUnitChunks];
#pragma unroll
  for (int c = 0; c < kUnitChunks; ++c) {
    const uint32_t voff = (hv && c < nvalid) ? vbase + (uint32_t)(c * kD * 4) : 0x80000000u;
    av[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, kBufSC1));
  }
  {
    float m = kNegInf, l = 0.f;
    if (hv && dg < nvalid) {
      const float* pm =
          reinterpret_cast<const float*>(a.part_ml + row0 + (int64_t)h * a.n_chunks + dg);
      m = __hip_atomic_load(pm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      l = __hip_atomic_load(pm + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    sh.ml[h][dg] = float2{m, l};
  }
  __syncthreads();
  if (!hv) return;
  float M = kNegInf;
#pragma unroll
  for (int c = 0; c < kUnitChunks; ++c) M = fmaxf(M, sh.ml[h][c].x);
  float num[4] = {0.f, 0.f, 0.f, 0.f}, den = 0.f;
#pragma unroll
  for (int c = 0; c < kUnitChunks; ++c) {
    const float2 ml = sh.ml[h][c];
    const float e = fast_exp2(ml.x - M);
    // (uint32_t) makes the vector element an rvalue: this clang's __builtin_bit_cast of an
    // ext_vector element lvalue reads element 0 whatever the index
#pragma unroll
    for (int j = 0; j < 4; ++j)
      num[j] = fmaf(e, __builtin_bit_cast(float, (uint32_t)av[c][j]), num[j]);
    den = fmaf(e, ml.y, den);
  }
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

// LDS through which the 4 waves share the q-dependent K operands
struct QShareLds {
  u32x4 qh[4][64];
  u32x4 ql[4][64];
  float bias[4][16];
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
  half8v qh[4], ql[4];
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

  // q-dependent operands of this wave's channel slice, shared through LDS
  __device__ void setup_q(const DecodeArgs& a, int b, int hkv, int lane, int wave, QShareLds& sh) {
    const int col = lane & 15, lg = lane >> 4;
    const bool valid = col < a.n_rep;
    const int hq = hkv * a.n_rep + (valid ? col : 0);
    const bool has_tau = a.inv_tau != nullptr;
    const half_t tau = has_tau ? a.inv_tau[hq] : (half_t)1.0f;
    const half_t* qr = q_row(a, b, hq);
    int oc[4] = {-1, -1, -1, -1};
    if constexpr (OUT) {
      const int4 o = *reinterpret_cast<const int4*>(a.k.oidx + hkv * 4);
      oc[0] = min(max(o.x, 0), kD - 1);
      oc[1] = min(max(o.y, 0), kD - 1);
      oc[2] = min(max(o.z, 0), kD - 1);
      oc[3] = min(max(o.w, 0), kD - 1);
    }
    // this wave builds the operands of channels 32 lg + 8 j + e, j = wave
    const int j = wave;
    const u32x4 qraw = *reinterpret_cast<const u32x4*>(qr + 32 * lg + 8 * j);
    const uint32_t qw[4] = {qraw.x, qraw.y, qraw.z, qraw.w};
    const half_t* sc = reinterpret_cast<const half_t*>(a.k.scale);
    const float s = (float)sc[hkv * a.k.ssh + lg * a.k.ssg];
    const float z = (float)a.k.zp[hkv * a.k.ssh + lg * a.k.ssg];
    float part = 0.f;
    half_t vh[8], vl[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = slot_elem(k);
      const int d = 32 * lg + 8 * j + e;
      const half2v h2 = as_h2(qw[e >> 1]);
      const half_t qe = qscale((e & 1) ? h2.y : h2.x, tau, has_tau);
      const bool use = valid && d != oc[0] && d != oc[1] && d != oc[2] && d != oc[3];
      const float qd = use ? (float)qe : 0.f;
      const float P = qd * s;  // exact: 11-bit x 11-bit significands
      const half_t hi = (half_t)P;
      const half_t lo = (half_t)(P - (float)hi);
      vh[k] = hi;
      vl[k] = lo;
      part += qd * z - slot_offset(k) * ((float)hi + (float)lo);
    }
    sh.qh[j][lane] = __builtin_bit_cast(u32x4, half8v{vh[0], vh[1], vh[2], vh[3], vh[4], vh[5], vh[6], vh[7]});
    sh.ql[j][lane] = __builtin_bit_cast(u32x4, half8v{vl[0], vl[1], vl[2], vl[3], vl[4], vl[5], vl[6], vl[7]});
    part = wave_sum_xor_groups(part);
    if (lg == 0) sh.bias[j][col] = part;
    const half_t h0 = (half_t)0.0f;
    qo = half8v{h0, h0, h0, h0, h0, h0, h0, h0};
    if constexpr (OUT) {
      const int i0 = 2 * (lg & 1);
      const half_t o0 = valid ? qscale(qr[oc[i0]], tau, has_tau) : h0;
      const half_t o1 = valid ? qscale(qr[oc[i0 + 1]], tau, has_tau) : h0;
      qo = half8v{o0, o1, h0, h0, h0, h0, h0, h0};
    }
  }

  // after the work-group barrier: pick up the operands all four waves built
  __device__ void finish_setup(const QShareLds& sh, int lane) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qh[j] = __builtin_bit_cast(half8v, sh.qh[j][lane]);
      ql[j] = __builtin_bit_cast(half8v, sh.ql[j][lane]);
    }
    const int col = lane & 15;
    bias = (sh.bias[0][col] + sh.bias[1][col]) + (sh.bias[2][col] + sh.bias[3][col]);
  }

  // rows of a partial last tile past the capacity read 0 (tok in voffset, range checked)
  __device__ __forceinline__ void load(int tok, Raw& r) const {
    const uint32_t v = vk + (uint32_t)tok * kRowK;
    r.w[0] = bload4(rk, v, 0);
    r.w[1] = bload4(rk, v + 16 * kRowK, 0);
    if constexpr (OUT) r.o = bload1(ro, vo + (uint32_t)tok * kRowO, 0);
  }

  __device__ __forceinline__ float4v qk(const Raw& r, int s, const NibConsts& nc) const {
    float4v c = {bias, bias, bias, bias};
    if constexpr (OUT) {
      const uint32_t w = (olo == (s == 0)) ? r.o : 0u;
      c = mfma16x16x32(pack8(w, 0u, 0u, 0u), qo, c);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half8v A = unpack5(r.w[s][j], nc);
      c = mfma16x16x32(A, qh[j], c);
      c = mfma16x16x32(A, ql[j], c);
    }
    return c;
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
  // whole tiles only: the descriptor spans ceil(capacity / 32) tiles
  __device__ __forceinline__ void load(int tok, Raw& r) const {
    const uint32_t soff = (uint32_t)tok * (kD / 2);  // tile index * 2048
    r.w[0] = bload4(rv, vv, soff);
    r.w[1] = bload4(rv, vv + 16u, soff);
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

template <bool OUT, int LOOK, bool PACK8>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(3)))
void decode_tiled_kernel(DecodeArgs a) {
  const int chunk = blockIdx.x, hkv = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, lg = lane >> 4;

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
  kf.setup_addr(a, b, hkv, lane);
  VAsymT vf;
  vf.setup(a, b, hkv, lane);

  // This wave's tiles start at tokens tw + i * kStep, i < ntiles; only the context's
  // last tile may be partial.
  const int first = chunk * kWaves + wave;
  const int stride = a.n_chunks * kWaves;
  const int ntiles = first < ntot ? (ntot - first + stride - 1) / stride : 0;
  const int tw = kTile * first;
  const int kStep = kTile * stride;
  const int t1 = ctx;
  const bool partial = ntiles > 0 && tw + (ntiles - 1) * kStep + kTile > t1;
  constexpr int R = LOOK + 1;                 // ring slots per stream
  constexpr int U = (R % 2 == 0) ? R : 2 * R;  // unroll: ring slot and x buffer are static
  typename KAsymT<OUT>::Raw kr[R];
  VAsymT::Raw vr[R];
  // K tiles 0..LOOK and V tiles 0..LOOK-1 are requested before the q set-up, so the
  // memory system is busy from the start of the kernel
#pragma unroll
  for (int s = 0; s <= LOOK; ++s) {
    if (s < ntiles) kf.load(tw + s * kStep, kr[s]);
    if (s < LOOK && s < ntiles) vf.load(tw + s * kStep, vr[s]);
  }
  kf.setup_q(a, b, hkv, lane, wave, qsh);
  NibConsts nc;
  nc.init();
  __syncthreads();
  kf.finish_setup(qsh, lane);

  float4v acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = float4v{0.f, 0.f, 0.f, 0.f};
  float m = kNegInf, l = 0.f;
  const float sm = a.sm_log2e;
  if (ntiles > 0) {
    float4v x[2][2];
    x[0][0] = kf.qk(kr[0], 0, nc);
    x[0][1] = kf.qk(kr[0], 1, nc);
    for (int i0 = 0; i0 < ntiles; i0 += U) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u;
        if (i >= ntiles) break;
        // step i: fetch K of tile i + LOOK + 1 (into the slot K of tile i used) and V of
        // tile i + LOOK (into the slot V of tile i - 1 used), QK of tile i + 1, then
        // softmax and PV of tile i
        if (i + LOOK + 1 < ntiles) kf.load(tw + (i + LOOK + 1) * kStep, kr[u % R]);
        if (i + LOOK < ntiles) vf.load(tw + (i + LOOK) * kStep, vr[(u + LOOK) % R]);
        if (i + 1 < ntiles) {
          x[(u + 1) & 1][0] = kf.qk(kr[(u + 1) % R], 0, nc);
          x[(u + 1) & 1][1] = kf.qk(kr[(u + 1) % R], 1, nc);
        }
        float4v x0 = x[u & 1][0], x1 = x[u & 1][1];
        if (partial && i == ntiles - 1) mask_tile(x0, x1, tw + i * kStep, t1, lg);
        half8v pb;
        if constexpr (PACK8) pb = softmax_tile8(x0, x1, sm, m, l, acc);
        else pb = softmax_tile(x0, x1, sm, m, l, acc);
        vf.mma(vr[u % R], pb, acc, nc);
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
  uint32_t* counter = a.counters + (int64_t)b * a.Hkv + hkv;
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

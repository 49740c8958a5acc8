// Split-K decode attention for gfx950 over INT4_ASYM K (optional fp16 outlier
// channels) and INT4_ASYM V stored in the TILE32 layout, optionally with the
// quantize-on-append of the step's new token in the same launch.
//
// One work-group = kTW (8) waves = one (batch b, kv head, chunk); the GQA heads of the kv
// head are the N = 16 columns of v_mfma_f32_16x16x32_f16 and each wave walks 32-token
// tiles.  At the headline shape one work-group fills one CU (two waves per SIMD).
//
//  * Tile schedule: the n_chunks work-groups of a (b, kv head) interleave tile by tile
//    (wave w of work-group c takes tiles c * kTW + w + i * n_chunks * kTW), so the device
//    streams each slab front to back and every wave gets the same number of tiles when
//    the context allows.  The schedule is static: results do not depend on timing.
//  * The two waves of a SIMD (w and w + 4) publish their step counts in LDS; the one
//    ahead lowers its priority (s_setprio), which cancels the SIMD's oldest-first issue
//    order that would otherwise let one of them finish far earlier.
//  * K rows are dense (64 bytes per token) and so is the outlier side-band (8 bytes).
//  * Every cache read is a buffer load.  The (b, kv head) slab of each stream is a
//    wave-uniform buffer resource whose size bounds the reads (bytes past it read as
//    zero, with no memory access), the per-tile offset is a scalar and the per-lane
//    offset is loop-invariant.  Loads past a wave's last tile are issued with an
//    out-of-range offset rather than skipped, which keeps the compiler's vmcnt waits
//    exact.
//  * V in the TILE32 layout stores, for each tile, the 32 bytes lane L needs for its PV
//    operand contiguously at L * 32: two dwordx4 loads per lane, fully coalesced.
//  * The 4 fp16 outlier channels of the 32 tokens of a tile (256 bytes) are fetched by
//    one dword load of the whole wave: lane (row, g) takes the channel pair g & 1 of
//    token 16 (g >> 1) + row, which is where the outlier MFMA of row block g >> 1
//    needs it.
//  * A packed dword becomes 8 fp16 operands with 5 ops.  K: v_and_b32 with the masks
//    0x00F000F0 (high nibbles of bytes 0 and 2 -> the subnormal 16 n * 2^-24) and
//    0x000F000F (low nibbles -> n * 2^-24), then the same on the dword shifted right by 8
//    (bytes 1 and 3); the q side is one fp16 operand per channel and the logits come out
//    scaled by 2^-24.  V: the same subnormals; the epilogue scales by 2^20 / 2^24 and
//    removes the code offset 8 against l.
//  * The probabilities enter the PV MFMAs as hi = fp16(p) and lo = fp16(p - hi), each
//    multiplied by the V operand (16 MFMAs per tile), so the softmax weights keep about
//    21 bits instead of fp16's 11 (see softmax_tile).
//  * The q-dependent operands (fp16(q * s), the bias) are built once per work-group and
//    shared through LDS; the q loads are issued before the first cache loads.
//  * K and V tiles are fetched LOOK steps ahead of their use (register rings of
//    LOOK + 1 tiles); QK of tile i + 1 is issued before softmax / PV of tile i.
//  * With at most kUnitChunks chunks per (b, kv head) the last work-group to finish
//    merges the partials (no second launch; its arrival counters live in the workspace,
//    which must be zero-filled before its first use and which every call leaves zero);
//    otherwise combine_kernel does.
//  * The other operand types (K: KI8T, KTokT, KKiviT, KKivi8T, KF16T; V: VI8RowT, VTokT,
//    VKiviRowT, VKivi8RowT, VF16RowT) read the reference's token-row layouts with the same
//    schedule, loads and merge.  Their fused append (kAppendRow) runs the append kernel's
//    row quantizer (append_row.h) in the writer wave, whose inputs are requested with the
//    q loads; with INT4_SYM sides (kRescue) the writer also finds the group rescue's
//    threshold over every new row of the step.
#pragma once

#include "decode_common.h"

#include <cstdlib>
#include <type_traits>

// Tiles a row format's fused-append writer hands to waves of the other SIMDs (at most 6;
// decode_tiled_kernel): with the INT4 group rescue (the writer also finds the rescue
// threshold), and for the other row formats.
#ifndef KVQ_SHED_RESCUE
#define KVQ_SHED_RESCUE 3
#endif
#ifndef KVQ_SHED_ROW
#define KVQ_SHED_ROW 1
#endif

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
// its n_rep heads, which every work-group of the launch stored write-through, and writes
// the output rows with combine_one's arithmetic.  Needs n_chunks <= kUnitChunks (64);
// KF::kMergeBatch chunk loads are in flight at a time.
constexpr int kTW = kTiledWaves;
constexpr int kBufSC1 = 16;  // cache-policy bits: sc1 (device-coherent load)
// Chunk partials whose loads the merging work-group issues together: one memory round trip
// per batch.  Each K format sets its batch (KF::kMergeBatch): 32 where its kernels split a
// context into many chunks (static INT8 K: 32 chunks per (b, kv head) at config 1), 8
// otherwise (the 32-load batch raised the INT4 kernels' VGPR count and cost them 0.5 us).

// LDS of the work-group merge.  A head's row holds its 128 channels contiguous, 16-byte
// aligned, plus one float4 of padding (rows 132 floats apart): a lane writes its 32 channels
// with 8 ds_write_b128 (channels 32 lg + 8 r .. + 7 are acc[0..7][r]) and the combine reads
// channel pairs with ds_read_b64.  (One float of padding and scalar writes, 32 per lane, cost
// about 0.2 us per launch at the headline shape.)
struct TiledMergeLds {
  float m[kTW][16];
  float l[kTW][16];
  float4v acc[kTW][16][kD / 4 + 1];
};

// Merges the (m, l, acc) states of the work-group's waves (through LDS) into its partial
// of each row and stores it write-through at device scope, so another work-group of the
// launch, on any XCD, can read it once the stores have completed.  acc[mb][r] of lane
// (head, lg) holds channel d = 32 lg + 8 r + mb.  First every wave writes its state
// (merge_to_lds, ending with a barrier); then, per row, waves [lo, hi) of the work-group
// are merged (merge_partial): wave w merges heads w, w + kTW, ..; lane l channels 2 l and
// 2 l + 1: partial = sum_w e_w acc_w with e_w = exp2(m_w - M), (M, sum_w e_w l_w) for the
// head's (m, l) pair.  A wave without a tile has m = -inf, weight 0.
template <bool PACK8>
__device__ __forceinline__ void merge_to_lds(const DecodeArgs& a, TiledMergeLds& sh, int wave,
                                             int lane, float m, float l, const float4v acc[8]) {
  const int col = lane & 15, lg = lane >> 4;
  if constexpr (PACK8) l += dpp_ror8f<0xF>(l, l);  // add the block-1 part from lane h + 8
  l = wave_sum_xor_groups(l);
  if (lg == 0) {
    sh.m[wave][col] = m;
    sh.l[wave][col] = l;
  }
  if (col < a.n_rep) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sh.acc[wave][col][8 * lg + 2 * r] = float4v{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
      sh.acc[wave][col][8 * lg + 2 * r + 1] = float4v{acc[4][r], acc[5][r], acc[6][r], acc[7][r]};
    }
  }
  __syncthreads();
}
__device__ __forceinline__ void merge_partial(const DecodeArgs& a, const TiledMergeLds& sh,
                                              int wave, int lane, int lo, int hi, int b, int hkv,
                                              int slot) {
  for (int h = wave; h < a.n_rep; h += kTW) {
    float mw[kTW];
#pragma unroll
    for (int w = 0; w < kTW; ++w) mw[w] = (w >= lo && w < hi) ? sh.m[w][h] : kNegInf;
    float M = mw[0];
#pragma unroll
    for (int w = 1; w < kTW; ++w) M = fmaxf(M, mw[w]);
    // (selects, not branches: the LDS reads of all kTW waves are issued together)
    float n0 = 0.f, n1 = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < kTW; ++w) {
      const bool in = w >= lo && w < hi;
      const float e = fast_exp2(mw[w] - M);
      const float2 v2 = reinterpret_cast<const float2*>(&sh.acc[w][h][0])[lane];
      const float lw = sh.l[w][h];
      n0 = in ? fmaf(e, v2.x, n0) : n0;
      n1 = in ? fmaf(e, v2.y, n1) : n1;
      den = in ? fmaf(e, lw, den) : den;
    }
    const int64_t pi = ((int64_t)b * a.Hq + hkv * a.n_rep + h) * a.n_chunks + slot;
    __hip_atomic_store(reinterpret_cast<uint64_t*>(a.part_acc + pi * kD + 2 * lane),
                       __builtin_bit_cast(uint64_t, float2{n0, n1}), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    if (lane == 0)
      __hip_atomic_store(reinterpret_cast<uint64_t*>(a.part_ml + pi),
                         __builtin_bit_cast(uint64_t, float2{M, den}), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The attention partial (m, l, acc of channels 2 lane, 2 lane + 1) of query head hq over the
// fp16 residual window of (b, kv head) (a.res_n tokens), in the units of the chunk partials:
// logits q' . k * sm * log2(e) with q' = fp16(q * inv_tau) in fp32, base-2 softmax.  The
// window's rows are read 16 tokens per batch, K and V of a batch in flight together; one wave
// reduction per token.
__device__ __forceinline__ void residual_partial(const DecodeArgs& a, int b, int hkv, int hq, int lane,
                                                 float& mr, float& lr, float& r0, float& r1) {
  const bool has_tau = a.inv_tau != nullptr;
  const half_t tau = has_tau ? a.inv_tau[hq] : (half_t)1.0f;
  const half2v q2 = *reinterpret_cast<const half2v*>(q_row(a, b, hq) + 2 * lane);
  const float q0 = (float)qscale(q2.x, tau, has_tau), q1 = (float)qscale(q2.y, tau, has_tau);
  const int64_t off = slab_off(a.rsb, a.rsh, b, hkv) + 2 * lane;
  const half_t* kr = a.res_k + off;
  const half_t* vr = a.res_v + off;
  constexpr int kRB = 16;
  mr = kNegInf;
  lr = r0 = r1 = 0.f;
  for (int t0 = 0; t0 < a.res_n; t0 += kRB) {
    half2v kb[kRB], vb[kRB];
#pragma unroll
    for (int u = 0; u < kRB; ++u) {
      const int t = t0 + u < a.res_n ? t0 + u : a.res_n - 1;  // in bounds; masked below
      kb[u] = *reinterpret_cast<const half2v*>(kr + (int64_t)t * kD);
      vb[u] = *reinterpret_cast<const half2v*>(vr + (int64_t)t * kD);
    }
    float sc[kRB];
    float mx = mr;
#pragma unroll
    for (int u = 0; u < kRB; ++u) {
      const float d = wave_sum64(fmaf(q0, (float)kb[u].x, q1 * (float)kb[u].y));
      sc[u] = t0 + u < a.res_n ? d * a.sm_log2e : kNegInf;
      mx = fmaxf(mx, sc[u]);
    }
    const float al = fast_exp2(mr - mx);
    lr *= al;
    r0 *= al;
    r1 *= al;
    mr = mx;
#pragma unroll
    for (int u = 0; u < kRB; ++u) {
      const float p = fast_exp2(sc[u] - mr);
      lr += p;
      r0 = fmaf(p, (float)vb[u].x, r0);
      r1 = fmaf(p, (float)vb[u].y, r1);
    }
  }
}

// The last work-group's merge of the nvalid chunk partials of each query head (its own
// included, read back like the others), with combine_one's arithmetic.  Wave w takes heads
// w, w + kTW, ..; lane l the (m, l) pair of chunk l and channels 2 l, 2 l + 1 of every
// chunk.  The buffer resources end after the nvalid-th chunk, so the loads of chunks past
// it read 0 without a branch; their weight is exp2(-inf) = 0.  Loads bypass the
// non-coherent cache levels (sc1); chunks are added in chunk order whichever work-group
// merges, so every call gives the same bits.  s, z: the V scale / zero-point of group
// lane / 16.
template <class VF, int kUnitBatch>
__device__ __forceinline__ void merge_chunks(const DecodeArgs& a, int b, int hkv, int nvalid,
                                             int wave, int lane) {
  // the V epilogue's scale / zero-point, requested with the first partial loads (loaded any
  // earlier, every work-group's merge would wait for them)
  float s, z;
  VF::epi_params(a, hkv, lane, s, z);
  static_assert(kUnitChunks <= 64, "one (m, l) pair per lane");
  for (int h = wave; h < a.n_rep; h += kTW) {
    const int64_t row = ((int64_t)b * a.Hq + hkv * a.n_rep + h) * a.n_chunks;
    const rsrc_t rml = buffer_rsrc(a.part_ml + row, (uint32_t)nvalid * 8u);
    const rsrc_t racc = buffer_rsrc(a.part_acc + row * kD, (uint32_t)nvalid * (kD * 4u));
    const u32x2 mlv = __builtin_bit_cast(
        u32x2, __builtin_amdgcn_raw_buffer_load_b64(rml, (int)(lane * 8), 0, kBufSC1));
    const uint32_t vbase = (uint32_t)lane * 8u;
    u32x2 av[kUnitBatch];
#pragma unroll
    for (int c = 0; c < kUnitBatch; ++c)
      av[c] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                            racc, (int)(vbase + (uint32_t)c * (kD * 4u)), 0, kBufSC1));
    // every load of the first batch is issued before the (m, l) pair is used (one memory
    // latency, not two)
    asm volatile("" ::: "memory");
    // the fp16 residual window's partial (KIVI-family V formats), while the chunk partials
    // are in flight
    float mr = kNegInf, lr = 0.f, rr0 = 0.f, rr1 = 0.f;
    if constexpr (VF::kResidual)
      if (a.res_n > 0) residual_partial(a, b, hkv, hkv * a.n_rep + h, lane, mr, lr, rr0, rr1);
    const float mc = lane < nvalid ? __builtin_bit_cast(float, (uint32_t)mlv.x) : kNegInf;
    float M = wave_max64(mc);
    if constexpr (VF::kResidual) M = fmaxf(M, mr);
    const float e = fast_exp2(mc - M);
    float den = wave_sum64(e * __builtin_bit_cast(float, (uint32_t)mlv.y));
    float er = 0.f;  // the window's weight (none without one)
    if constexpr (VF::kResidual) {
      er = fast_exp2(mr - M);
      den = fmaf(er, lr, den);
    }
    float n0 = 0.f, n1 = 0.f;
    for (int c0 = 0;;) {
#pragma unroll
      for (int c = 0; c < kUnitBatch; ++c) {
        // (uint32_t) makes the vector element an rvalue: this clang's __builtin_bit_cast of
        // an ext_vector element lvalue reads element 0 whatever the index
        const float ec = row_lane(e, c0 + c);
        n0 = fmaf(ec, __builtin_bit_cast(float, (uint32_t)av[c].x), n0);
        n1 = fmaf(ec, __builtin_bit_cast(float, (uint32_t)av[c].y), n1);
      }
      c0 += kUnitBatch;
      if (c0 >= nvalid) {
        if constexpr (VF::kResidual) {
          n0 = fmaf(er, rr0, n0);
          n1 = fmaf(er, rr1, n1);
        }
        break;
      }
#pragma unroll
      for (int c = 0; c < kUnitBatch; ++c)
        av[c] = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                       racc, (int)(vbase + (uint32_t)(c0 + c) * (kD * 4u)), 0, kBufSC1));
    }
    const half2v o = VF::epilogue(n0 / den, n1 / den, s, z);
    *reinterpret_cast<half2v*>(a.out + (int64_t)b * a.o_sb + (int64_t)(hkv * a.n_rep + h) * a.o_sh +
                               2 * lane) = o;
  }
}

// merge_chunks' steps for one (row, head) pair, split so that a wave can request the loads
// of two pairs before it combines either: merge_pair_issue requests the (m, l) pairs and the
// first batch of chunk partials, merge_pair_finish combines them (and any further batch)
// with the same arithmetic and writes the output row.
template <int kB>
struct PairLoads {
  rsrc_t racc;
  u32x2 ml;
  u32x2 av[kB];
};
template <int kB>
__device__ __forceinline__ void merge_pair_issue(const DecodeArgs& a, int b, int hkv, int h,
                                                 int nvalid, int lane, PairLoads<kB>& L) {
  const int64_t row = ((int64_t)b * a.Hq + hkv * a.n_rep + h) * a.n_chunks;
  const rsrc_t rml = buffer_rsrc(a.part_ml + row, (uint32_t)nvalid * 8u);
  L.racc = buffer_rsrc(a.part_acc + row * kD, (uint32_t)nvalid * (kD * 4u));
  L.ml = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rml, (int)(lane * 8), 0, kBufSC1));
#pragma unroll
  for (int c = 0; c < kB; ++c)
    L.av[c] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                            L.racc, (int)((uint32_t)lane * 8u + (uint32_t)c * (kD * 4u)), 0, kBufSC1));
}
template <class VF, int kB>
__device__ __forceinline__ void merge_pair_finish(const DecodeArgs& a, int b, int hkv, int h,
                                                  int nvalid, int lane, PairLoads<kB>& L,
                                                  float s, float z) {
  float mr = kNegInf, lr = 0.f, rr0 = 0.f, rr1 = 0.f;
  if constexpr (VF::kResidual)
    if (a.res_n > 0) residual_partial(a, b, hkv, hkv * a.n_rep + h, lane, mr, lr, rr0, rr1);
  const float mc = lane < nvalid ? __builtin_bit_cast(float, (uint32_t)L.ml.x) : kNegInf;
  float M = wave_max64(mc);
  if constexpr (VF::kResidual) M = fmaxf(M, mr);
  const float e = fast_exp2(mc - M);
  float den = wave_sum64(e * __builtin_bit_cast(float, (uint32_t)L.ml.y));
  float er = 0.f;
  if constexpr (VF::kResidual) {
    er = fast_exp2(mr - M);
    den = fmaf(er, lr, den);
  }
  float n0 = 0.f, n1 = 0.f;
  for (int c0 = 0;;) {
#pragma unroll
    for (int c = 0; c < kB; ++c) {
      const float ec = row_lane(e, c0 + c);
      n0 = fmaf(ec, __builtin_bit_cast(float, (uint32_t)L.av[c].x), n0);
      n1 = fmaf(ec, __builtin_bit_cast(float, (uint32_t)L.av[c].y), n1);
    }
    c0 += kB;
    if (c0 >= nvalid) {
      if constexpr (VF::kResidual) {
        n0 = fmaf(er, rr0, n0);
        n1 = fmaf(er, rr1, n1);
      }
      break;
    }
#pragma unroll
    for (int c = 0; c < kB; ++c)
      L.av[c] = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                     L.racc, (int)((uint32_t)lane * 8u + (uint32_t)(c0 + c) * (kD * 4u)), 0, kBufSC1));
  }
  const half2v o = VF::epilogue(n0 / den, n1 / den, s, z);
  *reinterpret_cast<half2v*>(a.out + (int64_t)b * a.o_sb + (int64_t)(hkv * a.n_rep + h) * a.o_sh +
                             2 * lane) = o;
}
// The shared split's merge of the rows whose last work-group this is (nr = 1 or 2: rows
// b0 (n0 partials) and b1 (n1)).  Pair p is (row p / n_rep, head p % n_rep); wave w takes
// pairs w, w + kTW, ..; a wave with two pairs requests the loads of both before it combines
// the first (one memory latency for the two rows, where merging them one after the other
// took two).
template <class VF, int kB>
__device__ __forceinline__ void merge_rows(const DecodeArgs& a, int hkv, int b0, int n0, int b1,
                                           int n1, int nr, int wave, int lane) {
  float s, z;
  VF::epi_params(a, hkv, lane, s, z);
  const int np = nr * a.n_rep;
  for (int p = wave; p < np; p += 2 * kTW) {
    const int q = p + kTW;
    const bool two = q < np;
    const int r0 = p >= a.n_rep, r1 = q >= a.n_rep;
    const int h0 = p - r0 * a.n_rep, h1 = two ? q - r1 * a.n_rep : 0;
    const int bb0 = r0 ? b1 : b0, nn0 = r0 ? n1 : n0;
    const int bb1 = r1 ? b1 : b0, nn1 = r1 ? n1 : n0;
    PairLoads<kB> L0, L1;
    merge_pair_issue<kB>(a, bb0, hkv, h0, nn0, lane, L0);
    if (two) merge_pair_issue<kB>(a, bb1, hkv, h1, nn1, lane, L1);
    asm volatile("" ::: "memory");
    merge_pair_finish<VF, kB>(a, bb0, hkv, h0, nn0, lane, L0, s, z);
    if (two) merge_pair_finish<VF, kB>(a, bb1, hkv, h1, nn1, lane, L1, s, z);
  }
}

// 8 packed codes -> 8 fp16 operands in k-slot order [e0, e4, e1, e5, e2, e6, e3, e7]
// (e = element within the dword; byte k holds e = 2k in its high nibble), read as fp16
// subnormals: a nibble in bits 4..7 of a 16-bit half is 16 n * 2^-24, one in bits 0..3 is
// n * 2^-24, both exact.  The MFMA takes subnormal fp16 inputs without flushing them, and
// with no offset in the operand the q side needs a single fp16 operand (a product q * s
// rounded to fp16 perturbs each term by at most 2^-11 of itself).  5 ops per 8 codes.
__device__ __forceinline__ half8v unpack_sub(uint32_t w, const NibConsts& nc) {
  const uint32_t w8 = w >> 8;
  return pack8(w & nc.m_hi, w & nc.m_lo, w8 & nc.m_hi, w8 & nc.m_lo);
}
__host__ __device__ constexpr int slot_elem(int k) { return (k & 1) * 4 + (k >> 1); }
// k-slots holding a high nibble (operand value 16 n * 2^-24)
__host__ __device__ constexpr bool slot_high(int k) { return ((k >> 1) & 1) == 0; }
constexpr float kTwo24 = 16777216.0f;       // 2^24
constexpr float kTwoM24 = 5.9604644775390625e-8f;  // 2^-24

// LDS through which the 4 waves share the q-dependent K operands, and the scaled q rows
// from which the outlier operand is gathered
struct QShareLds {
  u32x4 qh[4][64];
  u32x4 ql[4][64];  // the low halves of a hi + lo split operand (KKiviT)
  float bias[4][16];
  half_t qv[16][kD];  // q' of head column c (zero for padding columns)
};

// x = hi + lo with hi = fp16(x) and lo = fp16(x - hi) (x - hi is exact in fp32): the pair
// carries x to about 2^-22 of itself, where fp16(x) alone carries it to 2^-11
__device__ __forceinline__ void split_h(float x, half_t& hi, half_t& lo) {
  hi = (half_t)x;
  lo = (half_t)(x - (float)hi);
}

// The q-side inputs of one lane: q[32 lg + 8 wave .. + 7] of head column lane % 16, its
// inverse temperature and the K scale / zero-point of group lg.  They are fetched before
// the first cache loads, so waiting for them does not wait for those (vmcnt counts loads
// in issue order).
__device__ __forceinline__ int4 clamp_ch4(int4 o) {
  return int4{min(max(o.x, 0), kD - 1), min(max(o.y, 0), kD - 1), min(max(o.z, 0), kD - 1),
              min(max(o.w, 0), kD - 1)};
}
struct QIn {
  u32x4 q;
  half_t tau, s, z;
  int4 oc;
  uint32_t sj[4];  // static INT8 K: the loaded bits (static_scale_bits) of the scale of
                   // channel slice 32 lg + 8 j (any group size)
};

// INT4 asymmetric K with static scale s / zero-point z per (kv head, group of 32).  With
// code c = n - 8 the logit is
//   sum_d q_d (s c_d + z) = sum_d (q_d s) n_d + sum_d q_d (z - 8 s);
// the codes enter the MFMA as subnormals n * 2^-24 (16 n * 2^-24 for high nibbles, whose
// q operand is divided by 16), q_d s rounded to fp16 is the other operand, and the
// constant term starts the accumulator.  Outlier channels (q zeroed in the main MFMAs)
// are added by one MFMA of the same shape whose operands are the 4 fp16 outlier values
// and q' of those channels in the first two k-slots of each lane group.
template <bool OUT>
struct KAsymT {
  static constexpr int kRowFmt = -1;  // no row append
  static constexpr int kMergeBatch = 8;
  // hi / lo probabilities in one PV MFMA (softmax_tile8c) when the V format allows it:
  // measured 0.2 us faster at configs 2-3; with static INT8 K (short per-wave runs at
  // config 1) the post-loop fold costs more than the MFMAs it saves
  static constexpr bool kPackPV = true;
  using QInT = QIn;
  static constexpr bool kAppend = true;  // the fused quantize-on-append is built for this format
  static constexpr bool kAppendRow = false;  // (its own specialised writer code)
  static constexpr bool kAsym = true;
  static constexpr bool kGsAny = false;  // groups of 32
  static constexpr bool kOut = OUT;
  static constexpr bool kSub24 = true;  // logits scaled by 2^-24
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
    const uint8_t* kb = a.k.codes + slab_off(a.k.sb, a.k.sh, b, hkv);
    rk = buffer_rsrc(kb, (uint32_t)(a.cap * kRowK));
    vk = (uint32_t)(col * kRowK + 16 * lg);
    if constexpr (OUT) {
      const half_t* ob = a.k.oval + slab_off(a.k.osb, a.k.osh, b, hkv);
      ro = buffer_rsrc(ob, (uint32_t)(a.cap * kRowO));
      vo = (uint32_t)((16 * (lg >> 1) + col) * kRowO + (lg & 1) * 4);
    }
  }

  // issues the loads of the q-side inputs (padding columns read head 0's row)
  __device__ void fetch_q(const DecodeArgs& a, int b, int hkv, int lane, int wave, QIn& in) const {
    const int col = lane & 15, lg = lane >> 4;
    const int hq = hkv * a.n_rep + (col < a.n_rep ? col : 0);
    in.q = *reinterpret_cast<const u32x4*>(q_row(a, b, hq) + 32 * lg + 8 * (wave & 3));
    in.tau = a.inv_tau != nullptr ? a.inv_tau[hq] : (half_t)1.0f;
    in.s = reinterpret_cast<const half_t*>(a.k.scale)[hkv * a.k.ssh + lg * a.k.ssg];
    in.z = a.k.zp[hkv * a.k.ssh + lg * a.k.ssg];
    in.oc = int4{-1, -1, -1, -1};
    // raw indices: each use clamps them to [0, kD - 1] (arithmetic on a loaded value here
    // would make every wave wait for the q loads before it requests its first tiles)
    if constexpr (OUT) in.oc = *reinterpret_cast<const int4*>(a.k.oidx + hkv * 4);
  }

  // q-dependent operands of channel slice j = 0..3 (channels 32 lg + 8 j + e), shared
  // through LDS; called by waves 0..3 only.  Operand k = fp16(q'_d s) (fp16(q'_d s / 16) for a
  // high-nibble slot) multiplies n_d * 2^-24 (16 n_d * 2^-24), so the MFMA sums
  // e_d n_d * 2^-24 with e_d = the operand's value (x 16 for a high nibble), and
  //   logit = sum_d q'_d (s c_d + z) = 2^24 * mfma + sum_d (q'_d z - 8 e_d)  (c = n - 8).
  __device__ void setup_q(const DecodeArgs& a, const QIn& in, int lane, int j, QShareLds& sh) {
    const int col = lane & 15, lg = lane >> 4;
    const bool valid = col < a.n_rep;
    const bool has_tau = a.inv_tau != nullptr;
    const uint32_t qw[4] = {in.q.x, in.q.y, in.q.z, in.q.w};
    const float s = (float)in.s;
    const float z = (float)in.z;
    float part = 0.f;
    const int4 oc = clamp_ch4(in.oc);
    half_t vh[8], qs[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const half2v h2 = as_h2(qw[e >> 1]);
      qs[e] = valid ? qscale((e & 1) ? h2.y : h2.x, in.tau, has_tau) : (half_t)0.0f;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = slot_elem(k);
      const int d = 32 * lg + 8 * j + e;
      const bool use = !OUT || (d != oc.x && d != oc.y && d != oc.z && d != oc.w);
      const float qd = use ? (float)qs[e] : 0.f;
      const float P = qd * s;  // exact: 11-bit x 11-bit significands
      const half_t h = (half_t)(slot_high(k) ? P * 0.0625f : P);
      vh[k] = h;
      part += qd * z - 8.0f * (slot_high(k) ? 16.0f * (float)h : (float)h);
    }
    part = wave_sum_xor_groups(part);
    sh.qh[j][lane] = __builtin_bit_cast(u32x4, half8v{vh[0], vh[1], vh[2], vh[3], vh[4], vh[5], vh[6], vh[7]});
    *reinterpret_cast<u32x4*>(&sh.qv[col][32 * lg + 8 * j]) =
        __builtin_bit_cast(u32x4, half8v{qs[0], qs[1], qs[2], qs[3], qs[4], qs[5], qs[6], qs[7]});
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
      const int4 oc = clamp_ch4(in.oc);
      qo = half8v{sh.qv[col][odd ? oc.z : oc.x], sh.qv[col][odd ? oc.w : oc.y],
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

  // logits of the tile's two 16-token row blocks (x0: tokens 4 lg + r, x1: 16 + 4 lg + r),
  // scaled by 2^-24 (the softmax multiplies by sm * 2^24).  The outlier channels go through
  // a separate accumulator at unit scale, started at the bias, and are added at the end.
  __device__ __forceinline__ void qk(const Raw& r, const NibConsts& nc, float4v& x0,
                                     float4v& x1) const {
    float4v c0, c1;
    if constexpr (OUT) {
      c0 = float4v{0.f, 0.f, 0.f, 0.f};
      c1 = c0;
    } else {
      const float b24 = bias * kTwoM24;
      c0 = float4v{b24, b24, b24, b24};
      c1 = c0;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c0 = mfma16x16x32(unpack_sub(r.w[0][j], nc), qh[j], c0);
      c1 = mfma16x16x32(unpack_sub(r.w[1][j], nc), qh[j], c1);
    }
    if constexpr (OUT) {
      const float4v b4 = {bias, bias, bias, bias};
      const float4v o0 = mfma16x16x32(pack8(olo ? r.o : 0u, 0u, 0u, 0u), qo, b4);
      const float4v o1 = mfma16x16x32(pack8(olo ? 0u : r.o, 0u, 0u, 0u), qo, b4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c0[i] = fmaf(o0[i], kTwoM24, c0[i]);
        c1[i] = fmaf(o1[i], kTwoM24, c1[i]);
      }
    }
    x0 = c0;
    x1 = c1;
  }
};

// INT4 asymmetric V in the TILE32 layout.  acc[c] (c < 8) accumulates sum_t p * x for
// channel 8 col + c of the lane's d-row col, with the codes as the exact fp16 subnormals
// x = 16 n 2^-24 (even c, high nibble) or n 2^-24 (odd c) and p the hi + lo probability
// operands (softmax_tile); the epilogue applies out = s (acc / l * 2^20 or 2^24 - 8) + z.
struct VAsymT {
  static constexpr int kRowFmt = -1;  // no row append
  static constexpr bool kResidual = false;  // merges an fp16 residual window
  static constexpr bool kTile32 = true;
  static constexpr bool kPackedPV = true;  // mma1 with softmax_tile8c's operand
  // hooks of formats with per-token parameters (none here)
  template <class Raw>
  __device__ __forceinline__ void mask(Raw&, int, int, int) const {}
  __device__ __forceinline__ void finalize(float4v*, int) const {}
  __device__ __forceinline__ float* extra() { return nullptr; }
  rsrc_t rv;
  uint32_t vv;
  struct Raw {
    u32x4 w[2];
  };
  // the V scale / zero-point of group lane / 16 for the output epilogue
  __device__ static void epi_params(const DecodeArgs& a, int hkv, int lane, float& s, float& z) {
    const int g = lane >> 4;
    s = (float)reinterpret_cast<const half_t*>(a.v.scale)[hkv * a.v.ssh + g * a.v.ssg];
    z = (float)a.v.zp[hkv * a.v.ssh + g * a.v.ssg];
  }
  // channels 2 lane, 2 lane + 1 from the merged acc / l: 2^20 r0 and 2^24 r1 are n = c + 8
  __device__ static half2v epilogue(float r0, float r1, float s, float z) {
    return half2v{(half_t)fmaf(s, fmaf(r0, 1048576.0f, -8.0f), z),
                  (half_t)fmaf(s, fmaf(r1, 16777216.0f, -8.0f), z)};
  }

  __device__ void setup(const DecodeArgs& a, int b, int hkv, int lane) {
    const uint8_t* vb = a.v.codes + slab_off(a.v.sb, a.v.sh, b, hkv);
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
  template <bool ONE = false>
  __device__ __forceinline__ void mma(const Raw& r, half8v pb, half8v pl, float4v acc[8],
                                      const NibConsts& nc) const {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      // dword 2p + k of the lane: bytes (2k, 2k+1) of the two tokens of k-slot pair p
      const uint32_t a0 = k ? r.w[0].y : r.w[0].x, a1 = k ? r.w[0].w : r.w[0].z;
      const uint32_t a2 = k ? r.w[1].y : r.w[1].x, a3 = k ? r.w[1].w : r.w[1].z;
      const uint32_t s0 = a0 >> 8, s1 = a1 >> 8, s2 = a2 >> 8, s3 = a3 >> 8;
      const half8v c0 = pack8(a0 & nc.m_hi, a1 & nc.m_hi, a2 & nc.m_hi, a3 & nc.m_hi);
      const half8v c1 = pack8(a0 & nc.m_lo, a1 & nc.m_lo, a2 & nc.m_lo, a3 & nc.m_lo);
      const half8v c2 = pack8(s0 & nc.m_hi, s1 & nc.m_hi, s2 & nc.m_hi, s3 & nc.m_hi);
      const half8v c3 = pack8(s0 & nc.m_lo, s1 & nc.m_lo, s2 & nc.m_lo, s3 & nc.m_lo);
      acc[4 * k] = mfma16x16x32(c0, pb, acc[4 * k]);
      acc[4 * k + 1] = mfma16x16x32(c1, pb, acc[4 * k + 1]);
      acc[4 * k + 2] = mfma16x16x32(c2, pb, acc[4 * k + 2]);
      acc[4 * k + 3] = mfma16x16x32(c3, pb, acc[4 * k + 3]);
      if constexpr (!ONE) {
        acc[4 * k] = mfma16x16x32(c0, pl, acc[4 * k]);
        acc[4 * k + 1] = mfma16x16x32(c1, pl, acc[4 * k + 1]);
        acc[4 * k + 2] = mfma16x16x32(c2, pl, acc[4 * k + 2]);
        acc[4 * k + 3] = mfma16x16x32(c3, pl, acc[4 * k + 3]);
      }
    }
  }
  // one MFMA per block: pb is softmax_tile8c's combined hi / lo operand
  __device__ __forceinline__ void mma1(const Raw& r, half8v pc, float4v acc[8],
                                       const NibConsts& nc) const {
    mma<true>(r, pc, pc, acc, nc);
  }
};

// The scale of (kv head, group g) from a scale view that is static over b and t (stride-0
// view of per-token scales, fp16 or fp32): static_scale_bits loads its bits (fp32, or fp16
// in the low half), static_scale16 gives the fp16 scale (an fp32 scale rounded to fp16).
// They are split so that the set-up converts after the first cache tiles are requested:
// converting at the load made every wave wait for it before its first tile load.
__device__ __forceinline__ uint32_t static_scale_bits(const KvDev& v, int hkv, int g) {
  const int64_t i = (int64_t)hkv * v.ssh + (int64_t)g * v.ssg;
  return v.scale_f32 ? reinterpret_cast<const uint32_t*>(v.scale)[i]
                     : (uint32_t)reinterpret_cast<const uint16_t*>(v.scale)[i];
}
__device__ __forceinline__ half_t static_scale16(uint32_t bits, int f32) {
  return f32 ? (half_t)__builtin_bit_cast(float, bits) : __builtin_bit_cast(half_t, (uint16_t)bits);
}

// Two INT8 codes (the low bytes of the two halves of x, the high bytes zero) -> the fp16
// pair fp16(c * s16), rounded once as the reference's dequantisation (int8 -> fp16, times
// the fp16 scale, src/engine/patch_model.py:355-362): x ^ 0x64806480 gives 1024 + (c + 128)
// exactly, minus 1152 gives c, and the packed fp16 product with s16 rounds to nearest even.
__device__ __forceinline__ uint32_t i8pair_deq(uint32_t x, half2v s2) {
  const half2v off = {(half_t)1152.0f, (half_t)1152.0f};
  return as_u32((as_h2(x ^ 0x64806480u) - off) * s2);
}

// INT8 symmetric K with a static fp16 scale s per (kv head, group), i.e. per-token scales
// given as a view with stride 0 over b and t (the reference's static-scale cache,
// src/cache/int8_cache.py:298-488).  Lane (row, lg) of row block rb reads bytes
// [32 lg, 32 lg + 32) of token 16 rb + row.  GS_ANY = false: groups of 32, so those 32
// channels are group lg and share one scale.  GS_ANY = true: any group size (8 .. 128,
// a.gs); each 8-channel slice j takes the scale of its own group (3 more VGPRs; the group
// index comes from a.gs at run time, which costs the groups-of-32 kernel 0.2 us of set-up
// at config 1, hence two instantiations).  The A operand is the reference's
// dequantised k = fp16(c * s16) (i8pair_deq), the B operand q', so the logits are the
// reference's fp32 dot products of fp16 k and q up to the summation order.
template <bool GS_ANY>
struct KI8T {
  static constexpr int kRowFmt = -1;  // no row append
  static constexpr bool kGsAny = GS_ANY;
  static constexpr int kMergeBatch = 32;
  static constexpr bool kPackPV = false;
  using QInT = QIn;
  static constexpr bool kAppend = true;
  static constexpr bool kAppendRow = false;
  static constexpr bool kAsym = false;
  static constexpr bool kOut = false;
  static constexpr bool kSub24 = false;  // logits at unit scale
  static constexpr int kNS = GS_ANY ? 4 : 1;
  half8v qh[4];
  half2v s2[kNS];  // the scale of channel slice 32 lg + 8 j .. + 7 (its group), twice
  rsrc_t rk;
  uint32_t vk;
  int sf32;  // the scale view holds fp32
  struct Raw {
    u32x4 w[4];  // [2 rb + i]: bytes [32 lg + 16 i, 32 lg + 16 i + 16) of token 16 rb + row
  };

  __device__ void setup_addr(const DecodeArgs& a, int b, int hkv, int lane) {
    const int col = lane & 15, lg = lane >> 4;
    const uint8_t* kb = a.k.codes + slab_off(a.k.sb, a.k.sh, b, hkv);
    rk = buffer_rsrc(kb, (uint32_t)(a.cap * kD));
    vk = (uint32_t)(col * kD + 32 * lg);
    sf32 = a.k.scale_f32;
  }
  __device__ void fetch_q(const DecodeArgs& a, int b, int hkv, int lane, int wave, QIn& in) const {
    const int col = lane & 15, lg = lane >> 4;
    const int hq = hkv * a.n_rep + (col < a.n_rep ? col : 0);
    in.q = *reinterpret_cast<const u32x4*>(q_row(a, b, hq) + 32 * lg + 8 * (wave & 3));
    in.tau = a.inv_tau != nullptr ? a.inv_tau[hq] : (half_t)1.0f;
    if constexpr (GS_ANY) {
      // slice j of the lane's 32 channels lies in group (32 lg + 8 j) / gs (gs = 8 .. 128)
      const int sh = __builtin_ctz((unsigned)a.gs);
#pragma unroll
      for (int j = 0; j < 4; ++j) in.sj[j] = static_scale_bits(a.k, hkv, (32 * lg + 8 * j) >> sh);
    } else {
      in.sj[0] = static_scale_bits(a.k, hkv, lg);
    }
    in.s = (half_t)1.0f;  // (the fused append quantizes with its own table)
    in.z = (half_t)0.0f;
    in.oc = int4{-1, -1, -1, -1};
  }
  // channel slice j (channels 32 lg + 8 j + e) of the q operand q' = fp16(q * inv_tau),
  // shared through LDS
  __device__ void setup_q(const DecodeArgs& a, const QIn& in, int lane, int j, QShareLds& sh) {
    const int col = lane & 15;
    const bool valid = col < a.n_rep;
    const bool has_tau = a.inv_tau != nullptr;
    const uint32_t qw[4] = {in.q.x, in.q.y, in.q.z, in.q.w};
    half_t vh[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const half2v h2 = as_h2(qw[e >> 1]);
      vh[e] = valid ? qscale((e & 1) ? h2.y : h2.x, in.tau, has_tau) : (half_t)0.0f;
    }
    sh.qh[j][lane] = __builtin_bit_cast(u32x4, half8v{vh[0], vh[1], vh[2], vh[3], vh[4], vh[5], vh[6], vh[7]});
  }
  __device__ void finish_setup(const QShareLds& sh, const QIn& in, int lane) {
#pragma unroll
    for (int j = 0; j < 4; ++j) qh[j] = __builtin_bit_cast(half8v, sh.qh[j][lane]);
#pragma unroll
    for (int j = 0; j < kNS; ++j) {
      const half_t sv = static_scale16(in.sj[j], sf32);
      s2[j] = half2v{sv, sv};
    }
  }
  __device__ __forceinline__ void load(int tok, bool valid, Raw& r) const {
    const uint32_t v = vk + (valid ? (uint32_t)tok * kD : kOutOfRange);
    r.w[0] = bload4(rk, v, 0);
    r.w[1] = bload4(rk, v + 16, 0);
    r.w[2] = bload4(rk, v + 16 * kD, 0);
    r.w[3] = bload4(rk, v + 16 * kD + 16, 0);
  }
  // 8 codes of slice j (dwords lo = channels 0..3, hi = 4..7) -> fp16(c * s16) in channel
  // order
  __device__ __forceinline__ half8v deq8(uint32_t lo, uint32_t hi, int j) const {
    const half2v s = s2[GS_ANY ? j : 0];
    return pack8(i8pair_deq(perm_b32(0u, lo, 0x0C010C00u), s), i8pair_deq(perm_b32(0u, lo, 0x0C030C02u), s),
                 i8pair_deq(perm_b32(0u, hi, 0x0C010C00u), s), i8pair_deq(perm_b32(0u, hi, 0x0C030C02u), s));
  }
  __device__ __forceinline__ void qk(const Raw& r, const NibConsts& nc, float4v& x0,
                                     float4v& x1) const {
    (void)nc;
    float4v c0 = {0.f, 0.f, 0.f, 0.f};
    float4v c1 = c0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 w0 = r.w[j >> 1], w1 = r.w[2 + (j >> 1)];
      const uint32_t l0 = (j & 1) ? w0.z : w0.x, h0 = (j & 1) ? w0.w : w0.y;
      const uint32_t l1 = (j & 1) ? w1.z : w1.x, h1 = (j & 1) ? w1.w : w1.y;
      c0 = mfma16x16x32(deq8(l0, h0, j), qh[j], c0);
      c1 = mfma16x16x32(deq8(l1, h1, j), qh[j], c1);
    }
    x0 = c0;
    x1 = c1;
  }
};

// INT8 symmetric V in token rows (the reference layout) with a static scale per (kv head,
// group): groups of 32 (GS_ANY = false) or any group size a.gs (8 .. 128).  Lane (col, lg) reads the 8 bytes of channels 8 col .. 8 col + 7 of its 8
// PV k-slot tokens T(k) = 4 lg + k (k < 4), 16 + 4 lg + k - 4: each load instruction reads
// four whole 128-byte rows.  The A operand of MFMA c (channel 8 col + c) is the reference's
// v = fp16(c * s16) of the 8 tokens (one v_perm_b32 per pair of tokens, then i8pair_deq), so
// acc / l is the output.
template <bool GS_ANY>
struct VI8RowT {
  static constexpr int kRowFmt = -1;  // no row append
  static constexpr bool kResidual = false;  // merges an fp16 residual window
  static constexpr bool kPackedPV = true;  // mma1 with softmax_tile8c's operand
  static constexpr bool kTile32 = false;
  // hooks of formats with per-token parameters (none here)
  template <class Raw>
  __device__ __forceinline__ void mask(Raw&, int, int, int) const {}
  __device__ __forceinline__ void finalize(float4v*, int) const {}
  __device__ __forceinline__ float* extra() { return nullptr; }
  rsrc_t rv;
  uint32_t vv;
  uint32_t sbits;  // the scale of the group of channels 8 col .. 8 col + 7 (static_scale_bits)
  int sf32;
  struct Raw {
    u32x2 w[8];  // token T(k)
  };
  __device__ static void epi_params(const DecodeArgs& a, int hkv, int lane, float& s, float& z) {
    (void)a; (void)hkv; (void)lane;
    s = 1.f;
    z = 0.f;
  }
  __device__ static half2v epilogue(float r0, float r1, float s, float z) {
    (void)s; (void)z;
    return half2v{(half_t)r0, (half_t)r1};
  }
  __device__ void setup(const DecodeArgs& a, int b, int hkv, int lane) {
    const int col = lane & 15, lg = lane >> 4;
    const uint8_t* vb = a.v.codes + slab_off(a.v.sb, a.v.sh, b, hkv);
    rv = buffer_rsrc(vb, (uint32_t)(a.cap * kD));
    vv = (uint32_t)((4 * lg) * kD + 8 * col);
    sbits = static_scale_bits(a.v, hkv, GS_ANY ? (8 * col) >> __builtin_ctz((unsigned)a.gs) : col >> 2);
    sf32 = a.v.scale_f32;
  }
  // rows of a partial last tile past the capacity read 0; !valid: every load out of range
  __device__ __forceinline__ void load(int tok, bool valid, Raw& r) const {
    const uint32_t v = vv + (valid ? (uint32_t)tok * kD : kOutOfRange);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t t = (k < 4) ? (uint32_t)k : (uint32_t)(12 + k);  // 16 + k - 4
      r.w[k] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rv, (int)(v + t * kD), 0, kBufNT));
    }
  }
  template <bool ONE = false>
  __device__ __forceinline__ void mma(const Raw& r, half8v pb, half8v pl, float4v acc[8],
                                      const NibConsts& nc) const {
    (void)nc;
    // (converted here, loop-invariant: the set-up does not wait for the table load)
    const half_t sv = static_scale16(sbits, sf32);
    const half2v s2 = {sv, sv};
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      // byte c % 4 of the tokens T(2p) and T(2p + 1) into the low bytes of the two halves
      const uint32_t sel = (uint32_t)(c & 3) | 0x0C00u | ((uint32_t)(4 + (c & 3)) << 16) | 0x0C000000u;
      uint32_t R[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t lo = (c >> 2) ? r.w[2 * p].y : r.w[2 * p].x;
        const uint32_t hi = (c >> 2) ? r.w[2 * p + 1].y : r.w[2 * p + 1].x;
        R[p] = i8pair_deq(perm_b32(hi, lo, sel), s2);
      }
      const half8v av = pack8(R[0], R[1], R[2], R[3]);
      acc[c] = mfma16x16x32(av, pb, acc[c]);
      if constexpr (!ONE) acc[c] = mfma16x16x32(av, pl, acc[c]);
    }
  }
  // one MFMA per block: pb is softmax_tile8c's combined hi / lo operand
  __device__ __forceinline__ void mma1(const Raw& r, half8v pc, float4v acc[8],
                                       const NibConsts& nc) const {
    mma<true>(r, pc, pc, acc, nc);
  }
};

// ---- KIVI layout (the reference's asymmetric INT4 kernels,
// src/kernels/triton_decode_attn_int4_asym.py:28-277 and its v2 / GQA variants): packed
// nibbles in token rows, K value (n - 8) s_d + z_d with fp32 s, z per (b, h, channel), V
// value (n - 8) s_t + z_t with fp32 s, z per (b, h, token).

// q-side inputs of KKiviT: the lane's 8 channels' K scale and zero-point
struct KiviQIn {
  u32x4 q;
  half_t tau, s, z;  // s, z unused (the fused append is not built for this format)
  int4 oc;
  float4v ks[2], kz[2];
};

// K of the KIVI layout: as KAsymT<false> (subnormal nibbles, logits x 2^-24) with
// per-channel parameters.  The q operand q'_d s_d (/ 16 for a high nibble) is a hi + lo
// pair of fp16 values (split_h), each multiplied by the codes in its own MFMA, so the
// product is carried to about 2^-22 of itself: the reference computes k = (n - 8) s_d + z_d
// and q . k in fp32, and per-channel scales of K outlier channels can be two orders of
// magnitude above the rest, where one fp16 rounding of q'_d s_d (2^-11 of the term) would
// show in the logits.  The constant term sum_d q'_d (z_d - 8 s_d) is summed in fp32.
struct KKiviT : KAsymT<false> {
  static constexpr int kRowFmt = KVQ_FMT_INT4_KIVI;  // the fused append's K format
  using QInT = KiviQIn;
  static constexpr bool kAppend = false;
  static constexpr bool kAppendRow = true;  // the writer runs quant_row_x (fused step)
  static constexpr bool kRescue = false;     // (no INT4_SYM side)
  half8v ql[4];
  __device__ void fetch_q(const DecodeArgs& a, int b, int hkv, int lane, int wave, KiviQIn& in) const {
    const int col = lane & 15, lg = lane >> 4;
    const int hq = hkv * a.n_rep + (col < a.n_rep ? col : 0);
    in.q = *reinterpret_cast<const u32x4*>(q_row(a, b, hq) + 32 * lg + 8 * (wave & 3));
    in.tau = a.inv_tau != nullptr ? a.inv_tau[hq] : (half_t)1.0f;
    in.oc = int4{-1, -1, -1, -1};
    const int64_t o = slab_off(a.k.ssb, a.k.ssh, b, hkv) + 32 * lg + 8 * (wave & 3);
    const float* ps = reinterpret_cast<const float*>(a.k.scale) + o;
    const float* pz = reinterpret_cast<const float*>(a.k.zp) + o;
    in.ks[0] = *reinterpret_cast<const float4v*>(ps);
    in.ks[1] = *reinterpret_cast<const float4v*>(ps + 4);
    in.kz[0] = *reinterpret_cast<const float4v*>(pz);
    in.kz[1] = *reinterpret_cast<const float4v*>(pz + 4);
  }
  __device__ void setup_q(const DecodeArgs& a, const KiviQIn& in, int lane, int j, QShareLds& sh) {
    const int col = lane & 15, lg = lane >> 4;
    const bool valid = col < a.n_rep;
    const bool has_tau = a.inv_tau != nullptr;
    const uint32_t qw[4] = {in.q.x, in.q.y, in.q.z, in.q.w};
    float part = 0.f;
    half_t vh[8], vl[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = slot_elem(k);
      const half2v h2 = as_h2(qw[e >> 1]);
      const float qd = valid ? (float)qscale((e & 1) ? h2.y : h2.x, in.tau, has_tau) : 0.f;
      const float sd = in.ks[e >> 2][e & 3], zd = in.kz[e >> 2][e & 3];
      const float P = qd * sd;
      split_h(slot_high(k) ? P * 0.0625f : P, vh[k], vl[k]);
      part += qd * fmaf(-8.0f, sd, zd);
    }
    part = wave_sum_xor_groups(part);
    sh.qh[j][lane] = __builtin_bit_cast(u32x4, half8v{vh[0], vh[1], vh[2], vh[3], vh[4], vh[5], vh[6], vh[7]});
    sh.ql[j][lane] = __builtin_bit_cast(u32x4, half8v{vl[0], vl[1], vl[2], vl[3], vl[4], vl[5], vl[6], vl[7]});
    if (lg == 0) sh.bias[j][col] = part;
  }
  __device__ void finish_setup(const QShareLds& sh, const KiviQIn& in, int lane) {
    (void)in;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qh[j] = __builtin_bit_cast(half8v, sh.qh[j][lane]);
      ql[j] = __builtin_bit_cast(half8v, sh.ql[j][lane]);
    }
    const int col = lane & 15;
    bias = (sh.bias[0][col] + sh.bias[1][col]) + (sh.bias[2][col] + sh.bias[3][col]);
  }
  // logits x 2^-24 of the tile's two row blocks: the codes times the hi and the lo operand
  __device__ __forceinline__ void qk(const Raw& r, const NibConsts& nc, float4v& x0,
                                     float4v& x1) const {
    const float b24 = bias * kTwoM24;
    float4v c0 = {b24, b24, b24, b24};
    float4v c1 = c0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half8v a0 = unpack_sub(r.w[0][j], nc), a1 = unpack_sub(r.w[1][j], nc);
      c0 = mfma16x16x32(a0, qh[j], c0);
      c1 = mfma16x16x32(a1, qh[j], c1);
      c0 = mfma16x16x32(a0, ql[j], c0);
      c1 = mfma16x16x32(a1, ql[j], c1);
    }
    x0 = c0;
    x1 = c1;
  }
};

// K of the reference's MixedKVCache at 4 bits: INT4 asymmetric per token
// (src/quant/asymmetric_quant.py:246-270, src/cache/mixed_kv_cache.py:159-162): packed
// nibbles n = c + 8 in dense 64-byte rows and an fp32 scale s_t / zero-point z_t per token
// ([B, H, T], tokens contiguous; INT4_KIVI with per-token K parameters).  The reference
// dequantises K to fp16 before its attention (mixed_kv_cache.py:186-188: (n - 8) s + z in fp32,
// then .to(fp16)), and with outlier channels in the token's range that rounding moves the
// logits by more than the output tolerance allows, so the A operand is exactly that fp16
// value: lane (row, lg) of row block rb dequantises its 32 channels of token 16 rb + row with
// the token's s and z (one dword each per row block), byte to float by v_cvt_f32_ubyte, one
// fma, round to nearest fp16.  The B operand is q' in channel order.  Logits at unit scale.
struct KTokAsymT : KAsymT<false> {
  static constexpr int kRowFmt = KVQ_FMT_INT4_KIVI;  // the fused append's K format
  static constexpr bool kAppend = false;
  static constexpr bool kAppendRow = true;  // the writer runs quant_row_x (fused step)
  static constexpr bool kRescue = false;     // (no INT4_SYM side)
  static constexpr bool kSub24 = false;
  static constexpr bool kPackPV = false;
  rsrc_t rs, rz;
  uint32_t vs;  // lane byte offset of token row (lane & 15) in the parameter rows
  struct Raw {
    u32x4 w[2];
    float s[2], z[2];  // [rb]: the parameters of token 16 rb + row
  };
  __device__ void setup_addr(const DecodeArgs& a, int b, int hkv, int lane) {
    KAsymT<false>::setup_addr(a, b, hkv, lane);
    const int64_t o = slab_off(a.k.ssb, a.k.ssh, b, hkv);
    rs = buffer_rsrc(reinterpret_cast<const float*>(a.k.scale) + o, (uint32_t)(a.cap * 4));
    rz = buffer_rsrc(reinterpret_cast<const float*>(a.k.zp) + o, (uint32_t)(a.cap * 4));
    vs = (uint32_t)(4 * (lane & 15));
  }
  __device__ void fetch_q(const DecodeArgs& a, int b, int hkv, int lane, int wave, QIn& in) const {
    const int col = lane & 15, lg = lane >> 4;
    const int hq = hkv * a.n_rep + (col < a.n_rep ? col : 0);
    in.q = *reinterpret_cast<const u32x4*>(q_row(a, b, hq) + 32 * lg + 8 * (wave & 3));
    in.tau = a.inv_tau != nullptr ? a.inv_tau[hq] : (half_t)1.0f;
    in.s = (half_t)1.0f;
    in.z = (half_t)0.0f;
    in.oc = int4{-1, -1, -1, -1};
  }
  // channel slice j: q' = fp16(q * inv_tau) in channel order
  __device__ void setup_q(const DecodeArgs& a, const QIn& in, int lane, int j, QShareLds& sh) {
    const int col = lane & 15;
    const bool valid = col < a.n_rep;
    const bool has_tau = a.inv_tau != nullptr;
    const uint32_t qw[4] = {in.q.x, in.q.y, in.q.z, in.q.w};
    half_t vh[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const half2v h2 = as_h2(qw[e >> 1]);
      vh[e] = valid ? qscale((e & 1) ? h2.y : h2.x, in.tau, has_tau) : (half_t)0.0f;
    }
    sh.qh[j][lane] = __builtin_bit_cast(u32x4, half8v{vh[0], vh[1], vh[2], vh[3], vh[4], vh[5], vh[6], vh[7]});
  }
  __device__ void finish_setup(const QShareLds& sh, const QIn& in, int lane) {
    (void)in;
#pragma unroll
    for (int j = 0; j < 4; ++j) qh[j] = __builtin_bit_cast(half8v, sh.qh[j][lane]);
  }
  // codes as KAsymT; the parameters of the lane's tokens (0 past the capacity, and for a
  // !valid tile, which touches no memory)
  __device__ __forceinline__ void load(int tok, bool valid, Raw& r) const {
    const uint32_t v = vk + (valid ? (uint32_t)tok * kRowK : kOutOfRange);
    r.w[0] = bload4(rk, v, 0);
    r.w[1] = bload4(rk, v + 16 * kRowK, 0);
    const uint32_t p = vs + (valid ? (uint32_t)tok * 4u : kOutOfRange);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      r.s[rb] = __builtin_bit_cast(float, bload1(rs, p + 64u * rb, 0));
      r.z[rb] = __builtin_bit_cast(float, bload1(rz, p + 64u * rb, 0));
    }
  }
  // fp16((n - 8) s + z) of the 8 codes of dword w (byte b: channel 2 b in the high nibble,
  // 2 b + 1 in the low one), in channel order
  __device__ __forceinline__ static half8v deq8(uint32_t w, float s, float z) {
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu, lo = w & 0x0F0F0F0Fu;
    half_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // (float) of a byte lane compiles to v_cvt_f32_ubyte<k>
      const float n = (float)(((e & 1) ? lo : hi) >> (8 * (e >> 1)) & 0xFFu);
      // the reference's codes.to(fp32) * s + z: a rounded product, then a rounded sum
      h[e] = (half_t)__fadd_rn(__fmul_rn(n - 8.0f, s), z);
    }
    return half8v{h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]};
  }
  __device__ __forceinline__ void qk(const Raw& r, const NibConsts& nc, float4v& x0,
                                     float4v& x1) const {
    (void)nc;
    float4v c[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int j = 0; j < 4; ++j) c[rb] = mfma16x16x32(deq8(r.w[rb][j], r.s[rb], r.z[rb]), qh[j], c[rb]);
    x0 = c[0];
    x1 = c[1];
  }
};

// A tile's 32 packed INT4 token rows (64 bytes each, contiguous) passed through the wave's
// own LDS, for the V operand types that read token rows: lane l loads bytes [16 l, 16 l + 16)
// of each KB half with one 16-byte load (2 per tile instead of 8 dword gathers), writes them
// to rows kRowB = 80 bytes apart (16 bytes of padding put the 4 token rows one read touches
// per lane group in distinct banks), and reads back dword col of its 8 k-slot tokens T(k) =
// 4 lg + {0, 1, 2, 3, 16, 17, 18, 19}, two rows per ds_read2_b32.  LDS operations of one
// wave execute in order, so no barrier is needed.
struct Rows64Lds {
  static constexpr int kRowB = 80;
  static constexpr int kBytes = 32 * kRowB;
  uint32_t lc, wc, rc;
  __device__ void setup(int lane) {
    const int col = lane & 15, lg = lane >> 4;
    lc = (uint32_t)lane * 16u;
    wc = (uint32_t)(lane >> 2) * kRowB + (uint32_t)(lane & 3) * 16u;
    rc = (uint32_t)(4 * lg) * kRowB + (uint32_t)col * 4u;
  }
  // o: the tile's byte offset in the slab (kOutOfRange: nothing loaded)
  __device__ __forceinline__ void load(rsrc_t r, uint32_t o, u32x4& c0, u32x4& c1) const {
    c0 = bload4(r, lc + o, 0);
    c1 = bload4(r, lc + o + 16u * (kD / 2), 0);
  }
  __device__ __forceinline__ void write(uint8_t* base, const u32x4& c0, const u32x4& c1) const {
    *reinterpret_cast<u32x4*>(base + wc) = c0;
    *reinterpret_cast<u32x4*>(base + wc + 16 * kRowB) = c1;
  }
  // w[k]: dword col of token T(k)
  __device__ __forceinline__ void gather(const uint8_t* base, uint32_t w[8]) const {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t dt = p == 0 ? 0u : p == 1 ? 2u : p == 2 ? 16u : 18u;
      const uint32_t* cr = reinterpret_cast<const uint32_t*>(base + rc + dt * kRowB);
      w[2 * p] = cr[0];
      w[2 * p + 1] = cr[kRowB / 4];
    }
  }
};


// V of the KIVI layout in token rows (64 bytes).  Lane (col, lg) reads the dword of
// channels 8 col .. 8 col + 7 of each of its 8 PV k-slot tokens T(k) (four 64-byte rows
// per load instruction) and their fp32 scale / zero-point.  The codes enter the MFMA as
// the exact fp16 subnormals n 2^-24 (odd channel, low nibble) and 16 n 2^-24 (even
// channel, high nibble), and the B operand is w = p s_t (fp32) carried as a hi + lo pair of
// fp16 values (split_h, two MFMAs per operand), so
//   sum_t p v = sum_t w (n - 8) + sum_t p z_t = 2^24 acc (/ 16 for an even channel)
//               - 8 Lp + Cz,   Lp = sum_t (hi + lo),  Cz = sum_t p z_t (fp32),
// with w rounded to about 2^-22 of itself instead of the 2^-11 of one fp16 operand (the
// reference dequantises V in fp32).  The wave keeps Lp and Cz beside l (the softmax
// rescales them with l) and finalize() folds them into acc before the merge (out = acc / l).
template <bool STAGE>
struct VKiviRowTT {
  static constexpr bool kStage = STAGE;  // code rows through LDS (Rows64Lds)
  static constexpr int kRowFmt = KVQ_FMT_INT4_KIVI;  // the fused append's V format
  static constexpr bool kResidual = true;  // merges an fp16 residual window
  static constexpr bool kPackedPV = false;
  static constexpr bool kTile32 = false;
  rsrc_t rv, rs, rz;
  uint32_t vv, vp;
  Rows64Lds cst;  // STAGE
  float ex[2];  // Lp, Cz (rescaled with l by the softmax)
  struct Raw {
    uint32_t w[8];     // token T(k): bytes 4 col .. 4 col + 3
    float4v s[2], z[2];  // tokens 4 lg + i, 16 + 4 lg + i
    u32x4 c0, c1;      // STAGE: the tile's code rows as loaded
  };
  __device__ static void epi_params(const DecodeArgs& a, int hkv, int lane, float& s, float& z) {
    (void)a; (void)hkv; (void)lane;
    s = 1.f;
    z = 0.f;
  }
  __device__ static half2v epilogue(float r0, float r1, float s, float z) {
    (void)s; (void)z;
    return half2v{(half_t)r0, (half_t)r1};
  }
  __device__ void setup(const DecodeArgs& a, int b, int hkv, int lane) {
    const int col = lane & 15, lg = lane >> 4;
    const uint8_t* vb = a.v.codes + slab_off(a.v.sb, a.v.sh, b, hkv);
    rv = buffer_rsrc(vb, (uint32_t)(a.cap * (kD / 2)));
    vv = (uint32_t)((4 * lg) * (kD / 2) + 4 * col);
    const int64_t po = slab_off(a.v.ssb, a.v.ssh, b, hkv);
    rs = buffer_rsrc(reinterpret_cast<const float*>(a.v.scale) + po, (uint32_t)(a.cap * 4));
    rz = buffer_rsrc(reinterpret_cast<const float*>(a.v.zp) + po, (uint32_t)(a.cap * 4));
    vp = (uint32_t)(4 * lg) * 4u;
    ex[0] = ex[1] = 0.f;
    if constexpr (STAGE) cst.setup(lane);
  }
  // STAGE: the tile's code rows through the wave's LDS into w (Rows64Lds)
  __device__ __forceinline__ void stage(Raw& r, int wave) const {
    if constexpr (STAGE) {
      __shared__ __attribute__((aligned(16))) uint8_t vst[kTW][Rows64Lds::kBytes];
      cst.write(vst[wave], r.c0, r.c1);
      cst.gather(vst[wave], r.w);
    } else {
      (void)r;
      (void)wave;
    }
  }
  __device__ __forceinline__ float* extra() { return ex; }
  // rows of a partial last tile past the capacity read 0; !valid: every load out of range
  __device__ __forceinline__ void load(int tok, bool valid, Raw& r) const {
    if constexpr (STAGE) {
      cst.load(rv, valid ? (uint32_t)tok * (kD / 2) : kOutOfRange, r.c0, r.c1);
    } else {
      const uint32_t v = vv + (valid ? (uint32_t)tok * (kD / 2) : kOutOfRange);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t t = (k < 4) ? (uint32_t)k : (uint32_t)(12 + k);  // 16 + k - 4
        r.w[k] = bload1(rv, v + t * (kD / 2), 0);
      }
    }
    const uint32_t p = vp + (valid ? (uint32_t)tok * 4u : kOutOfRange);
    r.s[0] = __builtin_bit_cast(float4v, bload4(rs, p, 0));
    r.s[1] = __builtin_bit_cast(float4v, bload4(rs, p + 64u, 0));
    r.z[0] = __builtin_bit_cast(float4v, bload4(rz, p, 0));
    r.z[1] = __builtin_bit_cast(float4v, bload4(rz, p + 64u, 0));
  }
  // tokens at or past the context in the last, partial tile: parameters 0 (their memory
  // may hold anything; p is 0 there)
  __device__ __forceinline__ void mask(Raw& r, int tt, int ctx, int lg) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (tt + 4 * lg + i >= ctx) r.s[0][i] = r.z[0][i] = 0.f;
      if (tt + 16 + 4 * lg + i >= ctx) r.s[1][i] = r.z[1][i] = 0.f;
    }
  }
  __device__ __forceinline__ void mma(const Raw& r, half8v pb, half8v plo, float4v acc[8],
                                      const NibConsts& nc) {
    float sk[8], wk[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sk[i] = r.s[0][i];
      sk[4 + i] = r.s[1][i];
      wk[i] = r.z[0][i];
      wk[4 + i] = r.z[1][i];
    }
    float cz = ex[1];
    uint32_t ph[4], pl[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float p0 = (float)pb[2 * q] + (float)plo[2 * q];
      const float p1 = (float)pb[2 * q + 1] + (float)plo[2 * q + 1];
      cz = fmaf(p0, wk[2 * q], cz);
      cz = fmaf(p1, wk[2 * q + 1], cz);
      half_t h0, l0, h1, l1;
      split_h(p0 * sk[2 * q], h0, l0);
      split_h(p1 * sk[2 * q + 1], h1, l1);
      ph[q] = as_u32(half2v{h0, h1});
      pl[q] = as_u32(half2v{l0, l1});
    }
    ex[1] = cz;
    const half2v ones = {(half_t)1.0f, (half_t)1.0f};
    float lp = ex[0];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      lp = __builtin_amdgcn_fdot2(as_h2(ph[q]), ones, lp, false);
      lp = __builtin_amdgcn_fdot2(as_h2(pl[q]), ones, lp, false);
    }
    ex[0] = lp;
    const half8v wh = pack8(ph[0], ph[1], ph[2], ph[3]);
    const half8v wl = pack8(pl[0], pl[1], pl[2], pl[3]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // byte j of the tokens T(2p), T(2p + 1) into the low bytes of the two halves
      const uint32_t sel = (uint32_t)j | 0x0C00u | ((uint32_t)(4 + j) << 16) | 0x0C000000u;
      uint32_t R[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) R[p] = perm_b32(r.w[2 * p + 1], r.w[2 * p], sel);
      const half8v ahi = pack8(R[0] & nc.m_hi, R[1] & nc.m_hi, R[2] & nc.m_hi, R[3] & nc.m_hi);
      const half8v alo = pack8(R[0] & nc.m_lo, R[1] & nc.m_lo, R[2] & nc.m_lo, R[3] & nc.m_lo);
      acc[2 * j] = mfma16x16x32(ahi, wh, acc[2 * j]);
      acc[2 * j + 1] = mfma16x16x32(alo, wh, acc[2 * j + 1]);
      acc[2 * j] = mfma16x16x32(ahi, wl, acc[2 * j]);
      acc[2 * j + 1] = mfma16x16x32(alo, wl, acc[2 * j + 1]);
    }
  }
  // acc[mb][r] (channel 32 lg + 8 r + mb) = 2^24 acc (2^20 for an even channel, whose codes
  // entered as 16 n 2^-24) - 8 Lp + Cz, with Lp, Cz summed over the lane groups (the k-slots
  // of a head)
  __device__ __forceinline__ void finalize(float4v acc[8], int lane) {
    (void)lane;
    const float lp = wave_sum_xor_groups(ex[0]), cz = wave_sum_xor_groups(ex[1]);
    const float d = fmaf(-8.0f, lp, cz);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const float f = (mb & 1) ? kTwo24 : kTwo24 * 0.0625f;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[mb][r] = fmaf(acc[mb][r], f, d);
    }
  }
};
using VKiviRowT = VKiviRowTT<false>;
// the same with the code rows read by 16-byte loads and gathered through LDS (16-byte aligned
// code rows)
using VKiviRowTS = VKiviRowTT<true>;

// ---- The KIVI family with 8-bit codes and 16-bit sides: the reference's quant_bits=8 KIVI
// cache (src/cache/kivi_style_cache.py) and the per-layer (k_bits, v_bits) pairs of its
// allocator and mixed caches (src/cache/role_aware_allocator_cache.py,
// src/cache/mixed_kv_cache.py), where a 16-bit side stores fp16 values as they come.

// Two int8 codes (the low bytes of the two halves of x, the high bytes zero) -> the exact
// fp16 pair: x ^ 0x64806480 gives 1024 + (c + 128), minus 1152 gives c.
__device__ __forceinline__ uint32_t i8pair_exact(uint32_t x) {
  const half2v off = {(half_t)1152.0f, (half_t)1152.0f};
  return as_u32(as_h2(x ^ 0x64806480u) - off);
}

// K of the 8-bit KIVI layout: int8 codes in 128-byte token rows with per-channel fp32 scale
// s_d and zero-point z_d per (b, kv head).  logit = sum_d q'_d (c_d s_d + z_d): the codes
// enter the MFMA exactly (i8pair_exact), q'_d s_d as a hi + lo pair of fp16 operands (two
// MFMAs per slice, as KKiviT), and the constant sum_d q'_d z_d starts the accumulator.
// Lane (row, lg) of row block rb reads bytes [32 lg, 32 lg + 32) of token 16 rb + row.
struct KKivi8T {
  static constexpr int kRowFmt = KVQ_FMT_INT8_KIVI;  // the fused append's K format
  static constexpr int kMergeBatch = 8;
  static constexpr bool kPackPV = false;
  using QInT = KiviQIn;
  static constexpr bool kAppend = false;
  static constexpr bool kAppendRow = true;  // the writer runs quant_row_x (fused step)
  static constexpr bool kRescue = false;     // (no INT4_SYM side)
  static constexpr bool kAsym = false;
  static constexpr bool kGsAny = false;
  static constexpr bool kOut = false;
  static constexpr bool kSub24 = false;  // logits at unit scale
  half8v qh[4], ql[4];
  float bias;
  rsrc_t rk;
  uint32_t vk;
  struct Raw {
    u32x4 w[4];  // [2 rb + i]: bytes [32 lg + 16 i, + 16) of token 16 rb + row
  };
  __device__ void setup_addr(const DecodeArgs& a, int b, int hkv, int lane) {
    const int col = lane & 15, lg = lane >> 4;
    const uint8_t* kb = a.k.codes + slab_off(a.k.sb, a.k.sh, b, hkv);
    rk = buffer_rsrc(kb, (uint32_t)(a.cap * kD));
    vk = (uint32_t)(col * kD + 32 * lg);
  }
  __device__ void fetch_q(const DecodeArgs& a, int b, int hkv, int lane, int wave, KiviQIn& in) const {
    const int col = lane & 15, lg = lane >> 4;
    const int hq = hkv * a.n_rep + (col < a.n_rep ? col : 0);
    in.q = *reinterpret_cast<const u32x4*>(q_row(a, b, hq) + 32 * lg + 8 * (wave & 3));
    in.tau = a.inv_tau != nullptr ? a.inv_tau[hq] : (half_t)1.0f;
    in.oc = int4{-1, -1, -1, -1};
    const int64_t o = slab_off(a.k.ssb, a.k.ssh, b, hkv) + 32 * lg + 8 * (wave & 3);
    const float* ps = reinterpret_cast<const float*>(a.k.scale) + o;
    const float* pz = reinterpret_cast<const float*>(a.k.zp) + o;
    in.ks[0] = *reinterpret_cast<const float4v*>(ps);
    in.ks[1] = *reinterpret_cast<const float4v*>(ps + 4);
    in.kz[0] = *reinterpret_cast<const float4v*>(pz);
    in.kz[1] = *reinterpret_cast<const float4v*>(pz + 4);
  }
  // channel slice j (channels 32 lg + 8 j + e, in channel order)
  __device__ void setup_q(const DecodeArgs& a, const KiviQIn& in, int lane, int j, QShareLds& sh) {
    const int col = lane & 15, lg = lane >> 4;
    const bool valid = col < a.n_rep;
    const bool has_tau = a.inv_tau != nullptr;
    const uint32_t qw[4] = {in.q.x, in.q.y, in.q.z, in.q.w};
    float part = 0.f;
    half_t vh[8], vl[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const half2v h2 = as_h2(qw[e >> 1]);
      const float qd = valid ? (float)qscale((e & 1) ? h2.y : h2.x, in.tau, has_tau) : 0.f;
      split_h(qd * in.ks[e >> 2][e & 3], vh[e], vl[e]);
      part = fmaf(qd, in.kz[e >> 2][e & 3], part);
    }
    part = wave_sum_xor_groups(part);
    sh.qh[j][lane] = __builtin_bit_cast(u32x4, half8v{vh[0], vh[1], vh[2], vh[3], vh[4], vh[5], vh[6], vh[7]});
    sh.ql[j][lane] = __builtin_bit_cast(u32x4, half8v{vl[0], vl[1], vl[2], vl[3], vl[4], vl[5], vl[6], vl[7]});
    if (lg == 0) sh.bias[j][col] = part;
  }
  __device__ void finish_setup(const QShareLds& sh, const KiviQIn& in, int lane) {
    (void)in;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qh[j] = __builtin_bit_cast(half8v, sh.qh[j][lane]);
      ql[j] = __builtin_bit_cast(half8v, sh.ql[j][lane]);
    }
    const int col = lane & 15;
    bias = (sh.bias[0][col] + sh.bias[1][col]) + (sh.bias[2][col] + sh.bias[3][col]);
  }
  __device__ __forceinline__ void load(int tok, bool valid, Raw& r) const {
    const uint32_t v = vk + (valid ? (uint32_t)tok * kD : kOutOfRange);
    r.w[0] = bload4(rk, v, 0);
    r.w[1] = bload4(rk, v + 16, 0);
    r.w[2] = bload4(rk, v + 16 * kD, 0);
    r.w[3] = bload4(rk, v + 16 * kD + 16, 0);
  }
  __device__ __forceinline__ static half8v codes8(uint32_t lo, uint32_t hi) {
    return pack8(i8pair_exact(perm_b32(0u, lo, 0x0C010C00u)), i8pair_exact(perm_b32(0u, lo, 0x0C030C02u)),
                 i8pair_exact(perm_b32(0u, hi, 0x0C010C00u)), i8pair_exact(perm_b32(0u, hi, 0x0C030C02u)));
  }
  __device__ __forceinline__ void qk(const Raw& r, const NibConsts& nc, float4v& x0,
                                     float4v& x1) const {
    (void)nc;
    float4v c0 = {bias, bias, bias, bias};
    float4v c1 = c0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 w0 = r.w[j >> 1], w1 = r.w[2 + (j >> 1)];
      const half8v a0 = codes8((j & 1) ? w0.z : w0.x, (j & 1) ? w0.w : w0.y);
      const half8v a1 = codes8((j & 1) ? w1.z : w1.x, (j & 1) ? w1.w : w1.y);
      c0 = mfma16x16x32(a0, qh[j], c0);
      c1 = mfma16x16x32(a1, qh[j], c1);
      c0 = mfma16x16x32(a0, ql[j], c0);
      c1 = mfma16x16x32(a1, ql[j], c1);
    }
    x0 = c0;
    x1 = c1;
  }
};

// fp16 K in 256-byte token rows (a 16-bit K side): the logits are the fp32 dot products of
// the stored fp16 k with q' = fp16(q * inv_tau).  Lane (row, lg) of row block rb reads bytes
// [64 lg, 64 lg + 64) of token 16 rb + row: channels 32 lg + 8 j .. + 7 are slice j.
struct KF16T {
  static constexpr int kRowFmt = KVQ_FMT_FP16;  // the fused append's K format
  static constexpr int kMergeBatch = 8;
  static constexpr bool kPackPV = false;
  using QInT = QIn;
  static constexpr bool kAppend = false;
  static constexpr bool kAppendRow = true;  // the writer runs quant_row_x (fused step)
  static constexpr bool kRescue = false;     // (no INT4_SYM side)
  static constexpr bool kAsym = false;
  static constexpr bool kGsAny = false;
  static constexpr bool kOut = false;
  static constexpr bool kSub24 = false;
  static constexpr int kRow = 2 * kD;
  half8v qh[4];
  rsrc_t rk;
  uint32_t vk;
  struct Raw {
    u32x4 w[8];  // [4 rb + j]: slice j of token 16 rb + row
  };
  __device__ void setup_addr(const DecodeArgs& a, int b, int hkv, int lane) {
    const int col = lane & 15, lg = lane >> 4;
    const uint8_t* kb = a.k.codes + slab_off(a.k.sb, a.k.sh, b, hkv);
    rk = buffer_rsrc(kb, (uint32_t)(a.cap * kRow));
    vk = (uint32_t)(col * kRow + 64 * lg);
  }
  __device__ void fetch_q(const DecodeArgs& a, int b, int hkv, int lane, int wave, QIn& in) const {
    const int col = lane & 15, lg = lane >> 4;
    const int hq = hkv * a.n_rep + (col < a.n_rep ? col : 0);
    in.q = *reinterpret_cast<const u32x4*>(q_row(a, b, hq) + 32 * lg + 8 * (wave & 3));
    in.tau = a.inv_tau != nullptr ? a.inv_tau[hq] : (half_t)1.0f;
    in.s = (half_t)1.0f;
    in.z = (half_t)0.0f;
    in.oc = int4{-1, -1, -1, -1};
  }
  __device__ void setup_q(const DecodeArgs& a, const QIn& in, int lane, int j, QShareLds& sh) {
    const int col = lane & 15;
    const bool valid = col < a.n_rep;
    const bool has_tau = a.inv_tau != nullptr;
    const uint32_t qw[4] = {in.q.x, in.q.y, in.q.z, in.q.w};
    half_t vh[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const half2v h2 = as_h2(qw[e >> 1]);
      vh[e] = valid ? qscale((e & 1) ? h2.y : h2.x, in.tau, has_tau) : (half_t)0.0f;
    }
    sh.qh[j][lane] = __builtin_bit_cast(u32x4, half8v{vh[0], vh[1], vh[2], vh[3], vh[4], vh[5], vh[6], vh[7]});
  }
  __device__ void finish_setup(const QShareLds& sh, const QIn& in, int lane) {
    (void)in;
#pragma unroll
    for (int j = 0; j < 4; ++j) qh[j] = __builtin_bit_cast(half8v, sh.qh[j][lane]);
  }
  __device__ __forceinline__ void load(int tok, bool valid, Raw& r) const {
    const uint32_t v = vk + (valid ? (uint32_t)tok * kRow : kOutOfRange);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      r.w[j] = bload4(rk, v + 16 * j, 0);
      r.w[4 + j] = bload4(rk, v + 16 * kRow + 16 * j, 0);
    }
  }
  __device__ __forceinline__ void qk(const Raw& r, const NibConsts& nc, float4v& x0,
                                     float4v& x1) const {
    (void)nc;
    float4v c0 = {0.f, 0.f, 0.f, 0.f};
    float4v c1 = c0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c0 = mfma16x16x32(__builtin_bit_cast(half8v, r.w[j]), qh[j], c0);
      c1 = mfma16x16x32(__builtin_bit_cast(half8v, r.w[4 + j]), qh[j], c1);
    }
    x0 = c0;
    x1 = c1;
  }
};

// V of the 8-bit KIVI layout in 128-byte token rows, per-token fp32 s_t, z_t: lane (col, lg)
// reads the 8 bytes of channels 8 col .. 8 col + 7 of each of its 8 PV k-slot tokens T(k)
// (as VI8RowT) and the tokens' s, z (as VKiviRowT).  The codes enter the MFMA exactly
// (i8pair_exact), the B operand is w = p s_t as a hi + lo pair (two MFMAs per channel), and
//   sum_t p v = sum_t w c + Cz,   Cz = sum_t p z_t (fp32, rescaled with l by the softmax).
struct VKivi8RowT {
  static constexpr int kRowFmt = KVQ_FMT_INT8_KIVI;  // the fused append's V format
  static constexpr bool kResidual = true;  // merges an fp16 residual window
  static constexpr bool kPackedPV = false;
  static constexpr bool kTile32 = false;
  rsrc_t rv, rs, rz;
  uint32_t vv, vp;
  float ex[2];  // unused, Cz
  struct Raw {
    u32x2 w[8];          // token T(k): bytes 8 col .. 8 col + 7
    float4v s[2], z[2];  // tokens 4 lg + i, 16 + 4 lg + i
  };
  __device__ static void epi_params(const DecodeArgs& a, int hkv, int lane, float& s, float& z) {
    (void)a; (void)hkv; (void)lane;
    s = 1.f;
    z = 0.f;
  }
  __device__ static half2v epilogue(float r0, float r1, float s, float z) {
    (void)s; (void)z;
    return half2v{(half_t)r0, (half_t)r1};
  }
  __device__ void setup(const DecodeArgs& a, int b, int hkv, int lane) {
    const int col = lane & 15, lg = lane >> 4;
    const uint8_t* vb = a.v.codes + slab_off(a.v.sb, a.v.sh, b, hkv);
    rv = buffer_rsrc(vb, (uint32_t)(a.cap * kD));
    vv = (uint32_t)((4 * lg) * kD + 8 * col);
    const int64_t po = slab_off(a.v.ssb, a.v.ssh, b, hkv);
    rs = buffer_rsrc(reinterpret_cast<const float*>(a.v.scale) + po, (uint32_t)(a.cap * 4));
    rz = buffer_rsrc(reinterpret_cast<const float*>(a.v.zp) + po, (uint32_t)(a.cap * 4));
    vp = (uint32_t)(4 * lg) * 4u;
    ex[0] = ex[1] = 0.f;
  }
  __device__ __forceinline__ float* extra() { return ex; }
  __device__ __forceinline__ void load(int tok, bool valid, Raw& r) const {
    const uint32_t v = vv + (valid ? (uint32_t)tok * kD : kOutOfRange);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t t = (k < 4) ? (uint32_t)k : (uint32_t)(12 + k);  // 16 + k - 4
      r.w[k] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rv, (int)(v + t * kD), 0, kBufNT));
    }
    const uint32_t p = vp + (valid ? (uint32_t)tok * 4u : kOutOfRange);
    r.s[0] = __builtin_bit_cast(float4v, bload4(rs, p, 0));
    r.s[1] = __builtin_bit_cast(float4v, bload4(rs, p + 64u, 0));
    r.z[0] = __builtin_bit_cast(float4v, bload4(rz, p, 0));
    r.z[1] = __builtin_bit_cast(float4v, bload4(rz, p + 64u, 0));
  }
  // tokens at or past the context in the last, partial tile: parameters 0
  __device__ __forceinline__ void mask(Raw& r, int tt, int ctx, int lg) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (tt + 4 * lg + i >= ctx) r.s[0][i] = r.z[0][i] = 0.f;
      if (tt + 16 + 4 * lg + i >= ctx) r.s[1][i] = r.z[1][i] = 0.f;
    }
  }
  __device__ __forceinline__ void mma(const Raw& r, half8v pb, half8v plo, float4v acc[8],
                                      const NibConsts& nc) {
    (void)nc;
    float sk[8], wk[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sk[i] = r.s[0][i];
      sk[4 + i] = r.s[1][i];
      wk[i] = r.z[0][i];
      wk[4 + i] = r.z[1][i];
    }
    float cz = ex[1];
    uint32_t ph[4], pl[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float p0 = (float)pb[2 * q] + (float)plo[2 * q];
      const float p1 = (float)pb[2 * q + 1] + (float)plo[2 * q + 1];
      cz = fmaf(p0, wk[2 * q], cz);
      cz = fmaf(p1, wk[2 * q + 1], cz);
      half_t h0, l0, h1, l1;
      split_h(p0 * sk[2 * q], h0, l0);
      split_h(p1 * sk[2 * q + 1], h1, l1);
      ph[q] = as_u32(half2v{h0, h1});
      pl[q] = as_u32(half2v{l0, l1});
    }
    ex[1] = cz;
    const half8v wh = pack8(ph[0], ph[1], ph[2], ph[3]);
    const half8v wl = pack8(pl[0], pl[1], pl[2], pl[3]);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      // byte c % 4 of the tokens T(2p) and T(2p + 1) into the low bytes of the two halves
      const uint32_t sel = (uint32_t)(c & 3) | 0x0C00u | ((uint32_t)(4 + (c & 3)) << 16) | 0x0C000000u;
      uint32_t R[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t lo = (c >> 2) ? r.w[2 * p].y : r.w[2 * p].x;
        const uint32_t hi = (c >> 2) ? r.w[2 * p + 1].y : r.w[2 * p + 1].x;
        R[p] = i8pair_exact(perm_b32(hi, lo, sel));
      }
      const half8v av = pack8(R[0], R[1], R[2], R[3]);
      acc[c] = mfma16x16x32(av, wh, acc[c]);
      acc[c] = mfma16x16x32(av, wl, acc[c]);
    }
  }
  // acc[mb][r] += Cz, summed over the lane groups (the k-slots of a head)
  __device__ __forceinline__ void finalize(float4v acc[8], int lane) {
    (void)lane;
    const float cz = wave_sum_xor_groups(ex[1]);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[mb][r] += cz;
  }
};

// fp16 V in 256-byte token rows (a 16-bit V side): lane (col, lg) reads the 16 bytes of
// channels 8 col .. 8 col + 7 of each of its 8 PV k-slot tokens; the A operand of channel
// 8 col + c is the stored v of the 8 tokens (one v_perm_b32 per token pair), so acc / l is
// the output.
struct VF16RowT {
  static constexpr int kRowFmt = KVQ_FMT_FP16;  // the fused append's V format
  static constexpr bool kResidual = true;  // merges an fp16 residual window
  static constexpr bool kPackedPV = false;
  static constexpr bool kTile32 = false;
  static constexpr int kRow = 2 * kD;
  __device__ __forceinline__ void finalize(float4v*, int) const {}
  __device__ __forceinline__ float* extra() { return nullptr; }
  rsrc_t rv;
  uint32_t vv;
  struct Raw {
    u32x4 w[8];  // token T(k): channels 8 col .. 8 col + 7
  };
  // tokens at or past the context in the last, partial tile read as 0: their probability is
  // 0, but the memory may hold any fp16 bits, and 0 x inf or 0 x NaN would reach acc
  __device__ __forceinline__ void mask(Raw& r, int tt, int ctx, int lg) const {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int t = tt + (k < 4 ? 4 * lg + k : 12 + 4 * lg + k);
      if (t >= ctx) r.w[k] = u32x4{0u, 0u, 0u, 0u};
    }
  }
  __device__ static void epi_params(const DecodeArgs& a, int hkv, int lane, float& s, float& z) {
    (void)a; (void)hkv; (void)lane;
    s = 1.f;
    z = 0.f;
  }
  __device__ static half2v epilogue(float r0, float r1, float s, float z) {
    (void)s; (void)z;
    return half2v{(half_t)r0, (half_t)r1};
  }
  __device__ void setup(const DecodeArgs& a, int b, int hkv, int lane) {
    const int col = lane & 15, lg = lane >> 4;
    const uint8_t* vb = a.v.codes + slab_off(a.v.sb, a.v.sh, b, hkv);
    rv = buffer_rsrc(vb, (uint32_t)(a.cap * kRow));
    vv = (uint32_t)((4 * lg) * kRow + 16 * col);
  }
  __device__ __forceinline__ void load(int tok, bool valid, Raw& r) const {
    const uint32_t v = vv + (valid ? (uint32_t)tok * kRow : kOutOfRange);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t t = (k < 4) ? (uint32_t)k : (uint32_t)(12 + k);  // 16 + k - 4
      r.w[k] = bload4(rv, v + t * kRow, 0);
    }
  }
  __device__ __forceinline__ void mma(const Raw& r, half8v pb, half8v pl, float4v acc[8],
                                      const NibConsts& nc) const {
    (void)nc;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      // half c % 2 of dword c / 2 of the tokens T(2p), T(2p + 1) -> the two halves
      const uint32_t b0 = 2u * (uint32_t)(c & 1);
      const uint32_t sel = b0 | ((b0 + 1) << 8) | ((b0 + 4) << 16) | ((b0 + 5) << 24);
      uint32_t R[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) R[p] = perm_b32(r.w[2 * p + 1][c >> 1], r.w[2 * p][c >> 1], sel);
      const half8v av = pack8(R[0], R[1], R[2], R[3]);
      acc[c] = mfma16x16x32(av, pb, acc[c]);
      acc[c] = mfma16x16x32(av, pl, acc[c]);
    }
  }
};

// ---- Per-token scales: INT8 codes with fp16 scales or packed INT4-symmetric codes with fp32
// scales per (b, kv head, token, group), in token rows (the reference's dynamic, adaptive and
// group-rescue caches, src/cache/int8_cache.py:298-488, src/cache/int4_cache.py:298-590, read
// by src/kernels/triton_decode_attn_int8.py:306-519 and triton_decode_attn_int4.py:62-121).
// Both sides are dequantised as the reference's torch path does, k = fp16(c * fp16(s)), and
// enter the MFMAs as fp16 values (the arithmetic of the row kernel's KTok / VTok).  A static
// table given as a stride-0 view reads like per-token scales (every token one line).
// NS = scales of a K lane's 32 channels: 1 for groups of 32 or more, 2 for groups of 16.
// bytes of a (b, kv head)'s per-token scale rows: cap rows of stride sst elements, or one
// row of 128 / gs groups for a stride-0 (static) view
__device__ __forceinline__ uint32_t scale_bytes(int64_t cap, int64_t sst, int gs, int es) {
  return (uint32_t)(sst > 0 ? cap * sst * es : (int64_t)(kD / gs) * es);
}

template <bool I4, int NS>
struct KTokT {
  static constexpr int kRowFmt = I4 ? KVQ_FMT_INT4_SYM : KVQ_FMT_INT8_SYM;  // the fused append's K format
  static_assert(NS == 1 || NS == 2, "groups of 16 or more");
  // (16 cost the per-token INT8 / INT4 baselines 0.35 / 0.6 us per launch at config 3's
  // shape, 8 chunks per (b, kv head))
  static constexpr int kMergeBatch = 8;
  static constexpr bool kPackPV = false;
  using QInT = QIn;
  static constexpr bool kAppend = false;
  // the writer runs quant_row_x (fused step); with INT4_SYM sides it also finds the group
  // rescue's threshold over every row of the append (rescue_thr_wave)
  static constexpr bool kAppendRow = true;
  static constexpr bool kRescue = I4;
  static constexpr bool kAsym = false;
  static constexpr bool kGsAny = true;
  static constexpr bool kOut = false;
  static constexpr bool kSub24 = false;  // logits at unit scale
  static constexpr int kRow = I4 ? kD / 2 : kD;  // code bytes per token
  static constexpr int kEs = I4 ? 4 : 2;         // scale bytes (fp32 / fp16)
  half8v qh[4];
  rsrc_t rk, rs;
  uint32_t vk, vs, sst;  // lane code offset, lane scale offset, scale bytes per token
  struct Raw {
    u32x4 w[I4 ? 2 : 4];  // I4: [rb] = bytes [16 lg, 16 lg + 16) of token 16 rb + row;
                          // INT8: [2 rb + i] = bytes [32 lg + 16 i, + 16)
    uint32_t s[2];        // the NS scales of row block rb (fp16 pair, fp16 or fp32 bits)
    uint32_t s2[I4 && NS == 2 ? 2 : 1];  // the second fp32 scale of row block rb (NS = 2)
  };

  __device__ void setup_addr(const DecodeArgs& a, int b, int hkv, int lane) {
    const int col = lane & 15, lg = lane >> 4;
    const uint8_t* kb = a.k.codes + slab_off(a.k.sb, a.k.sh, b, hkv);
    rk = buffer_rsrc(kb, (uint32_t)(a.cap * kRow));
    vk = (uint32_t)(col * kRow + (kRow / 4) * lg);
    // the lane's first group: 32 lg / gs; with NS = 2 the next one follows (stride_g = 1)
    const int g0 = (32 * lg) >> __builtin_ctz((unsigned)a.gs);
    const char* sb = reinterpret_cast<const char*>(a.k.scale) +
                     slab_off(a.k.ssb, a.k.ssh, b, hkv) * kEs;
    sst = (uint32_t)(a.k.sst * kEs);
    rs = buffer_rsrc(sb, scale_bytes(a.cap, a.k.sst, a.gs, kEs));
    vs = (uint32_t)(col * sst + g0 * a.k.ssg * kEs);
  }
  __device__ void fetch_q(const DecodeArgs& a, int b, int hkv, int lane, int wave, QIn& in) const {
    const int col = lane & 15, lg = lane >> 4;
    const int hq = hkv * a.n_rep + (col < a.n_rep ? col : 0);
    in.q = *reinterpret_cast<const u32x4*>(q_row(a, b, hq) + 32 * lg + 8 * (wave & 3));
    in.tau = a.inv_tau != nullptr ? a.inv_tau[hq] : (half_t)1.0f;
    in.s = (half_t)1.0f;
    in.z = (half_t)0.0f;
    in.oc = int4{-1, -1, -1, -1};
  }
  // channel slice j of the q operand q' = fp16(q * inv_tau), in the k-slot order of the
  // codes (INT4: unpack_dword_64pn's), shared through LDS
  __device__ void setup_q(const DecodeArgs& a, const QIn& in, int lane, int j, QShareLds& sh) {
    const int col = lane & 15;
    const bool valid = col < a.n_rep;
    const bool has_tau = a.inv_tau != nullptr;
    const uint32_t qw[4] = {in.q.x, in.q.y, in.q.z, in.q.w};
    half_t vh[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int el = I4 ? kNibSlotElem(e) : e;
      const half2v h2 = as_h2(qw[el >> 1]);
      vh[e] = valid ? qscale((el & 1) ? h2.y : h2.x, in.tau, has_tau) : (half_t)0.0f;
    }
    sh.qh[j][lane] = __builtin_bit_cast(u32x4, half8v{vh[0], vh[1], vh[2], vh[3], vh[4], vh[5], vh[6], vh[7]});
  }
  __device__ void finish_setup(const QShareLds& sh, const QIn& in, int lane) {
    (void)in;
#pragma unroll
    for (int j = 0; j < 4; ++j) qh[j] = __builtin_bit_cast(half8v, sh.qh[j][lane]);
  }
  __device__ __forceinline__ void load(int tok, bool valid, Raw& r) const {
    const uint32_t v = vk + (valid ? (uint32_t)tok * kRow : kOutOfRange);
    if constexpr (I4) {
      r.w[0] = bload4(rk, v, 0);
      r.w[1] = bload4(rk, v + 16 * kRow, 0);
    } else {
      r.w[0] = bload4(rk, v, 0);
      r.w[1] = bload4(rk, v + 16, 0);
      r.w[2] = bload4(rk, v + 16 * kRow, 0);
      r.w[3] = bload4(rk, v + 16 * kRow + 16, 0);
    }
    const uint32_t p = vs + (valid ? (uint32_t)tok * sst : kOutOfRange);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const uint32_t o = p + (uint32_t)rb * 16u * sst;
      if constexpr (I4 && NS == 2) {
        const u32x2 s = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, (int)o, 0, kBufNT));
        r.s[rb] = s.x;
        r.s2[rb] = s.y;
      } else if constexpr (I4 || NS == 2) {
        r.s[rb] = bload1(rs, o, 0);  // one fp32, or two fp16
      } else {
        r.s[rb] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)o, 0, kBufNT);
      }
    }
  }
  // the fp16 scale of slice j in row block rb, twice
  __device__ __forceinline__ uint32_t scale2(const Raw& r, int rb, int j) const {
    half_t s;
    if constexpr (I4) {
      const uint32_t bits = (NS == 2 && j >= 2) ? r.s2[rb] : r.s[rb];
      s = (half_t)__builtin_bit_cast(float, bits);
    } else {
      const half2v h = as_h2(r.s[rb]);
      s = (NS == 2 && j >= 2) ? h.y : h.x;
    }
    return splat_h2(s);
  }
  __device__ __forceinline__ void qk(const Raw& r, const NibConsts& nc, float4v& x0,
                                     float4v& x1) const {
    float4v c[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t s2 = scale2(r, rb, j);
        uint32_t u[4];
        if constexpr (I4) {
          const u32x4 w = r.w[rb];
          const uint32_t d = j == 0 ? w.x : j == 1 ? w.y : j == 2 ? w.z : w.w;
          unpack_dword_64pn(d, nc, u);
#pragma unroll
          for (int i = 0; i < 4; ++i) u[i] = deq_pair(u[i], (half_t)72.0f, s2);
        } else {
          const u32x4 w = r.w[2 * rb + (j >> 1)];
          const uint32_t lo = (j & 1) ? w.z : w.x, hi = (j & 1) ? w.w : w.y;
          u[0] = i8pair_deq(perm_b32(0u, lo, 0x0C010C00u), as_h2(s2));
          u[1] = i8pair_deq(perm_b32(0u, lo, 0x0C030C02u), as_h2(s2));
          u[2] = i8pair_deq(perm_b32(0u, hi, 0x0C010C00u), as_h2(s2));
          u[3] = i8pair_deq(perm_b32(0u, hi, 0x0C030C02u), as_h2(s2));
        }
        c[rb] = mfma16x16x32(pack8(u[0], u[1], u[2], u[3]), qh[j], c[rb]);
      }
    }
    x0 = c[0];
    x1 = c[1];
  }
};

// V with per-token scales in token rows: lane (col, lg) reads channels 8 col .. 8 col + 7
// (8 INT8 bytes or 4 packed INT4 bytes) of its 8 PV k-slot tokens T(k) = 4 lg + k (k < 4),
// 16 + 4 lg + k - 4, and the scale of their group (8 col) / gs.  The A operand of MFMA c
// (channel 8 col + c) is vhat = fp16(c * fp16(s)) of the 8 tokens, so acc / l is the output.
// STAGE (INT4 only; groups of 16 or 32 in dense scale rows, 16-byte aligned): the tile's 2 KB of code rows and its
// block of scales are read with 16-byte loads (lane l: bytes [16 l, 16 l + 16) of each) and
// passed through the wave's own LDS (stage()), from which each lane reads its gathered
// operands with ds_read2_b32; the same operands reach the MFMAs as with the 8 + 8 dword
// gathers per lane and tile that the other instantiation issues.
template <bool I4, bool STAGE = false>
struct VTokT {
  static constexpr bool kStage = I4 && STAGE;
  // LDS layout of a staged tile (per wave): the 32 code rows (Rows64Lds), then the 32 scale
  // rows (16 or 32 bytes: groups of 32 or 16), 48 bytes apart (so that the 4 rows one read
  // touches per lane group fall in distinct banks)
  static constexpr int kSRow = 48;
  static constexpr int kSOff = Rows64Lds::kBytes;
  static constexpr int kStageBytes = kSOff + 32 * kSRow;
  static constexpr int kRowFmt = I4 ? KVQ_FMT_INT4_SYM : KVQ_FMT_INT8_SYM;  // the fused append's V format
  static constexpr bool kResidual = false;  // merges an fp16 residual window
  static constexpr bool kPackedPV = false;
  static constexpr bool kTile32 = false;
  static constexpr int kRow = I4 ? kD / 2 : kD;
  static constexpr int kEs = I4 ? 4 : 2;
  __device__ __forceinline__ void finalize(float4v*, int) const {}
  __device__ __forceinline__ float* extra() { return nullptr; }
  rsrc_t rv, rs;
  uint32_t vv, vs, sst;
  // kStage: the code rows' staging, the lane's scale-block load offset, LDS write offset and
  // read base
  Rows64Lds cst;
  uint32_t ls, ws, rsb;
  struct Raw {
    uint32_t w[8][I4 ? 1 : 2];  // token T(k)
    uint32_t s[8];              // token T(k)'s scale (fp32 or fp16 bits)
    u32x4 c0, c1, sc;           // kStage: the tile as loaded (16 bytes per lane of each)
  };
  __device__ static void epi_params(const DecodeArgs& a, int hkv, int lane, float& s, float& z) {
    (void)a; (void)hkv; (void)lane;
    s = 1.f;
    z = 0.f;
  }
  __device__ static half2v epilogue(float r0, float r1, float s, float z) {
    (void)s; (void)z;
    return half2v{(half_t)r0, (half_t)r1};
  }
  __device__ void setup(const DecodeArgs& a, int b, int hkv, int lane) {
    const int col = lane & 15, lg = lane >> 4;
    const uint8_t* vb = a.v.codes + slab_off(a.v.sb, a.v.sh, b, hkv);
    rv = buffer_rsrc(vb, (uint32_t)(a.cap * kRow));
    vv = (uint32_t)((4 * lg) * kRow + (I4 ? 4 : 8) * col);
    const int gi = (8 * col) >> __builtin_ctz((unsigned)a.vgs);
    const char* sb = reinterpret_cast<const char*>(a.v.scale) +
                     slab_off(a.v.ssb, a.v.ssh, b, hkv) * kEs;
    sst = (uint32_t)(a.v.sst * kEs);
    rs = buffer_rsrc(sb, scale_bytes(a.cap, a.v.sst, a.vgs, kEs));
    vs = (uint32_t)((4 * lg) * sst + gi * a.v.ssg * kEs);
    if constexpr (kStage) {
      // a token's scale row: sst = 4 * (128 / gs) bytes, 32 (groups of 16) or 16 (of 32)
      const uint32_t byte = (uint32_t)lane * 16u;
      cst.setup(lane);
      ls = byte < 32u * sst ? byte : kOutOfRange;
      ws = kSOff + (byte / sst) * kSRow + byte % sst;
      // pair p reads the scales of tokens T(2 p), T(2 p) + 1 = 4 lg + {0, 2, 16, 18}[p] + {0, 1}
      rsb = kSOff + (uint32_t)(4 * lg) * kSRow + (uint32_t)gi * 4u;
    }
  }
  // kStage: write the tile's rows and scales to the wave's LDS and read back the lane's
  // gathered operands (LDS operations of one wave execute in order: no barrier)
  __device__ __forceinline__ void stage(Raw& r, int wave) const {
    if constexpr (kStage) {
      __shared__ __attribute__((aligned(16))) uint8_t vst[kTW][kStageBytes];
      uint8_t* base = vst[wave];
      cst.write(base, r.c0, r.c1);
      if (ls != kOutOfRange) *reinterpret_cast<u32x4*>(base + ws) = r.sc;
      uint32_t w[8];
      cst.gather(base, w);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t dt = p == 0 ? 0u : p == 1 ? 2u : p == 2 ? 16u : 18u;
        r.w[2 * p][0] = w[2 * p];
        r.w[2 * p + 1][0] = w[2 * p + 1];
        const uint32_t* sr = reinterpret_cast<const uint32_t*>(base + rsb + dt * kSRow);
        r.s[2 * p] = sr[0];
        r.s[2 * p + 1] = sr[kSRow / 4];
      }
    } else {
      (void)r;
      (void)wave;
    }
  }
  // rows of a partial last tile past the capacity read 0; !valid: every load out of range
  __device__ __forceinline__ void load(int tok, bool valid, Raw& r) const {
    if constexpr (kStage) {
      cst.load(rv, valid ? (uint32_t)tok * kRow : kOutOfRange, r.c0, r.c1);
      r.sc = bload4(rs, ls + (valid ? (uint32_t)tok * sst : kOutOfRange), 0);
      return;
    }
    const uint32_t v = vv + (valid ? (uint32_t)tok * kRow : kOutOfRange);
    const uint32_t p = vs + (valid ? (uint32_t)tok * sst : kOutOfRange);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t t = (k < 4) ? (uint32_t)k : (uint32_t)(12 + k);  // 16 + k - 4
      if constexpr (I4) {
        r.w[k][0] = bload1(rv, v + t * kRow, 0);
        r.s[k] = bload1(rs, p + t * sst, 0);
      } else {
        const u32x2 x = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(rv, (int)(v + t * kRow), 0, kBufNT));
        r.w[k][0] = x.x;
        r.w[k][1] = x.y;
        r.s[k] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)(p + t * sst), 0, kBufNT);
      }
    }
  }
  // tokens at or past the context in the last, partial tile: scale 0 (their memory may
  // hold anything; p is 0 there)
  __device__ __forceinline__ void mask(Raw& r, int tt, int ctx, int lg) const {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int t = tt + 4 * lg + ((k < 4) ? k : 12 + k);
      if (t >= ctx) r.s[k] = 0u;
    }
  }
  __device__ __forceinline__ uint32_t spair(const Raw& r, int p) const {
    if constexpr (I4)
      return pair_h2((half_t)__builtin_bit_cast(float, r.s[2 * p]),
                     (half_t)__builtin_bit_cast(float, r.s[2 * p + 1]));
    else
      return (r.s[2 * p] & 0xFFFFu) | (r.s[2 * p + 1] << 16);
  }
  __device__ __forceinline__ void mma(const Raw& r, half8v pb, half8v pl, float4v acc[8],
                                      const NibConsts& nc) const {
    uint32_t sp[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) sp[p] = spair(r, p);
    if constexpr (I4) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        // byte k of the tokens T(2p), T(2p + 1) into the low bytes of the two halves
        const uint32_t sel = (uint32_t)k | 0x0C00u | ((uint32_t)(4 + k) << 16) | 0x0C000000u;
        uint32_t h[4], o[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t R = perm_b32(r.w[2 * p + 1][0], r.w[2 * p][0], sel);
          h[p] = deq_pair(and_or(R, nc.m_hi, nc.c64), (half_t)72.0f, sp[p]);
          o[p] = deq_pair(and_or(R, nc.m_lo, nc.c1024), (half_t)1032.0f, sp[p]);
        }
        const half8v ah = pack8(h[0], h[1], h[2], h[3]), ao = pack8(o[0], o[1], o[2], o[3]);
        acc[2 * k] = mfma16x16x32(ah, pb, acc[2 * k]);
        acc[2 * k + 1] = mfma16x16x32(ao, pb, acc[2 * k + 1]);
        acc[2 * k] = mfma16x16x32(ah, pl, acc[2 * k]);
        acc[2 * k + 1] = mfma16x16x32(ao, pl, acc[2 * k + 1]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t sel = (uint32_t)(c & 3) | 0x0C00u | ((uint32_t)(4 + (c & 3)) << 16) | 0x0C000000u;
        uint32_t R[4];
#pragma unroll
        for (int p = 0; p < 4; ++p)
          R[p] = i8pair_deq(perm_b32(r.w[2 * p + 1][c >> 2], r.w[2 * p][c >> 2], sel), as_h2(sp[p]));
        const half8v av = pack8(R[0], R[1], R[2], R[3]);
        acc[c] = mfma16x16x32(av, pb, acc[c]);
        acc[c] = mfma16x16x32(av, pl, acc[c]);
      }
    }
  }
};

// Fused quantize-on-append of the new token of (b, kv head): one wave (the writer), two
// values per lane, the arithmetic of the append kernel: asym_pack_pair with the decode's
// static tables for INT4_ASYM, int8_pack_pair with the append's static table for INT8.  K
// goes to row wpos (INT4_ASYM: its outlier channels verbatim to the side-band), V to its
// TILE32 bytes or its row.  The other waves issue nothing for it (even out-of-range memory
// operations would occupy their address unit ahead of their first cache loads).  NaN / Inf
// set status[0] and clamped elements are added to status[1] (per side).
// Loaded bits only: a conversion at the fetch would make the writer wait there for every
// load issued before (the first cache tiles), ahead of the work-group's set-up barrier.
struct AppendIn {
  uint32_t k2, v2;  // fp16 pair of channels 2 lane, 2 lane + 1
  uint32_t o;       // lanes < 4: fp16 K value of outlier channel lane (INT4_ASYM K)
  uint32_t ks;      // INT8 K: the table entry of the group of channels 2 lane, 2 lane + 1
  uint32_t vs, vz;  // V: INT8 table entry of that group, or INT4_ASYM fp16 scale /
                    // zero-point of group lane / 16
};
struct AppendFlags {
  bool kbad = false, vbad = false;
  int kclip = 0, vclip = 0;
};

// entry of group g of the append's static INT8 table tab (fp32 bits when f32, else fp16)
__device__ __forceinline__ uint32_t app_int8_entry(const void* tab, int f32, int64_t sh,
                                                   int64_t sg, int hkv, int g) {
  const int64_t i = (int64_t)hkv * sh + (int64_t)g * sg;
  return f32 ? reinterpret_cast<const uint32_t*>(tab)[i]
             : (uint32_t)reinterpret_cast<const uint16_t*>(tab)[i];
}
// its fp16 scale
__device__ __forceinline__ float app_int8_scale(uint32_t e, int f32) {
  const float s = f32 ? __builtin_bit_cast(float, e)
                      : (float)__builtin_bit_cast(half_t, (uint16_t)e);
  return (float)int8_static_scale16(s, f32 != 0);
}
__device__ __forceinline__ float h16(uint32_t e) {
  return (float)__builtin_bit_cast(half_t, (uint16_t)e);
}

// oc: the kv head's 4 outlier channels (from the q set-up's inputs); called by the writer
template <class KF, class VF>
__device__ __forceinline__ void append_fetch(const DecodeArgs& a, int b, int hkv, int lane,
                                             int4 oc, AppendIn& in) {
  const FusedAppend& f = a.app;
  const half_t* xk = f.kx + slab_off(f.ksb, f.ksh, b, hkv);
  const half_t* xv = f.vx + slab_off(f.vsb, f.vsh, b, hkv);
  const rsrc_t rk = buffer_rsrc(xk, kD * 2), rv = buffer_rsrc(xv, kD * 2);
  in.k2 = bload1(rk, 4u * lane, 0);
  in.v2 = bload1(rv, 4u * lane, 0);
  in.o = 0;
  if constexpr (KF::kOut) {
    const int4 c4 = clamp_ch4(oc);
    const int ch = lane == 0 ? c4.x : lane == 1 ? c4.y : lane == 2 ? c4.z : c4.w;
    in.o = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(
        rk, (int)(lane < 4 ? 2u * (uint32_t)ch : kOutOfRange), 0, kBufNT);
  }
  const int g = lane >> 4;  // group of 32
  int g8 = g;               // INT8 sides: the group of channels 2 lane, 2 lane + 1
  if constexpr (KF::kGsAny) g8 = (2 * lane) >> __builtin_ctz((unsigned)a.gs);
  in.ks = 0;
  if constexpr (!KF::kAsym) in.ks = app_int8_entry(f.kst, f.kst_f32, f.kst_sh, f.kst_sg, hkv, g8);
  if constexpr (VF::kTile32) {
    // V scale / zero-point of group lane / 16 (fp16, element offsets hkv * ssh + g * ssg)
    in.vs = reinterpret_cast<const uint16_t*>(a.v.scale)[hkv * a.v.ssh + g * a.v.ssg];
    in.vz = reinterpret_cast<const uint16_t*>(a.v.zp)[hkv * a.v.ssh + g * a.v.ssg];
  } else {
    in.vs = app_int8_entry(f.vst, f.vst_f32, f.vst_sh, f.vst_sg, hkv, g8);
    in.vz = 0;
  }
}

// ks / kz: the INT4_ASYM K scale / zero-point of group lane / 16 (the q set-up reads the same)
template <class KF, class VF>
__device__ __forceinline__ void append_store(const DecodeArgs& a, const KF& kf, const VF& vf,
                                             int lane, const AppendIn& in, float ks, float kz,
                                             AppendFlags& fl) {
  const int64_t t = a.app.wpos;
  const half2v k2 = as_h2(in.k2), v2 = as_h2(in.v2);
  int kclip = 0, vclip = 0;
  if constexpr (KF::kAsym) {
    const uint32_t kb = asym_pack_pair((float)k2.x, (float)k2.y, ks, kz, kclip);
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)kb, kf.rk, (int)(uint32_t)(t * kRowK + lane), 0, 0);
  } else {
    const float ks = app_int8_scale(in.ks, a.app.kst_f32);
    const uint16_t kp = int8_pack_pair((float)k2.x, (float)k2.y, (half_t)ks, kclip);
    __builtin_amdgcn_raw_buffer_store_b16(kp, kf.rk, (int)(uint32_t)(t * kD + 2 * lane), 0, 0);
  }
  if constexpr (VF::kTile32) {
    const uint32_t vb = asym_pack_pair((float)v2.x, (float)v2.y, h16(in.vs), h16(in.vz), vclip);
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)vb, vf.rv, (int)(uint32_t)tile32_offset(t, lane), 0, 0);
  } else {
    const float vs = app_int8_scale(in.vs, a.app.vst_f32);
    const uint16_t vp = int8_pack_pair((float)v2.x, (float)v2.y, (half_t)vs, vclip);
    __builtin_amdgcn_raw_buffer_store_b16(vp, vf.rv, (int)(uint32_t)(t * kD + 2 * lane), 0, 0);
  }
  if constexpr (KF::kOut)
    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)in.o, kf.ro,
                                          (int)(lane < 4 ? (uint32_t)(t * kRowO + 2 * lane) : kOutOfRange), 0, 0);
  fl.kbad |= __ballot(!(__builtin_isfinite((float)k2.x) && __builtin_isfinite((float)k2.y))) != 0;
  fl.vbad |= __ballot(!(__builtin_isfinite((float)v2.x) && __builtin_isfinite((float)v2.y))) != 0;
  fl.kclip += wave_sum_int(kclip);
  fl.vclip += wave_sum_int(vclip);
}

// The fused append of the row formats: the writer quantises the (b, kv head) row of each
// side of the one-token append exactly as kvq_quant_append's kernel does (quant_row_x on
// row b * H + h), codes, per-token scales and status words included.  An INT4 side with the
// group rescue first finds its threshold over every row of the append on its own
// (rescue_thr_wave: the host admits only thresholds within the walk's reach of the top).
__device__ __forceinline__ bool rescue_side(const AppendDev& d) {
  return d.fmt == KVQ_FMT_INT4_SYM && d.st != nullptr && d.rq > 0.f && !d.rescue_all;
}
// The writer's inputs, requested at the start of the kernel (under the streaming that
// follows, a load issued at the store would wait a loaded round trip): its own new rows and
// their static scales, and with the group rescue every new row of the append.
struct RowPre {
  half2v k, v;
  uint32_t sk, sv;  // the static scales' bits (row_static_bits)
};
__device__ __forceinline__ void append_row_fetch(const DecodeArgs& a, int b, int hkv, int lane,
                                                 RowPre& p) {
  const int row = b * a.ark.H + hkv;
  p.k = load_x(a.ark, row, lane);
  p.sk = row_static_bits(a.ark, row, lane);
  p.v = load_x(a.arv, row, lane);
  p.sv = row_static_bits(a.arv, row, lane);
}
// (the rescue is compiled only where it can occur: INT4_SYM K and V, RESCUE)
// KFMT / VFMT: the sides' formats (the kernel's operand types; the host admits only appends
// of those formats), so the writer's kernel holds only their quantizer code.  One token:
// row b * H + hkv.
template <bool RESCUE, int KFMT, int VFMT>
__device__ __forceinline__ void append_row_pair(const DecodeArgs& a, int b, int hkv, int lane,
                                                const RowPre& p, const RescueRows& rk,
                                                const RescueRows& rv) {
  const int row = b * a.ark.H + hkv;
  float tk = 0.f, tv = 0.f;
  if constexpr (RESCUE) {
    // the writer's scales of each side (one writer per work-group; one array per side, so the
    // V side's writes cannot pass the K side's reads)
    __shared__ float rdyn_k[kRescueRows * 8], rdyn_v[kRescueRows * 8];
    if (rescue_side(a.ark)) tk = rescue_thr_rows(a.ark, lane, rk, rdyn_k);
    quant_row_bhs<KFMT>(a.ark, b, hkv, 0, row, lane, tk, p.k, static_value(a.ark, p.sk));
    if (rescue_side(a.arv)) tv = rescue_thr_rows(a.arv, lane, rv, rdyn_v);
  } else {
    quant_row_bhs<KFMT>(a.ark, b, hkv, 0, row, lane, tk, p.k, static_value(a.ark, p.sk));
  }
  quant_row_bhs<VFMT>(a.arv, b, hkv, 0, row, lane, tv, p.v, static_value(a.arv, p.sv));
}

__device__ __forceinline__ void append_status(const FusedAppend& f, const AppendFlags& fl) {
  if (f.kstatus) {
    if (fl.kbad) atomicOr(&f.kstatus[0], 1);
    if (fl.kclip) atomicAdd(&f.kstatus[1], fl.kclip);
  }
  if (f.vstatus) {
    if (fl.vbad) atomicOr(&f.vstatus[0], 1);
    if (fl.vclip) atomicAdd(&f.vstatus[1], fl.vclip);
  }
}

// The rows of one work-group: runs of waves in its kv head's wave space.  Row b's run is
// waves [p, p + w) of that space, wave k of the run (k = v - p for wave v) taking tiles
// k, k + w, k + 2 w, ..  (tile = 32 tokens; only the row's last tile, t - 1, may be
// partial), so at step i the run reads one contiguous stretch of w tiles and the device
// streams each slab front to back.  The work-group's waves are v0 .. v0 + kTW - 1: waves
// [0, x) of it are row r[0]'s, [x, nact) row r[1]'s (nrows = 2), waves from nact on have
// no row.  Its partial of row r sits in slot v0 / kTW - p / kTW of the row; the row has
// one partial per work-group whose part of the run holds a tile.
struct ShareRow {
  int b;     // the batch row
  int p, w;  // its run of waves
  int t;     // its tiles
  int ctx;   // its context length (clamped to the capacity)
};
struct WgRows {
  int hkv, v0, nrows, x, nact;
  ShareRow r[2];
  uint64_t empty;  // shared split, work-group 0: the rows with an empty context
};
// what the merge needs of the work-group's rows, kept in LDS over the main loop (held in
// scalar registers there, they pushed the loop's own scalars into spills)
struct SegInfo {
  int b[2];     // the rows
  int lo[2], hi[2];  // their waves [lo, hi)
  int slot[2];  // the work-group's partial slot of each
  int n[2];     // each row's partial count
  int tile[2];  // whether the work-group's part holds a tile
};
__device__ __forceinline__ int ceil_div_pos(int x, int y) {  // x >= 0, y >= 1, x < 2^24
  int q = (int)((float)x / (float)y);
  q += q * y < x;
  q -= q > 0 && (q - 1) * y >= x;
  return q;
}
// exclusive prefix sum over the wave's 64 lanes (DPP within rows of 16, then the rows'
// totals by readlane)
__device__ __forceinline__ int wave_excl_scan(int x) {
  int v = x;
  int t = __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += t;
  t = __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += t;
  t = __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += t;
  t = __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += t;
  // v = inclusive sum within the row of 16 lanes
  const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31),
            r2 = __builtin_amdgcn_readlane(v, 47);
  const int lane = threadIdx.x & 63;
  const int base = lane < 16 ? 0 : lane < 32 ? r0 : lane < 48 ? r0 + r1 : r0 + r1 + r2;
  return v + base - x;
}
// the most waves a row's run takes: its partials (one per work-group its run touches) fit
// the merge's kUnitChunks
constexpr int kShareWaveCap = kTW * (kUnitChunks - 1);
// One-dimensional split per kv head (a.share): grid x = the kv head's work-groups.  Rows of
// equal context length: the uniform split (row b takes work-groups [b u, (b + 1) u), u =
// a.u_chunks, waves as in the non-shared split, so the bits are the same).  A ragged batch:
// the W = kTW C waves of C = a.share_c work-groups are shared out over the rows by length.
// Nonempty row b (t_b tiles) takes a run of w_b = min(kShareWaveCap, max(kTW, ceil(t_b /
// T))) waves, runs in row order, with T found from ceil(total / W) upwards so that the runs
// fit W (T = max t_b always fits: C >= the row count).  Runs of at least kTW waves give
// every work-group at most two rows.  Empty rows take no waves; work-group 0 writes their
// outputs.  Every wave of every work-group computes the same shares (lane b handles row b),
// so the assignment is fixed by the context lengths alone.  lin: the work-group's index over
// the whole grid (x fastest); kv head lin / n and work-group lin % n of it (n work-groups per
// kv head), so the work-groups that do work come first and are the first dispatched.
__device__ WgRows share_waves(const DecodeArgs& a, int lin) {
  const int lane = threadIdx.x & 63;
  const bool row = lane < a.B;
  const int len = row ? (int)row_context(a, lane) : 0;
  const int t = (len + kTile - 1) / kTile;
  WgRows wr{};
  wr.nrows = 0;
  const int t0 = __builtin_amdgcn_readlane(t, 0);
  const bool equal = __ballot(row && t != t0) == 0;
  const int n = equal ? a.u_chunks * a.B : a.share_c;  // work-groups per kv head
  wr.hkv = lin / n;
  const int g = lin - wr.hkv * n;
  wr.v0 = g * kTW;
  if (wr.hkv >= a.Hkv) return wr;  // past every kv head's work-groups
  int w;
  if (equal) {  // equal lengths: the uniform split
    w = row && t0 > 0 ? a.u_chunks * kTW : 0;
    wr.empty = t0 == 0 ? __ballot(row) : 0;
  } else {
    const int W = a.share_c * kTW;
    const int total = (int)wave_sum64((float)t);
    auto runs = [&](int T) {
      const int c = t == 0 ? 0 : min(kShareWaveCap, max(kTW, ceil_div_pos(t, T)));
      return c;
    };
    // (float steps: T is only a start and a stride; the loop's test is exact)
    int T = max(1, (int)ceilf((float)total / (float)W));
    int S = (int)wave_sum64((float)runs(T));
    while (S > W) {  // S(T) falls as T grows; S(max t_b) <= W
      T = max(T + 1, (int)ceilf((float)T * ((float)S / (float)W)));
      S = (int)wave_sum64((float)runs(T));
    }
    w = runs(T);
    wr.empty = __ballot(row && t == 0);
  }
  const int p = wave_excl_scan(w);
  const int S = __builtin_amdgcn_readlane(p + w, 63);
  const int v0 = wr.v0;
  if (v0 >= S) return wr;
  const int v1 = min(v0 + kTW, S) - 1;
  const uint64_t ha = __ballot(row && p <= v0 && v0 < p + w);
  const uint64_t hb = __ballot(row && p <= v1 && v1 < p + w);
  const int ba = __builtin_ctzll(ha), bb = __builtin_ctzll(hb);
  wr.r[0] = ShareRow{ba, __builtin_amdgcn_readlane(p, ba), __builtin_amdgcn_readlane(w, ba),
                     __builtin_amdgcn_readlane(t, ba), __builtin_amdgcn_readlane(len, ba)};
  wr.r[1] = ShareRow{bb, __builtin_amdgcn_readlane(p, bb), __builtin_amdgcn_readlane(w, bb),
                     __builtin_amdgcn_readlane(t, bb), __builtin_amdgcn_readlane(len, bb)};
  wr.nrows = ba == bb ? 1 : 2;
  wr.nact = v1 - v0 + 1;
  wr.x = ba == bb ? wr.nact : wr.r[0].p + wr.r[0].w - v0;
  return wr;
}

// merge_chunks with the batch cut to 8 partials when the unit has at most 8: the loads of a
// larger batch past the unit's partials read nothing (out of range) but are not free (a
// 32-partial batch cost the static-INT8-K kernels 1.3 us per launch at 8 chunks per (b, kv
// head)); the 8-partial round is the same arithmetic in the same chunk order, so the same bits.
// The static INT8 pair with group-32 rows keeps the one 32-partial path: its launches split a
// context into many chunks (32 at config 1), and a second path changed its code and cost it
// 0.13 us.  Call sites take merge_chunks_n only where kMergeSplit8 holds.
template <class KF, class VF>
constexpr bool kMergeSplit8 = KF::kMergeBatch > 8 &&
                              !(std::is_same_v<KF, KI8T<false>> && std::is_same_v<VF, VI8RowT<false>>);
template <class KF, class VF>
__device__ __forceinline__ void merge_chunks_n(const DecodeArgs& a, int b, int hkv, int nvalid,
                                               int wave, int lane) {
  if (nvalid <= 8)
    merge_chunks<VF, 8>(a, b, hkv, nvalid, wave, lane);
  else
    merge_chunks<VF, KF::kMergeBatch>(a, b, hkv, nvalid, wave, lane);
}

// SHARE: the instantiation for the shared split (a.share); the other one carries none of
// its code (it cost the grid split 0.2 us per launch at the headline shape).
// V operand types that pass their tiles through LDS (VTokT<true, true>) have kStage
template <class T, class = void>
struct v_staged : std::false_type {};
template <class T>
struct v_staged<T, std::void_t<decltype(T::kStage)>> : std::bool_constant<T::kStage> {};

template <class KF, class VF, int LOOK, bool PACK8, bool SHARE, int WPE = 2>
__global__ __launch_bounds__(kTW * 64) __attribute__((amdgpu_waves_per_eu(WPE)))
void decode_tiled_kernel(DecodeArgs a) {
  // One field of each kernel-argument line the prologue reads, so that the first batch of
  // scalar loads fetches every such line: a line first touched later costs one more round
  // trip before the first cache load (measured 0.15-0.25 us per launch).  The row formats'
  // prologue reads most of the arguments: one dword of every 64-byte line up to the append's
  // two row sides (it touched about 20 lines one after another, 2 us per launch); so does
  // the shared split, whose prologue reads the split's fields before the cache descriptors
  // (1.1 us per launch at config 4); the others read four lines (touching all costs them
  // 0.2 us).  The row sides (ark, arv) are read by the writer wave alone, where it uses
  // them (touching their lines in every wave cost the shared split 0.27 us per launch); the
  // shared split of the other formats touches the lines before the append's and the
  // append's first (0.15 us per launch against every line up to the row sides).
  if constexpr (KF::kAppendRow) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(&a);
#pragma unroll
    for (int i = 0; i < (int)(__builtin_offsetof(DecodeArgs, ark) / 4); i += 16)
      asm volatile("" ::"s"(w[i]));
  } else if constexpr (SHARE) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(&a);
#pragma unroll
    for (int i = 0; i < (int)(__builtin_offsetof(DecodeArgs, app) / 4); i += 16)
      asm volatile("" ::"s"(w[i]));
    asm volatile("" ::"s"(a.app.kx), "s"(a.app.wpos));
  } else {
    asm volatile("" ::"s"(a.v.scale), "s"(a.ctx), "s"(a.app.kx), "s"(a.app.wpos));
  }
  constexpr bool APP = KF::kAppend || KF::kAppendRow;  // a fused append (the writer's code) is built
  constexpr bool OUT = KF::kOut;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, lg = lane >> 4;
  // This work-group's rows (WgRows): the shared split's, or the grid's (chunk, kv head, b)
  // with the row's run of n_chunks * kTW waves from wave 0 (its length read below).
  WgRows wr;
  if constexpr (SHARE) {
    wr = share_waves(a, (int)(blockIdx.y * gridDim.x + blockIdx.x));
    if (wr.hkv >= a.Hkv) return;  // past every kv head's work-groups
    // the rows with an empty context: work-group 0 of the kv head writes their outputs
    // (zero rows, or the residual window alone)
    if (wr.v0 == 0 && wr.empty != 0) {
      const int eh = __builtin_amdgcn_readfirstlane(wr.hkv);
      for (uint64_t e = wr.empty; e != 0; e &= e - 1) {
        const int rb = __builtin_amdgcn_readfirstlane(__builtin_ctzll(e));
        if (VF::kResidual && a.res_n > 0) {
          if constexpr (kMergeSplit8<KF, VF>) merge_chunks_n<KF, VF>(a, rb, eh, 0, wave, lane);
          else merge_chunks<VF, KF::kMergeBatch>(a, rb, eh, 0, wave, lane);
        } else {
          for (int idx = threadIdx.x; idx < a.n_rep * kD; idx += kTW * 64)
            a.out[(int64_t)rb * a.o_sb + (int64_t)(eh * a.n_rep + (idx >> 7)) * a.o_sh +
                  (idx & (kD - 1))] = (half_t)0.0f;
        }
      }
    }
    if (wr.nrows == 0) return;  // past every row's run (uniform over the work-group)
  } else {
    wr.hkv = blockIdx.y;
    wr.v0 = blockIdx.x * kTW;
    wr.nrows = 1;
    wr.x = wr.nact = kTW;
    wr.empty = 0;
    wr.r[0] = ShareRow{(int)blockIdx.z, 0, a.n_chunks * kTW, 0, 0};
    wr.r[1] = wr.r[0];
  }
  const int hkv = __builtin_amdgcn_readfirstlane(wr.hkv);
  // the wave's row: waves [0, x) row r[0]'s, [x, nact) row r[1]'s; waves from nact on have
  // none and take no tile (first at the capacity)
  const bool rowless = wave >= wr.nact;
  const int ri = wave < wr.x ? 0 : 1;
  const int b = __builtin_amdgcn_readfirstlane(ri == 0 ? wr.r[0].b : wr.r[1].b);
  const int rp = __builtin_amdgcn_readfirstlane(ri == 0 ? wr.r[0].p : wr.r[1].p);
  const int stride = __builtin_amdgcn_readfirstlane(ri == 0 ? wr.r[0].w : wr.r[1].w);
  const int ncap = (a.cap + kTile - 1) / kTile;
  const int first = rowless ? ncap : wr.v0 + wave - rp;  // the wave's first tile

  // Fused quantize-on-append.  The writer is the wave whose schedule (below) holds the new
  // token's tile wt: its stores precede, in program order, its loads of that tile.  They
  // are issued after the set-up, when the new rows (requested with q) have arrived, or
  // before the first cache loads when wt is one of the wave's first LOOK + 1 tiles.  A
  // writer whose work-group has no tile of the context stores before it leaves.
  const bool app_on = APP && a.app.kx != nullptr;
  const int wt = app_on ? (int)(a.app.wpos / kTile) : 0;
  const bool writer = app_on && !rowless && first == wt % stride;
  // Tiles shed by the writer.  A row format's writer quantizes its row pair before its loop
  // (with the group rescue it also finds the threshold over every new row), so its stream
  // starts late and it used to end its loop several us after every other wave of its
  // (b, kv head).  Its first kShed tiles go one each to waves of the other three SIMDs
  // (giving them to its SIMD partner, which shares the writer's issue slots, gained less),
  // which take them before their own.  The schedule stays static (results do not depend on
  // timing), and the writer keeps tile wt: shedding applies only when the writer holds at
  // least kShed + LOOK + 2 tiles, so wt is neither shed nor one of its early loads.
  int t_first = first;        // the wave's first tile
  int sw_at = -1, sw_to = 0;  // a receiver continues at sw_to after tile sw_at
  int extra = 0;              // tiles taken (+) or shed (-): the pacing compares remainders
  if constexpr (KF::kAppendRow && !SHARE) {
    constexpr int kShed = KF::kRescue ? KVQ_SHED_RESCUE : KVQ_SHED_ROW;
    static_assert(kShed >= 0 && kShed <= 6, "one shed tile per wave of the other SIMDs");
    const int wfirst = wt % stride;              // the writer's first tile
    const int ww = wfirst - wr.v0;               // its wave, when in this work-group
    const int nw = (wt - wfirst) / stride + 1;   // its tiles up to wt
    if (kShed > 0 && app_on && ww >= 0 && ww < kTW && nw >= kShed + LOOK + 2) {
      // receiver i (i < kShed <= 6) of the writer's tile i: the waves of the other three SIMDs,
      // in the order (ww + 1) % 4, its partner, (ww + 2) % 4, ..
      const int sd = (wave - ww) & 3;                 // SIMD distance from the writer's
      const int ri = sd == 0 ? -1 : 2 * (sd - 1) + (((wave ^ ww) & 4) ? 1 : 0);
      if (wave == ww) {
        t_first = first + kShed * stride;
        extra = -kShed;
      } else if (ri >= 0 && ri < kShed) {
        t_first = wfirst + ri * stride;
        sw_at = t_first;
        sw_to = first;
        extra = 1;
      }
    }
  }
  auto tnext = [&](int t) {
    if constexpr (KF::kAppendRow && !SHARE) return t == sw_at ? sw_to : t + stride;
    else return t + stride;
  };
  AppendIn ain;
  AppendFlags afl;
  [[maybe_unused]] RowPre rpre;
  [[maybe_unused]] RescueRows rxk, rxv;

  __shared__ QShareLds qsh[2];  // the q operands of the work-group's rows
  __shared__ TiledMergeLds msh;
  // Waves w and w + 4 share a SIMD, which issues the older of two ready waves first;
  // each publishes its step count and, when ahead of its partner, lowers its priority,
  // so the two stay in step (the tile schedule, and so every result bit, is fixed).
  __shared__ int progress[kTW];
  progress[wave] = -extra;
  KF kf;
  // the q-side inputs are requested first: the wait for them then does not include the
  // cache tiles requested next
  // (waves 0..3 build the operands of row r[0], waves 4..7 those of r[1]; the q-side fields
  // every wave reads itself are the kv head's)
  typename KF::QInT qin;
  const int bq = __builtin_amdgcn_readfirstlane(wr.nrows == 2 && wave >= 4 ? wr.r[1].b : wr.r[0].b);
  kf.fetch_q(a, bq, hkv, lane, wave, qin);
  if constexpr (KF::kAppendRow) {
    if (writer) {
      append_row_fetch(a, b, hkv, lane, rpre);
      if constexpr (KF::kRescue)
        if (rescue_side(a.ark) || rescue_side(a.arv)) {
          rescue_fetch(a.ark, lane, rxk);
          rescue_fetch(a.arv, lane, rxv);
        }
    }
  }
  kf.setup_addr(a, b, hkv, lane);
  VF vf;
  vf.setup(a, b, hkv, lane);
  // the fused append's two steps (compiled only for the format that has it)
  auto app_fetch = [&]() {
    if constexpr (KF::kAppend) append_fetch<KF, VF>(a, b, hkv, lane, qin.oc, ain);
  };
  auto app_store = [&]() {
    if constexpr (KF::kAppend) append_store(a, kf, vf, lane, ain, (float)qin.s, (float)qin.z, afl);
    else if constexpr (KF::kAppendRow)
      append_row_pair<KF::kRescue, KF::kRowFmt, VF::kRowFmt>(a, b, hkv, lane, rpre, rxk, rxv);
  };

  // Tile schedule (WgRows): the wave takes tiles first + i * stride of its row.  The
  // schedule is static, so results do not depend on timing.
  // tile[j] = tile of step i + j (j <= LOOK + 1)
  int tile[LOOK + 2];
#pragma unroll
  for (int j = 0; j <= LOOK; ++j) tile[j] = j == 0 ? t_first : tnext(tile[j - 1]);
  constexpr int R = LOOK + 1;                 // ring slots per stream
  constexpr int U = (R % 2 == 0) ? R : 2 * R;  // unroll: ring slot and x buffer are static
  typename KF::Raw kr[R];
  typename VF::Raw vr[R];
  // The K and V tiles of step 0 are requested before the q set-up (bounded by the capacity; tiles past the context are never used), so the memory
  // system is busy from the start of the kernel; the rest of the ring (K of steps 1..LOOK,
  // V of steps 1..LOOK-1) after the set-up.  A larger first burst delays the q loads
  // queued with it, and the set-up waits for those (measured: the whole ring up front
  // costs about 0.4 us per launch at the headline shape; warming loads of the next tiles
  // during the set-up cost 1.4 us).  Every ring load is issued unconditionally (out of
  // range for a tile past the bound): conditional loads would make the compiler's vmcnt
  // waits conservative at the joins, i.e. wait for the tiles just requested.
  asm volatile("" ::: "memory");
  const bool early_write = writer && wt / stride <= LOOK;
  if (early_write) {
    app_fetch();
    app_store();
  }
  kf.load(kTile * tile[0], tile[0] < ncap, kr[0]);
  vf.load(kTile * tile[0], tile[0] < ncap, vr[0]);

  // The context length of the grid's row is read here, after the first tiles are requested
  // (bounded by the capacity; tiles past the context are never used) but ahead of every
  // wait: through the scalar cache, whose wait does not include the cache tiles (a vector
  // load whose vmcnt wait also waited for the first tiles cost about 0.5 us per launch).
  if constexpr (!SHARE) {
    const int c = (int)row_context(a, b);
    wr.r[0].t = wr.r[1].t = (c + kTile - 1) / kTile;
    wr.r[0].ctx = wr.r[1].ctx = c;
  }
  const int ntot = __builtin_amdgcn_readfirstlane(ri == 0 ? wr.r[0].t : wr.r[1].t);
  const int ctx = __builtin_amdgcn_readfirstlane(ri == 0 ? wr.r[0].ctx : wr.r[1].ctx);
  const bool partial = (ctx & (kTile - 1)) != 0;
  // the work-group's part of each of its rows: waves [lo, hi), its slot among the row's
  // partials, whether it holds a tile (its first wave's first tile is in the row), and the
  // row's partial count (one per work-group of its run up to the last wave with a tile)
  int seg_lo[2], seg_hi[2], seg_slot[2], seg_n[2];
  bool seg_tile[2];
#pragma unroll
  for (int sgi = 0; sgi < 2; ++sgi) {
    const ShareRow& r = wr.r[sgi];
    seg_lo[sgi] = sgi == 0 ? 0 : wr.x;
    seg_hi[sgi] = sgi == 0 ? wr.x : wr.nact;
    seg_slot[sgi] = wr.v0 / kTW - r.p / kTW;
    seg_n[sgi] = (r.p + min(r.w, r.t) - 1) / kTW - r.p / kTW + 1;
    seg_tile[sgi] = sgi < wr.nrows && seg_lo[sgi] < seg_hi[sgi] && wr.v0 + seg_lo[sgi] - r.p < r.t;
  }
  __shared__ SegInfo seg;
  if (SHARE && threadIdx.x == 0) {
#pragma unroll
    for (int sgi = 0; sgi < 2; ++sgi) {
      seg.b[sgi] = wr.r[sgi].b;
      seg.lo[sgi] = seg_lo[sgi];
      seg.hi[sgi] = seg_hi[sgi];
      seg.slot[sgi] = seg_slot[sgi];
      seg.n[sgi] = seg_n[sgi];
      seg.tile[sgi] = seg_tile[sgi];
    }
  }  // (read after the main loop; the set-up barrier orders the writes before)
  if (!seg_tile[0] && !seg_tile[1]) {  // no tile for this work-group (uniform)
    if (writer) {
      if (!early_write) {
        app_fetch();
        app_store();
      }
      if (lane == 0) append_status(a.app, afl);
    }
    if (!SHARE && ntot == 0 && wr.v0 == 0 && a.fused) {
      if (VF::kResidual && a.res_n > 0) {  // empty quantized context: the residual window alone
        if constexpr (kMergeSplit8<KF, VF>) merge_chunks_n<KF, VF>(a, b, hkv, 0, wave, lane);
        else merge_chunks<VF, KF::kMergeBatch>(a, b, hkv, 0, wave, lane);
      } else {  // empty context: zero rows
        for (int idx = threadIdx.x; idx < a.n_rep * kD; idx += kTW * 64)
          a.out[(int64_t)b * a.o_sb + (int64_t)(hkv * a.n_rep + (idx >> 7)) * a.o_sh +
                (idx & (kD - 1))] = (half_t)0.0f;
      }
    }
    return;
  }
  // The writer fetches the new rows now and stores their codes in the loop, at the last
  // step that precedes its loads of tile wt (step wt_step - LOOK - 1), or right after the
  // set-up when wt lies past the wave's tiles.
  const bool late_write = writer && !early_write;
  const int wt_step = (wt - first) / stride;
  const int store_step = late_write ? wt_step - LOOK - 1 : -1;
  if (late_write) app_fetch();
  // (one row: waves 4..7 would build the same)
  if (wave < 4 || wr.nrows == 2) kf.setup_q(a, qin, lane, wave & 3, qsh[wave >> 2]);
  NibConsts nc;
  nc.init();
  __syncthreads();
#pragma unroll
  for (int s = 1; s <= LOOK; ++s) {
    kf.load(kTile * tile[s], tile[s] < ntot, kr[s]);
    if (s < LOOK) vf.load(kTile * tile[s], tile[s] < ntot, vr[s]);
  }
  kf.finish_setup(qsh[ri], qin, lane);
  // (wt past the context: the wave may have fewer steps than store_step; the row formats'
  // writer always stores here, outside the loop)
  const bool store_now = late_write && (KF::kAppendRow || wt >= ntot || store_step <= 0);
  if (store_now) {
    // with the group rescue the writer's append is a long serial chain (two threshold walks
    // and two row quantizations, about 14 us); at raised priority its SIMD partner, running
    // its loop meanwhile, cannot take its issue slots (int4_fused 39.2 -> 38.4 us per
    // layer-step at config 3's shape; without the rescue the raise cost 0.3 us)
    constexpr bool kLong = [] {
      if constexpr (KF::kAppendRow) return KF::kRescue;
      else return false;
    }();
    if constexpr (kLong) __builtin_amdgcn_s_setprio(3);
    app_store();
    if constexpr (kLong) __builtin_amdgcn_s_setprio(0);
  }

  float4v acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = float4v{0.f, 0.f, 0.f, 0.f};
  float m = kNegInf, l = 0.f;
  const float sm = KF::kSub24 ? a.sm_log2e * kTwo24 : a.sm_log2e;  // logits of KAsymT: x 2^-24
  int steps = 0;
  if (tile[0] < ntot) {
    float4v x[2][2];
    kf.qk(kr[0], nc, x[0][0], x[0][1]);
    while (tile[0] < ntot) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        // step i (i % U == u): the tiles of this wave form a prefix of its schedule
        if (tile[0] >= ntot) break;
        if constexpr (!KF::kAppendRow)
          if (late_write && !store_now && steps == store_step) app_store();
        tile[LOOK + 1] = tnext(tile[LOOK]);
        // fetch K of step i + LOOK + 1 (into the slot K of step i used) and V of step
        // i + LOOK (into the slot V of step i - 1 used), QK of step i + 1, then softmax
        // and PV of step i
        kf.load(kTile * tile[LOOK + 1], tile[LOOK + 1] < ntot, kr[u % R]);
        vf.load(kTile * tile[LOOK], tile[LOOK] < ntot, vr[(u + LOOK) % R]);
        // (staged V: this step's tile through the wave's LDS, while QK and the softmax run)
        if constexpr (v_staged<VF>::value) vf.stage(vr[u % R], wave);
        if (tile[1] < ntot) kf.qk(kr[(u + 1) % R], nc, x[(u + 1) & 1][0], x[(u + 1) & 1][1]);
        float4v x0 = x[u & 1][0], x1 = x[u & 1][1];
        if (partial && tile[0] == ntot - 1) {
          mask_tile(x0, x1, kTile * tile[0], ctx, lg);
          vf.mask(vr[u % R], kTile * tile[0], ctx, lg);
        }
        if constexpr (PACK8 && KF::kPackPV && VF::kPackedPV) {
          half8v pc;
          softmax_tile8c(x0, x1, sm, m, l, acc, pc, col < 8);
          vf.mma1(vr[u % R], pc, acc, nc);
        } else {
          half8v pb, pl;
          if constexpr (PACK8) softmax_tile8(x0, x1, sm, m, l, acc, pb, pl, vf.extra());
          else softmax_tile(x0, x1, sm, m, l, acc, pb, pl, vf.extra());
          vf.mma(vr[u % R], pb, pl, acc, nc);
        }
        ++steps;
        progress[wave] = steps - extra;
        if (__builtin_amdgcn_readfirstlane(progress[wave ^ 4]) < steps - extra)
          __builtin_amdgcn_s_setprio(0);
        else
          __builtin_amdgcn_s_setprio(2);
#pragma unroll
        for (int j = 0; j <= LOOK; ++j) tile[j] = tile[j + 1];
      }
    }
  }
  __builtin_amdgcn_s_setprio(0);
  if constexpr (PACK8 && KF::kPackPV && VF::kPackedPV) fold_lo(acc);
  if (writer && lane == 0) append_status(a.app, afl);

  // Merge.  The waves' states are merged in LDS and the work-group's partial is stored
  // write-through (combine_kernel merges them when a.fused == 0).  Once every store of the
  // work-group has completed, one thread counts it in (word 0 of the (b, kv head)'s
  // counter slot); the last of the (b, kv head)'s work-groups merges every partial, writes
  // the output and resets the counter.
  __shared__ int is_last[2];
  vf.finalize(acc, lane);
  merge_to_lds<PACK8>(a, msh, wave, lane, m, l, acc);
  if constexpr (!SHARE) {  // one row, all kTW waves (constant descriptors: no LDS reads)
    const int nvalid = min(a.n_chunks, (ntot + kTW - 1) / kTW);  // chunks holding a tile
    uint32_t* slot = a.counters + ((int64_t)b * a.Hkv + hkv) * kCtrSlotWords;
    merge_partial(a, msh, wave, lane, 0, kTW, b, hkv, (int)blockIdx.x);
    if (!a.fused) return;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
      is_last[0] = __hip_atomic_fetch_add(slot, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   (uint32_t)(nvalid - 1);
    __syncthreads();
    if (!is_last[0]) return;
    if constexpr (kMergeSplit8<KF, VF>) merge_chunks_n<KF, VF>(a, b, hkv, nvalid, wave, lane);
    else merge_chunks<VF, KF::kMergeBatch>(a, b, hkv, nvalid, wave, lane);
    if (threadIdx.x == 0) __hip_atomic_store(slot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  auto sgv = [](const int& x) { return __builtin_amdgcn_readfirstlane(x); };
#pragma unroll
  for (int sgi = 0; sgi < 2; ++sgi)
    if (sgv(seg.tile[sgi]))
      merge_partial(a, msh, wave, lane, sgv(seg.lo[sgi]), sgv(seg.hi[sgi]), sgv(seg.b[sgi]), hkv,
                    sgv(seg.slot[sgi]));
  if (!a.fused) return;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // lane r of wave 0 counts the work-group in on row r's counter (both rows in one atomic
  // instruction); the last arriver resets it (every work-group of the row has counted)
  if (threadIdx.x < 2) {
    const int sgi = threadIdx.x;
    bool last = false;
    if (seg.tile[sgi]) {
      uint32_t* slot = a.counters + ((int64_t)seg.b[sgi] * a.Hkv + hkv) * kCtrSlotWords;
      last = __hip_atomic_fetch_add(slot, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (uint32_t)(seg.n[sgi] - 1);
      if (last) __hip_atomic_store(slot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    is_last[sgi] = last;
  }
  __syncthreads();
  const int l0 = sgv(is_last[0]), l1 = sgv(is_last[1]);
  if (!l0 && !l1) return;
  constexpr int kB = KF::kMergeBatch < 16 ? KF::kMergeBatch : 16;
  const int mb0 = sgv(seg.b[l0 ? 0 : 1]), mn0 = sgv(seg.n[l0 ? 0 : 1]), mn1 = sgv(seg.n[1]);
  const int nr = l0 && l1 ? 2 : 1;
  // (at most 8 partials per merged row: rounds of 8, as merge_chunks_n)
  if (kMergeSplit8<KF, VF> && kB > 8 && mn0 <= 8 && (nr == 1 || mn1 <= 8))
    merge_rows<VF, (kB > 8 ? 8 : kB)>(a, hkv, mb0, mn0, sgv(seg.b[1]), mn1, nr, wave, lane);
  else
    merge_rows<VF, kB>(a, hkv, mb0, mn0, sgv(seg.b[1]), mn1, nr, wave, lane);
}

template <class KF, class VF, bool PACK8, bool SHARE, int LOOK = 1>
const void* tiled_ptr() {
  return reinterpret_cast<const void*>(&decode_tiled_kernel<KF, VF, LOOK, PACK8, SHARE>);
}
// the kernels for n_rep <= 8 (pack8) pack the second row block's softmax into the padding
// lanes
template <class KF, class VF, int LOOK = 1>
TiledFn tiled_pick(bool pack8) {
  return TiledFn{pack8 ? tiled_ptr<KF, VF, true, false, LOOK>() : tiled_ptr<KF, VF, false, false, LOOK>(),
                 pack8 ? tiled_ptr<KF, VF, true, true, LOOK>() : tiled_ptr<KF, VF, false, true, LOOK>(),
                 KF::kRowFmt, VF::kRowFmt};
}

}  // namespace
}  // namespace kvq

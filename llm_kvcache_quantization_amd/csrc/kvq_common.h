// Shared device helpers for the gfx950 (CDNA4) quantized-KV decode path.
//
// Wavefront = 64 lanes.  MFMA operand layout used throughout (v_mfma_f32_16x16x32_f16
// and v_mfma_f32_16x16x16_f16):
//   A (16 x K): lane l supplies row (l % 16), k-slots owned by lane group (l / 16)
//   B (K x 16): lane l supplies column (l % 16), k-slots owned by lane group (l / 16)
//   D (16 x 16): lane l holds rows 4*(l/16) + r (r = 0..3) of column (l % 16)
// A and B use the same lane-group -> k-slot assignment, so any consistent
// permutation of the reduction index between A and B is harmless; the kernels
// rely on that to read packed codes without shuffles.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvq {

typedef _Float16 half_t;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ float4v mfma16x16x32(half8v a, half8v b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float4v mfma16x16x16(half4v a, half4v b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half2v as_h2(uint32_t x) { return __builtin_bit_cast(half2v, x); }
__device__ __forceinline__ uint32_t as_u32(half2v x) { return __builtin_bit_cast(uint32_t, x); }

__device__ __forceinline__ half8v pack8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4 v = {a, b, c, d};
  return __builtin_bit_cast(half8v, v);
}
__device__ __forceinline__ half4v pack4(uint32_t a, uint32_t b) {
  u32x2 v = {a, b};
  return __builtin_bit_cast(half4v, v);
}

// byte-select: result byte i = sel byte i, where 0..3 pick lo bytes, 4..7 pick hi bytes,
// 0x0c gives 0x00 (v_perm_b32 semantics).
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Nibble -> fp16 conversion by the exponent trick.  A half with exponent field 0x15
// (0x5400 = 64.0) has a mantissa LSB worth 1/16, so a nibble placed in bits 4..7 of
// each 16-bit half gives 64 + n exactly: (x & 0x00F000F0) | 0x54005400.  With exponent
// 0x19 (0x6400 = 1024.0) the LSB is worth 1, so a nibble in bits 0..3 gives 1024 + n:
// (x & 0x000F000F) | 0x64006400.  Both are one v_and_or_b32 per two values.
//
// The masks and magics live in VGPRs (NibConsts) so the compiler can select the
// three-operand v_and_or_b32: a VOP3 instruction on gfx9 cannot encode literals.
struct NibConsts {
  uint32_t m_hi, m_lo, c64, c1024;
  __device__ __forceinline__ void init() {
    m_hi = 0x00F000F0u;
    m_lo = 0x000F000Fu;
    c64 = 0x54005400u;
    c1024 = 0x64006400u;
    asm volatile("" : "+v"(m_hi), "+v"(m_lo), "+v"(c64), "+v"(c1024));
  }
};
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) { return (x & m) | c; }

// Packed INT4 dword w holds bytes b0..b3; byte k = (code[2k] << 4) | code[2k+1]
// (high nibble = even element).  unpack_dword_64pn returns the 8 elements as fp16
// values 64 + n in the k-slot order [0, 4, 1, 5, 2, 6, 3, 7] (element within dword).
__device__ __forceinline__ void unpack_dword_64pn(uint32_t w, const NibConsts& nc, uint32_t out[4]) {
  out[0] = and_or(w, nc.m_hi, nc.c64);        // e0, e4
  out[1] = and_or(w << 4, nc.m_hi, nc.c64);   // e1, e5
  out[2] = and_or(w >> 8, nc.m_hi, nc.c64);   // e2, e6
  out[3] = and_or(w >> 4, nc.m_hi, nc.c64);   // e3, e7
}
// k-slot -> element-within-dword map for unpack_dword_64pn
__host__ __device__ constexpr int kNibSlotElem(int slot) {
  return (slot & 1) ? ((slot >> 1) + 4) : (slot >> 1);
}

// INT8 bytes -> fp16 pair (1024 + u), u = byte ^ 0x80 (so value - 1152 = signed code).
constexpr uint32_t kMagic1024 = 0x64006400u;

__device__ __forceinline__ float wave_max_xor_groups(float x) {
  // reduce across the 4 lane groups (lanes l, l^16, l^32, l^48)
  x = fmaxf(x, __shfl_xor(x, 16, 64));
  x = fmaxf(x, __shfl_xor(x, 32, 64));
  return x;
}
__device__ __forceinline__ float wave_sum_xor_groups(float x) {
  x += __shfl_xor(x, 16, 64);
  x += __shfl_xor(x, 32, 64);
  return x;
}

__device__ __forceinline__ int wave_sum_int(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

// Wave-wide max / sum without the LDS crossbar: DPP within each row of 16 lanes (xor 1,
// xor 2 in the quad, then rotations by 4 and 8), then the four row results by readlane.
// Every lane gets the same value; the order of operations is fixed.
template <int CTRL>
__device__ __forceinline__ float dppf(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                               0xF, 0xF, false));
}
__device__ __forceinline__ float row_lane(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}
__device__ __forceinline__ float wave_max64(float x) {
  x = fmaxf(x, dppf<0xB1>(x));   // quad_perm [1, 0, 3, 2]
  x = fmaxf(x, dppf<0x4E>(x));   // quad_perm [2, 3, 0, 1]
  x = fmaxf(x, dppf<0x124>(x));  // row_ror:4
  x = fmaxf(x, dppf<0x128>(x));  // row_ror:8
  return fmaxf(fmaxf(row_lane(x, 0), row_lane(x, 16)), fmaxf(row_lane(x, 32), row_lane(x, 48)));
}
__device__ __forceinline__ float wave_sum64(float x) {
  x += dppf<0xB1>(x);
  x += dppf<0x4E>(x);
  x += dppf<0x124>(x);
  x += dppf<0x128>(x);
  return (row_lane(x, 0) + row_lane(x, 16)) + (row_lane(x, 32) + row_lane(x, 48));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max of 8 floats with v_max3_f32 (no NaN canonicalisation; inputs are finite or -inf)
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float max8f(float a, float b, float c, float d, float e, float f,
                                       float g, float h) {
  return max3f(max3f(a, b, c), max3f(d, e, f), max3f(g, h, h));
}

// Byte offset, within the (b, h) slab of a KVQ_LAYOUT_TILE32 cache, of packed byte bi
// (0..63) of token t: tile t / 32 holds for lane L = 16 g + c the 32 bytes of its PV
// operand, dword 2 p + k = bytes (4c + 2k, 4c + 2k + 1) of the two tokens a = 0, 1 of
// pair p, where token r = t % 32 = 16 (p / 2) + 4 g + 2 (p % 2) + a.
__host__ __device__ __forceinline__ int64_t tile32_offset(int64_t t, int bi) {
  const int r = (int)(t & 31);
  const int g = (r & 15) >> 2, p = 2 * (r >> 4) + ((r & 3) >> 1), a = r & 1;
  const int c = bi >> 2, k = (bi >> 1) & 1, j = bi & 1;
  return (t >> 5) * 2048 + ((16 * g + c) * 8 + 2 * p + k) * 4 + 2 * a + j;
}

// Asymmetric INT4 with a static scale s and zero-point z of the pair's group:
// c = clamp(rne((x - z) / s), -8, 7), packed as ((c0 + 8) << 4) | (c1 + 8) (even element
// in the high nibble).  The quotient is an IEEE fp32 division, as torch's.  Adds the
// number of clamped elements to clipped.  (src/kernels/triton_quantize_pack_int4.py:18-62,
// tests/test_fused_quantize_pack.py:8-17, src/quant/int4_basic.py:263-270)
__device__ __forceinline__ uint8_t asym_pack_pair(float x0, float x1, float s, float z,
                                                  int& clipped) {
  const float r0 = rintf(__fdiv_rn(x0 - z, s));
  const float r1 = rintf(__fdiv_rn(x1 - z, s));
  clipped += (r0 < -8.f || r0 > 7.f) + (r1 < -8.f || r1 > 7.f);
  const int c0 = (int)fminf(fmaxf(r0, -8.f), 7.f);
  const int c1 = (int)fminf(fmaxf(r1, -8.f), 7.f);
  return (uint8_t)(((c0 + 8) << 4) | (c1 + 8));
}

// fp16 scale of a static INT8 table entry s: max(s, 1e-5) rounded to fp16
// (src/quant/int8_basic.py:159).  An fp16 table clamps in fp16: no fp16 value lies strictly
// between 1e-5 and fp16(1e-5), so clamping at fp16(1e-5) gives the same result.
__device__ __forceinline__ half_t int8_static_scale16(float s, bool f32) {
  return f32 ? (half_t)fmaxf(s, 1e-5f) : (half_t)fmaxf(s, (float)(half_t)1e-5f);
}

// INT8 symmetric with the fp16 scale s16 of the pair's group:
// c = clamp(rne(fp16(x / s16)), -127, 127), the quotient rounded to fp16 before the integer
// rounding as torch's Half division does (src/quant/int8_basic.py:111-164).  Returns the two
// codes as little-endian bytes and adds the codes at +-127 to clipped
// (src/cache/int8_cache.py:407-419).
__device__ __forceinline__ uint16_t int8_pack_pair(float x0, float x1, half_t s16, int& clipped) {
  const float sf = (float)s16;
  const float q0 = rintf((float)(half_t)__fdiv_rn(x0, sf));
  const float q1 = rintf((float)(half_t)__fdiv_rn(x1, sf));
  const int c0 = (int)fminf(fmaxf(q0, -127.f), 127.f);
  const int c1 = (int)fminf(fmaxf(q1, -127.f), 127.f);
  clipped += (c0 == 127 || c0 == -127) + (c1 == 127 || c1 == -127);
  return (uint16_t)((uint8_t)(int8_t)c0 | ((uint16_t)(uint8_t)(int8_t)c1 << 8));
}

// streaming loads: the code bytes are read once, so do not keep them in the caches
template <class T>
__device__ __forceinline__ T ld_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const T*>(p));
}

}  // namespace kvq

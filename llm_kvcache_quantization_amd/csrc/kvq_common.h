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

// Nibble -> fp16 "64 + n" (exponent 6, mantissa LSB = 1/16 so n<<4 lands on the units):
// (x & 0x00F000F0) | 0x54005400 turns the nibbles sitting in bits 4..7 and 20..23 into
// two halves 64+n.  Exact.
constexpr uint32_t kNibMask = 0x00F000F0u;
constexpr uint32_t kMagic64 = 0x54005400u;
__device__ __forceinline__ uint32_t nib_hi_pair(uint32_t x) { return (x & kNibMask) | kMagic64; }

// Packed INT4 dword w holds bytes b0..b3; byte k = (code[2k] << 4) | code[2k+1]
// (high nibble = even element).  unpack_dword_64pn returns the 8 elements as
// fp16 values 64 + n in the k-slot order [0, 4, 1, 5, 2, 6, 3, 7] (element index
// within the dword).
__device__ __forceinline__ void unpack_dword_64pn(uint32_t w, uint32_t out[4]) {
  out[0] = nib_hi_pair(w);        // e0, e4
  out[1] = nib_hi_pair(w << 4);   // e1, e5
  out[2] = nib_hi_pair(w >> 8);   // e2, e6
  out[3] = nib_hi_pair(w >> 4);   // e3, e7
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

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace kvq

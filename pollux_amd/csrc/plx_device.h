// Device helpers shared by the .hip translation units.
#pragma once

#include <hip/hip_fp16.h>

#include "plx_internal.h"

namespace plx {

// fp32 -> bf16 bits, round to nearest even (finite inputs; the same rounding
// the reference's bf16 casts use).
__device__ __forceinline__ uint32_t bf16_rne_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t b) { return __uint_as_float(b << 16); }

// Raw buffer loads: descriptor word 3 on gfx9 (gfx950), and a byte offset past
// every buffer range the kernels use (such a load reads zeros and touches no
// memory, so a load that may fall outside its data needs no branch).
constexpr int kBufferFlags = 0x00020000;
constexpr int kBufferOutOfRange = 0x7FFFFFF0;

// fp32 value of raw codebook coordinate k in -4..4: k * fp32(1/sqrt 8) rounded to fp32.
__device__ __forceinline__ float raw_value_f32(int k) {
  return static_cast<float>(k) * __uint_as_float(kLeechScaleBits);
}

// fp16 bits of the materialised weight for raw coordinate k and row scale sig
// (pollux.py:492-499): fp16(fp32(fp16(cb16[k] * sig)) * fp32(1/sqrt 2)), both
// products in fp32 then rounded to fp16, cb16 = fp16(k * fp32(1/sqrt 8)).
// An fp32 result kept as computed before it is rounded again: the empty asm stops
// the compiler from folding fp32 product + fp16 conversion into one mixed-precision
// FMA (v_fma_mixlo_f16 with a +0 addend), which turns a -0 product into +0 and
// rounds the exact product to fp16 once where torch rounds it to fp32 first.
__device__ __forceinline__ float f32_kept(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

__device__ __forceinline__ uint32_t dq_value(int k, float sig, float sl) {
  const float c16 = __half2float(__float2half_rn(raw_value_f32(k)));
  const float t = __half2float(__float2half_rn(f32_kept(c16 * sig)));
  return __half_as_ushort(__float2half_rn(f32_kept(t * sl)));
}

// Lane exchange within rows of 16 lanes by DPP (no trip through the LDS
// crossbar): CTRL 0xB1 = quad_perm [1,0,3,2] (lane ^ 1), 0x4E = quad_perm
// [2,3,0,1] (lane ^ 2), 0x141 = half-row mirror (lane i of 8 reads 7 - i),
// 0x140 = row mirror (lane i of 16 reads 15 - i).  All lanes must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

// Sums (MAX: maxima) of N values over groups of G consecutive lanes (G = 8,
// 16, 32 or 64), every lane of a group ending with its group's result, in
// the same order in every group.  Within a row of 16 the steps are DPP moves
// (xor 1, xor 2, then the two mirrors, which pair quads and half-rows that
// already hold equal values), across rows shuffles; each step is taken for
// all N values before the next, so their latencies overlap (a shuffle chain
// per value waits for every step).  All lanes must be active.
template <int G, bool MAX = false, int N>
__device__ __forceinline__ void group_reduce(float (&v)[N]) {
  static_assert(G == 8 || G == 16 || G == 32 || G == 64, "groups of 8, 16, 32 or 64 lanes");
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = op(v[i], dpp_f32<0xB1>(v[i]));
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = op(v[i], dpp_f32<0x4E>(v[i]));
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = op(v[i], dpp_f32<0x141>(v[i]));
  if constexpr (G >= 16) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = op(v[i], dpp_f32<0x140>(v[i]));
  }
  if constexpr (G >= 32) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = op(v[i], __shfl_xor(v[i], 16, 64));
  }
  if constexpr (G >= 64) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = op(v[i], __shfl_xor(v[i], 32, 64));
  }
}

__device__ __forceinline__ float wave_reduce_sum(float v) {
  float a[1] = {v};
  group_reduce<64>(a);
  return a[0];
}

// Index n of a packed stream: 18 bits at bit 18*(n%4) of group n/4, read as
// the 24-bit big-endian window starting at byte 9*(n/4) + 2*(n%4).
__device__ __forceinline__ int32_t packed_index(const uint8_t *__restrict__ packed, int64_t n) {
  const uint8_t *b = packed + (n >> 2) * 9 + 2 * (n & 3);
  const uint32_t v = (static_cast<uint32_t>(b[0]) << 16) | (static_cast<uint32_t>(b[1]) << 8) | b[2];
  return static_cast<int32_t>((v >> (6 - 2 * (n & 3))) & 0x3FFFFu);
}

// Four 18-bit indices -> one 9-byte big-endian group (castor.py:237-245).
__device__ __forceinline__ void group_to_bytes(int32_t i0, int32_t i1, int32_t i2, int32_t i3, uint8_t *b) {
  b[0] = static_cast<uint8_t>(i0 >> 10);
  b[1] = static_cast<uint8_t>(i0 >> 2);
  b[2] = static_cast<uint8_t>(((i0 & 0x03) << 6) | ((i1 >> 12) & 0x3F));
  b[3] = static_cast<uint8_t>(i1 >> 4);
  b[4] = static_cast<uint8_t>(((i1 & 0x0F) << 4) | ((i2 >> 14) & 0x0F));
  b[5] = static_cast<uint8_t>(i2 >> 6);
  b[6] = static_cast<uint8_t>(((i2 & 0x3F) << 2) | ((i3 >> 16) & 0x03));
  b[7] = static_cast<uint8_t>(i3 >> 8);
  b[8] = static_cast<uint8_t>(i3);
}

// One 9-byte group -> four indices (castor.py:254-257).
__device__ __forceinline__ void bytes_to_group(const uint8_t *b, int32_t *v) {
  const int32_t c0 = b[0], c1 = b[1], c2 = b[2], c3 = b[3], c4 = b[4], c5 = b[5], c6 = b[6], c7 = b[7], c8 = b[8];
  v[0] = (c0 << 10) | (c1 << 2) | (c2 >> 6);
  v[1] = ((c2 & 0x3F) << 12) | (c3 << 4) | (c4 >> 4);
  v[2] = ((c4 & 0x0F) << 14) | (c5 << 6) | (c6 >> 2);
  v[3] = ((c6 & 0x03) << 16) | (c7 << 8) | c8;
}

// Byte tables of the bf16 codebook values by 3-bit value id (ids 0..7 = raw
// coordinates {0, 1, 2, 4, -4, -3, -2, -1}, the id order of the kp_dq table):
// x = low bytes of ids 0-3, y = low bytes of ids 4-7, z / w = high bytes.
__device__ __forceinline__ uint4 bf16_value_table() {
  const int kv[8] = {0, 1, 2, 4, -4, -3, -2, -1};
  uint32_t e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = bf16_rne_bits(raw_value_f32(kv[i]));
  uint4 t;
  t.x = (e[0] & 0xFFu) | (e[1] & 0xFFu) << 8 | (e[2] & 0xFFu) << 16 | (e[3] & 0xFFu) << 24;
  t.y = (e[4] & 0xFFu) | (e[5] & 0xFFu) << 8 | (e[6] & 0xFFu) << 16 | (e[7] & 0xFFu) << 24;
  t.z = (e[0] >> 8) | (e[1] >> 8) << 8 | (e[2] >> 8) << 16 | (e[3] >> 8) << 24;
  t.w = (e[4] >> 8) | (e[5] >> 8) << 8 | (e[6] >> 8) << 16 | (e[7] >> 8) << 24;
  return t;
}

// The same byte tables for the raw integers themselves (bf16 of {0, 1, 2, 4,
// -4, -3, -2, -1}, all exact).
__device__ __forceinline__ uint4 int_value_table() {
  const int kv[8] = {0, 1, 2, 4, -4, -3, -2, -1};
  uint32_t e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = bf16_rne_bits(static_cast<float>(kv[i]));
  uint4 t;
  t.x = (e[0] & 0xFFu) | (e[1] & 0xFFu) << 8 | (e[2] & 0xFFu) << 16 | (e[3] & 0xFFu) << 24;
  t.y = (e[4] & 0xFFu) | (e[5] & 0xFFu) << 8 | (e[6] & 0xFFu) << 16 | (e[7] & 0xFFu) << 24;
  t.z = (e[0] >> 8) | (e[1] >> 8) << 8 | (e[2] >> 8) << 16 | (e[3] >> 8) << 24;
  t.w = (e[4] >> 8) | (e[5] >> 8) << 8 | (e[6] >> 8) << 16 | (e[7] >> 8) << 24;
  return t;
}

// One kp_dq word (byte i = id of coordinate i | id of coordinate 4+i << 4)
// -> the 8 16-bit values as pairs (coordinates 0,1 | 2,3 | 4,5 | 6,7), low
// half first, through 6 v_perm_b32 byte lookups in a 4-word table t.
__device__ __forceinline__ uint4 ids_to_pairs(uint32_t w, uint4 t) {
  const uint32_t s_lo = w & 0x0F0F0F0Fu, s_hi = (w >> 4) & 0x0F0F0F0Fu;
  const uint32_t l_lo = __builtin_amdgcn_perm(t.y, t.x, s_lo), h_lo = __builtin_amdgcn_perm(t.w, t.z, s_lo);
  const uint32_t l_hi = __builtin_amdgcn_perm(t.y, t.x, s_hi), h_hi = __builtin_amdgcn_perm(t.w, t.z, s_hi);
  return make_uint4(__builtin_amdgcn_perm(h_lo, l_lo, 0x05010400u), __builtin_amdgcn_perm(h_lo, l_lo, 0x07030602u),
                    __builtin_amdgcn_perm(h_hi, l_hi, 0x05010400u), __builtin_amdgcn_perm(h_hi, l_hi, 0x07030602u));
}

__device__ __forceinline__ bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace plx

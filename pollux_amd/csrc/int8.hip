// Per-row INT8 periphery: the embedding / LM-head format of .plx files.
//
// quantize (pack._quantize_int8, pack.py:124-136), per row r of [rows, cols]:
//   mu    = max(max_j |w_j|, 1e-8)
//   q_j   = int8(clamp(rint((w_j / mu) * 127), -128, 127))     IEEE fp32 ops, RNE
//   mu16  = fp16(mu)
// dequantize (PackedInt8Embedding/Linear.materialize, pollux.py:521-530,
// 551-560), evaluated the way torch evaluates it on fp16 device tensors:
//   s16   = fp16(fp32(mu16) * fp32(1/127))      (tensor / scalar = multiply by
//                                                 the fp32 reciprocal)
//   w_j   = fp16(fp32(q_j) * fp32(s16))
//
// One wave per row; both kernels stream the row with 16-byte accesses when
// the row is 16-byte aligned, else element-wise.

#include <hip/hip_fp16.h>

#include "plx_device.h"

namespace plx {
namespace {

constexpr int kRowsPerBlock = 4;

__device__ __forceinline__ int8_t q_of(float w, float mu) {
  const float v = rintf((w / mu) * 127.0f);
  return static_cast<int8_t>(static_cast<int>(fminf(fmaxf(v, -128.0f), 127.0f)));
}

__global__ __launch_bounds__(256) void int8_quant_kernel(const float *__restrict__ w, int64_t rows, int64_t cols,
                                                         int8_t *__restrict__ q, uint16_t *__restrict__ mu16,
                                                         bool vec4) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (row >= rows) return;
  const float *r = w + row * cols;
  int8_t *qr = q + row * cols;
  float amax = 0.f;
  if (vec4) {
    const float4 *r4 = reinterpret_cast<const float4 *>(r);
    for (int64_t i = lane; i < cols / 4; i += 64) {
      const float4 v = r4[i];
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
  } else {
    for (int64_t i = lane; i < cols; i += 64) amax = fmaxf(amax, fabsf(r[i]));
  }
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  const float mu = fmaxf(amax, __uint_as_float(kEpsBits));
  if (lane == 0) mu16[row] = __half_as_ushort(__float2half_rn(mu));
  if (vec4) {
    const float4 *r4 = reinterpret_cast<const float4 *>(r);
    for (int64_t i = lane; i < cols / 4; i += 64) {
      const float4 v = r4[i];
      const uint32_t b = static_cast<uint8_t>(q_of(v.x, mu)) | static_cast<uint32_t>(static_cast<uint8_t>(q_of(v.y, mu))) << 8 |
                         static_cast<uint32_t>(static_cast<uint8_t>(q_of(v.z, mu))) << 16 |
                         static_cast<uint32_t>(static_cast<uint8_t>(q_of(v.w, mu))) << 24;
      reinterpret_cast<uint32_t *>(qr)[i] = b;
    }
  } else {
    for (int64_t i = lane; i < cols; i += 64) qr[i] = q_of(r[i], mu);
  }
}

__global__ __launch_bounds__(256) void int8_dequant_kernel(const int8_t *__restrict__ q,
                                                           const uint16_t *__restrict__ mu16, int64_t rows,
                                                           int64_t cols, uint16_t *__restrict__ w16, bool vec4) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (row >= rows) return;
  const float inv127 = 1.0f / 127.0f;
  const float s = __half2float(__float2half_rn(__half2float(__ushort_as_half(mu16[row])) * inv127));
  const int8_t *qr = q + row * cols;
  uint16_t *out = w16 + row * cols;
  auto one = [&](int8_t v) { return __half_as_ushort(__float2half_rn(static_cast<float>(v) * s)); };
  if (vec4) {
    for (int64_t i = lane; i < cols / 4; i += 64) {
      const uint32_t b = reinterpret_cast<const uint32_t *>(qr)[i];
      const uint32_t h0 = one(static_cast<int8_t>(b)), h1 = one(static_cast<int8_t>(b >> 8));
      const uint32_t h2 = one(static_cast<int8_t>(b >> 16)), h3 = one(static_cast<int8_t>(b >> 24));
      reinterpret_cast<uint2 *>(out)[i] = make_uint2(h0 | h1 << 16, h2 | h3 << 16);
    }
  } else {
    for (int64_t i = lane; i < cols; i += 64) out[i] = one(qr[i]);
  }
}

}  // namespace

int launch_int8_quant(const float *w, int64_t rows, int64_t cols, int8_t *q, uint16_t *mu16, hipStream_t s) {
  const bool vec4 = cols % 4 == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0 && (reinterpret_cast<uintptr_t>(q) & 3u) == 0;
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  hipLaunchKernelGGL(int8_quant_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, w, rows, cols, q, mu16,
                     vec4);
  return check_launch("int8_quant_kernel");
}

int launch_int8_dequant(const int8_t *q, const uint16_t *mu16, int64_t rows, int64_t cols, uint16_t *w16,
                        hipStream_t s) {
  const bool vec4 = cols % 4 == 0 && (reinterpret_cast<uintptr_t>(q) & 3u) == 0 &&
                    (reinterpret_cast<uintptr_t>(w16) & 7u) == 0;
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  hipLaunchKernelGGL(int8_dequant_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, q, mu16, rows, cols,
                     w16, vec4);
  return check_launch("int8_dequant_kernel");
}

}  // namespace plx

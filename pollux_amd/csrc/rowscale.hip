// Row RMS scale (castor.py:309-313) and the pack-time fp16 scale (pack.py:164).
//
//   sigma   = sqrt(fp32(sum_j fp32(w_j^2)) / cols + 1e-8)       all fp32 ops
//   sigma16 = fp16(max(sigma * fp32(sqrt 12), 1e-8))
//
// One wave per row.  The fp32 squares are summed in fp64 and rounded once, so
// the sum is the correctly rounded fp32 sum whatever the lane order; the
// reference's CPU reduction order differs, which leaves sigma within an ulp or
// two of the reference (tested), and every later step is IEEE-exact fp32
// (correctly rounded division and square root; no fast-math).

#include "plx_device.h"

namespace plx {
namespace {

constexpr int kRowsPerBlock = 4;

__global__ __launch_bounds__(256) void row_rms_kernel(const float *__restrict__ w, int64_t rows, int64_t cols,
                                                      float *__restrict__ sigma, uint16_t *__restrict__ sigma16,
                                                      bool vec4) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (row >= rows) return;
  const float *r = w + row * cols;
  double acc = 0.0;
  if (vec4) {
    const float4 *r4 = reinterpret_cast<const float4 *>(r);
    const int64_t n4 = cols / 4;
    for (int64_t i = lane; i < n4; i += 64) {
      const float4 v = r4[i];
      acc += static_cast<double>(v.x * v.x);
      acc += static_cast<double>(v.y * v.y);
      acc += static_cast<double>(v.z * v.z);
      acc += static_cast<double>(v.w * v.w);
    }
  } else {
    for (int64_t i = lane; i < cols; i += 64) {
      const float v = r[i];
      acc += static_cast<double>(v * v);
    }
  }
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane != 0) return;
  const float eps = __uint_as_float(kEpsBits);
  const float mean = static_cast<float>(acc) / static_cast<float>(cols);
  const float s = sqrtf(mean + eps);
  if (sigma) sigma[row] = s;
  if (sigma16) {
    const float t = fmaxf(s * __uint_as_float(kSqrt12Bits), eps);
    sigma16[row] = __half_as_ushort(__float2half_rn(t));
  }
}

}  // namespace

int launch_row_rms(const float *w, int64_t rows, int64_t cols, float *sigma, uint16_t *sigma16, hipStream_t s) {
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const bool vec4 = (cols % 4 == 0) && ((reinterpret_cast<uintptr_t>(w) & 15u) == 0);
  hipLaunchKernelGGL(row_rms_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, w, rows, cols, sigma,
                     sigma16, vec4);
  return check_launch("row_rms_kernel");
}

}  // namespace plx

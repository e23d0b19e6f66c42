// LUT-gather dequantization to fp16 (replaces PackedH24Linear.materialize,
// pollux.py:485-504).
//
//   W[r, 24a + c] = fp16( fp32(fp16(cb16[idx] * sigma16[r])) * fp32(1/sqrt 2) )
//
// cb16 is the RNE fp16 cast of the fp32 codebook (castor.py:193-199); both
// products are computed in fp32 and rounded to fp16, the way torch evaluates
// ``atoms * sigma_rows.view(-1,1,1) * s_lattice`` on fp16 tensors (fp32
// opmath; the Python float scalar enters as fp32).  The codebook is read as
// raw int8 coordinates, so per row the output takes one of 8 values; each
// thread forms that row's values once (in registers) and writes 24 fp16
// values per atom.
//
// Indices above 196,560 (not produced by the reference packer) decode as the
// origin, so corrupt input can never read outside the table.

#include <hip/hip_fp16.h>

#include "plx_device.h"

namespace plx {
namespace {

constexpr int kThreads = 256;                  // one atom per thread
constexpr int kGroupsPerBlock = kThreads / 4;  // 64 groups = 576 packed bytes

__device__ __forceinline__ uint32_t dq_value(int k, float sig, float sl) {
  const float c16 = __half2float(__float2half_rn(raw_value_f32(k)));
  const float t = __half2float(__float2half_rn(c16 * sig));
  return __half_as_ushort(__float2half_rn(t * sl));
}

__global__ __launch_bounds__(kThreads) void dequant_kernel(const uint8_t *__restrict__ packed,
                                                           const uint16_t *__restrict__ sigma16, int64_t n_atoms,
                                                           int64_t atoms_per_row, const int8_t *__restrict__ cb_raw,
                                                           uint16_t *__restrict__ w16) {
  __shared__ __align__(16) uint8_t lds[kGroupsPerBlock * 9];
  const int64_t a0 = static_cast<int64_t>(blockIdx.x) * kThreads;
  const int64_t g0 = a0 / 4;
  const int64_t n_groups = (n_atoms + 3) / 4;
  const int64_t groups_here = min(static_cast<int64_t>(kGroupsPerBlock), n_groups - g0);
  const uint8_t *src = packed + g0 * 9;
  if (groups_here == kGroupsPerBlock && aligned16(packed)) {
    if (threadIdx.x < kGroupsPerBlock * 9 / 16)
      reinterpret_cast<uint4 *>(lds)[threadIdx.x] = reinterpret_cast<const uint4 *>(src)[threadIdx.x];
  } else {
    const int nb = static_cast<int>(groups_here * 9);
    for (int i = threadIdx.x; i < nb; i += kThreads) lds[i] = src[i];
  }
  __syncthreads();
  const int64_t a = a0 + threadIdx.x;
  if (a >= n_atoms) return;
  int32_t v[4];
  bytes_to_group(lds + (threadIdx.x / 4) * 9, v);
  const int sel = threadIdx.x & 3;
  int32_t code = sel == 0 ? v[0] : sel == 1 ? v[1] : sel == 2 ? v[2] : v[3];
  if (code > kKissing) code = 0;

  // Output value of raw coordinate k: mag(|k|) with the fp16 sign bit set for
  // k < 0 (every step of dq_value is an odd function, so this is exact).
  const float sig = __half2float(__ushort_as_half(sigma16[a / atoms_per_row]));
  const float sl = __uint_as_float(kSLatticeBits);
  const uint32_t m0 = dq_value(0, sig, sl);
  const uint64_t m14 = static_cast<uint64_t>(dq_value(1, sig, sl)) | (static_cast<uint64_t>(dq_value(2, sig, sl)) << 16) |
                       (static_cast<uint64_t>(dq_value(3, sig, sl)) << 32) |
                       (static_cast<uint64_t>(dq_value(4, sig, sl)) << 48);

  const uint2 *row = reinterpret_cast<const uint2 *>(cb_raw + static_cast<size_t>(code) * kDim);
  uint4 *dst = reinterpret_cast<uint4 *>(w16 + a * kDim);
#pragma unroll
  for (int p = 0; p < 3; ++p) {
    const uint2 r = row[p];  // 8 raw coordinates
    uint32_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t word = e < 4 ? r.x : r.y;
      const int k = static_cast<int8_t>((word >> (8 * (e & 3))) & 0xFFu);
      const int m = k < 0 ? -k : k;
      const uint32_t mag = m == 0 ? m0 : static_cast<uint32_t>(m14 >> (16 * (m - 1))) & 0xFFFFu;
      h[e] = k < 0 ? (mag ^ 0x8000u) : mag;
    }
    dst[p] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
  }
}

}  // namespace

int launch_dequant_f16(const uint8_t *packed, const uint16_t *sigma16, int64_t rows, int64_t cols, uint16_t *w16,
                       hipStream_t s) {
  if ((reinterpret_cast<uintptr_t>(w16) & 15u) != 0) return fail(PLX_EINVAL, "dequant: output must be 16-byte aligned");
  const DeviceTables *tab = nullptr;
  int st = get_tables(&tab);
  if (st != PLX_OK) return st;
  const int64_t apr = cols / kDim;
  const int64_t n_atoms = rows * apr;
  const dim3 g(static_cast<unsigned>((n_atoms + kThreads - 1) / kThreads));
  hipLaunchKernelGGL(dequant_kernel, g, dim3(kThreads), 0, s, packed, sigma16, n_atoms, apr, tab->cb_raw, w16);
  return check_launch("dequant_kernel");
}

}  // namespace plx

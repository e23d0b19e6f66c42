// 18-bit index packing (castor.py:226-260) as HBM-streaming kernels.
//
// Format: four indices per 9-byte group, the 72-bit big-endian concatenation
// i0|i1|i2|i3 of their low 18 bits; the stream is zero padded to a multiple of
// four.  Indices pass through int32 first (castor.py:233 ``.to(torch.int32)``).
//
// One thread owns one group.  A 256-thread block owns 256 groups = 2,304
// packed bytes, which it moves between HBM and LDS as 144 16-byte vectors so
// the byte-granular side of each kernel is read / written fully coalesced.

#include "plx_device.h"

namespace plx {
namespace {

constexpr int kThreads = 256;
constexpr int kBlockBytes = kThreads * 9;  // 2304 = 144 * 16
typedef int64_t i64x2_t __attribute__((ext_vector_type(2)));

template <bool I64>
__global__ __launch_bounds__(kThreads) void pack_kernel(const void *__restrict__ idx, int64_t n,
                                                        uint8_t *__restrict__ out, int64_t n_groups,
                                                        bool vec_ok) {
  __shared__ __align__(16) uint8_t lds[kBlockBytes];
  const int64_t g0 = static_cast<int64_t>(blockIdx.x) * kThreads;
  const int64_t g = g0 + threadIdx.x;
  if (g < n_groups) {
    int32_t v[4];
    const int64_t base = g * 4;
    if (base + 4 <= n) {
      if (I64) {
        const longlong2 *p = reinterpret_cast<const longlong2 *>(static_cast<const int64_t *>(idx) + base);
        if (vec_ok) {
          const longlong2 a = p[0], b = p[1];
          v[0] = static_cast<int32_t>(a.x); v[1] = static_cast<int32_t>(a.y);
          v[2] = static_cast<int32_t>(b.x); v[3] = static_cast<int32_t>(b.y);
        } else {
          const int64_t *q = static_cast<const int64_t *>(idx) + base;
          for (int k = 0; k < 4; ++k) v[k] = static_cast<int32_t>(q[k]);
        }
      } else {
        const int32_t *q = static_cast<const int32_t *>(idx) + base;
        if (vec_ok) {
          const int4 a = *reinterpret_cast<const int4 *>(q);
          v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        } else {
          for (int k = 0; k < 4; ++k) v[k] = q[k];
        }
      }
    } else {
      for (int k = 0; k < 4; ++k) {
        const int64_t i = base + k;
        v[k] = 0;
        if (i < n) v[k] = I64 ? static_cast<int32_t>(static_cast<const int64_t *>(idx)[i])
                              : static_cast<const int32_t *>(idx)[i];
      }
    }
    group_to_bytes(v[0], v[1], v[2], v[3], lds + threadIdx.x * 9);
  }
  __syncthreads();
  const int64_t groups_here = min(static_cast<int64_t>(kThreads), n_groups - g0);
  uint8_t *dst = out + g0 * 9;
  if (groups_here == kThreads && vec_ok) {
    if (threadIdx.x < kBlockBytes / 16)
      reinterpret_cast<uint4 *>(dst)[threadIdx.x] = reinterpret_cast<const uint4 *>(lds)[threadIdx.x];
  } else {
    const int nb = static_cast<int>(groups_here * 9);
    for (int i = threadIdx.x; i < nb; i += kThreads) dst[i] = lds[i];
  }
}

__global__ __launch_bounds__(kThreads) void unpack_kernel(const uint8_t *__restrict__ packed, int64_t num_indices,
                                                          int64_t *__restrict__ out, int64_t n_groups,
                                                          bool vec_ok) {
  __shared__ __align__(16) uint8_t lds[kBlockBytes];
  const int64_t g0 = static_cast<int64_t>(blockIdx.x) * kThreads;
  const int64_t groups_here = min(static_cast<int64_t>(kThreads), n_groups - g0);
  const uint8_t *src = packed + g0 * 9;
  if (groups_here == kThreads && vec_ok) {
    if (threadIdx.x < kBlockBytes / 16)
      reinterpret_cast<uint4 *>(lds)[threadIdx.x] = reinterpret_cast<const uint4 *>(src)[threadIdx.x];
  } else {
    const int nb = static_cast<int>(groups_here * 9);
    for (int i = threadIdx.x; i < nb; i += kThreads) lds[i] = src[i];
  }
  __syncthreads();
  // Thread t writes index pairs t and t + 256 of the block (16 B each), so
  // every store instruction covers 1 KiB contiguous; non-temporal, since the
  // int64 stream is not read back by this kernel.
  const int64_t i_blk = g0 * 4;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int pr = h * kThreads + threadIdx.x;
    const int64_t base = i_blk + 2 * pr;
    if (base >= num_indices) break;
    int32_t iv[4];
    bytes_to_group(lds + (pr >> 1) * 9, iv);
    const int64_t lo = (pr & 1) ? iv[2] : iv[0], hi = (pr & 1) ? iv[3] : iv[1];
    if (base + 2 <= num_indices && vec_ok) {
      const i64x2_t v = {lo, hi};
      __builtin_nontemporal_store(v, reinterpret_cast<i64x2_t *>(out + base));
    } else {
      out[base] = lo;
      if (base + 1 < num_indices) out[base + 1] = hi;
    }
  }
}

inline bool host_aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

int launch_pack(const void *idx, int idx_is_i64, int64_t n, uint8_t *out, hipStream_t s) {
  const int64_t n_groups = (n + 3) / 4;
  const int64_t blocks = (n_groups + kThreads - 1) / kThreads;
  const bool vec_ok = host_aligned16(idx) && host_aligned16(out);
  profile_before(s, PLX_PROF_PACK);
  if (idx_is_i64)
    hipLaunchKernelGGL(pack_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s, idx, n, out,
                       n_groups, vec_ok);
  else
    hipLaunchKernelGGL(pack_kernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s, idx, n, out,
                       n_groups, vec_ok);
  profile_after(s, PLX_PROF_PACK);
  return check_launch("pack_kernel");
}

int launch_unpack(const uint8_t *packed, int64_t num_indices, int64_t *out, hipStream_t s) {
  const int64_t n_groups = (num_indices + 3) / 4;
  const int64_t blocks = (n_groups + kThreads - 1) / kThreads;
  const bool vec_ok = host_aligned16(packed) && host_aligned16(out);
  profile_before(s, PLX_PROF_UNPACK);
  hipLaunchKernelGGL(unpack_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s, packed, num_indices,
                     out, n_groups, vec_ok);
  profile_after(s, PLX_PROF_UNPACK);
  return check_launch("unpack_kernel");
}

}  // namespace plx

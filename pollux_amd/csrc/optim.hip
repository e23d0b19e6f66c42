// Fused optimiser update of one H24 parameter (replaces the H24 branch of
// pollux_step, pollux.py:836-878); the requantize that follows it
// (pollux.py:880-884) reuses the quantizer's launch path.
//
// One thread per 24-element atom reads grad, m, v and the latent once and
// writes m, v and the latent once.  Every operation reproduces one torch op of
// the reference and its rounding (fp32 tensors, Python floats entering as
// fp32, as torch evaluates them on the CPU):
//   m   = fma(g, 1-b1, m*b1)                 m.mul_(b1).add_(g, alpha=1-b1)
//   v   = fma((1-b2)*g, g, v*b2)             v.mul_(b2).addcmul_(g, g, value=1-b2)
//   q   = (m/bc1) / (sqrt(v/bc2) + eps)      m_unbiased / denom
//   s   = neg_scale * q                      -(kinetic_scale/inertia) * (...)
//   |s| over the atom: 8 accumulators (lane i: coordinates i, i+8, i+16,
//       fma-accumulated), summed in lane order, sqrt   torch.linalg.vector_norm
//   s  *= min((1 / (|s| + eps)) * cap, 1)    the per-atom speed cap (torch
//                                            evaluates float / tensor as a
//                                            reciprocal times the float)
//   latent = latent*wdf + s                  latent.mul_(wdf); latent.add_(s)
// The scalars (b1, 1-b1, b2, 1-b2, clamped bc1 / bc2, neg_scale, wdf, cap) are
// device-resident fp32 values the caller computes with the reference's own
// 0-dim tensor ops, so the step needs no host synchronisation.  Floating-point
// contraction is off in the update kernel: a multiply and an add the reference
// rounds separately stay separate, and every FMA is an explicit __fmaf_rn.
// Division and sqrtf are the correctly rounded forms (hipcc's default);
// __fsqrt_rn is not used: in this toolchain it maps to the approximate
// hardware square root.
//
// The per-tensor energy |s|_2 over all capped steps (pollux.py:886-888) is a
// two-level reduction in a fixed order: per block, then one block over the
// block partials.

#include "plx_device.h"

namespace plx {
namespace {

constexpr int kOptThreads = 256;

__device__ __forceinline__ void load24(const float *__restrict__ p, float *v) {
  const float4 *q = reinterpret_cast<const float4 *>(p);
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    const float4 t = q[i];
    v[4 * i] = t.x;
    v[4 * i + 1] = t.y;
    v[4 * i + 2] = t.z;
    v[4 * i + 3] = t.w;
  }
}

__device__ __forceinline__ void store24(float *__restrict__ p, const float *v) {
  float4 *q = reinterpret_cast<float4 *>(p);
#pragma unroll
  for (int i = 0; i < 6; ++i) q[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}

__global__ __launch_bounds__(kOptThreads) void adam_h24_kernel(const float *__restrict__ grad, float *__restrict__ m,
                                                               float *__restrict__ v, float *__restrict__ latent,
                                                               int64_t n_atoms, const float *__restrict__ scal,
                                                               float *__restrict__ partial) {
  // no contraction: a multiply feeding an add (latent * wdf + s) stays two
  // roundings, as in the reference; every FMA below is an explicit __fmaf_rn
#pragma clang fp contract(off)
  __shared__ float red[kOptThreads];
  const int64_t a = static_cast<int64_t>(blockIdx.x) * kOptThreads + threadIdx.x;
  float e2 = 0.f;  // this atom's sum of squared capped steps
  if (a < n_atoms) {
    const float b1 = scal[0], omb1 = scal[1], b2 = scal[2], omb2 = scal[3];
    const float bc1 = scal[4], bc2 = scal[5], neg_scale = scal[6], wdf = scal[7], cap = scal[8];
    const float eps = __uint_as_float(kEpsBits);
    float g[kDim], mm[kDim], vv[kDim], s[kDim];
    load24(grad + a * kDim, g);
    load24(m + a * kDim, mm);
    load24(v + a * kDim, vv);
#pragma unroll
    for (int c = 0; c < kDim; ++c) {
      mm[c] = __fmaf_rn(g[c], omb1, mm[c] * b1);
      vv[c] = __fmaf_rn(omb2 * g[c], g[c], vv[c] * b2);
      const float mu = mm[c] / bc1;
      const float den = sqrtf(vv[c] / bc2) + eps;
      s[c] = neg_scale * (mu / den);
    }
    store24(m + a * kDim, mm);
    store24(v + a * kDim, vv);
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = __fmaf_rn(s[i + 16], s[i + 16], __fmaf_rn(s[i + 8], s[i + 8], s[i] * s[i]));
    float n2 = acc[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) n2 = n2 + acc[i];
    // torch evaluates `cap / t` (a Python float over a tensor) as reciprocal(t) * cap
    const float fac = fminf((1.0f / (sqrtf(n2) + eps)) * cap, 1.0f);
    float lat[kDim];
    load24(latent + a * kDim, lat);
#pragma unroll
    for (int c = 0; c < kDim; ++c) {
      const float sc = s[c] * fac;
      lat[c] = lat[c] * wdf + sc;
      e2 = __fmaf_rn(sc, sc, e2);
    }
    store24(latent + a * kDim, lat);
  }
  red[threadIdx.x] = e2;
  __syncthreads();
#pragma unroll
  for (int w = kOptThreads / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

// norm_out[0] = sqrt(sum of the block partials), summed in a fixed order.
__global__ __launch_bounds__(kOptThreads) void energy_kernel(const float *__restrict__ partial, int64_t n,
                                                             float *__restrict__ norm_out) {
  __shared__ float red[kOptThreads];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += kOptThreads) s = __fadd_rn(s, partial[i]);
  red[threadIdx.x] = s;
  __syncthreads();
#pragma unroll
  for (int w = kOptThreads / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] = __fadd_rn(red[threadIdx.x], red[threadIdx.x + w]);
    __syncthreads();
  }
  if (threadIdx.x == 0) norm_out[0] = sqrtf(red[0]);
}

int64_t opt_blocks(int64_t n_atoms) { return (n_atoms + kOptThreads - 1) / kOptThreads; }

}  // namespace

size_t adam_h24_workspace_bytes(int64_t n_atoms) {
  return n_atoms <= 0 ? 0 : ((static_cast<size_t>(opt_blocks(n_atoms)) * sizeof(float) + 255) & ~static_cast<size_t>(255));
}

int launch_adam_h24(const float *grad, float *m, float *v, float *latent, int64_t n_atoms, const float *scalars,
                    float *adam_norm_out, void *workspace, hipStream_t s) {
  if (n_atoms <= 0) return PLX_OK;
  const uintptr_t al = reinterpret_cast<uintptr_t>(grad) | reinterpret_cast<uintptr_t>(m) |
                       reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(latent);
  if ((al & 15u) != 0) return fail(PLX_EINVAL, "pollux_step_h24: grad, m, v and latent must be 16-byte aligned");
  const int64_t blocks = opt_blocks(n_atoms);
  if (blocks > 0x7FFFFFFFll) return fail(PLX_EINVAL, "pollux_step_h24: %lld atoms exceed one launch", static_cast<long long>(n_atoms));
  float *partial = static_cast<float *>(workspace);
  hipLaunchKernelGGL(adam_h24_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kOptThreads), 0, s, grad, m, v, latent,
                     n_atoms, scalars, partial);
  int st = check_launch("adam_h24_kernel");
  if (st != PLX_OK) return st;
  if (adam_norm_out) {
    hipLaunchKernelGGL(energy_kernel, dim3(1), dim3(kOptThreads), 0, s, partial, blocks, adam_norm_out);
    st = check_launch("energy_kernel");
  }
  return st;
}

}  // namespace plx

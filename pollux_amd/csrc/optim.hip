// Fused optimiser update of one H24 parameter (replaces the H24 branch of
// pollux_step, pollux.py:836-878); the requantize that follows it
// (pollux.py:880-884) reuses the quantizer's launch path.
//
// A block of NT threads owns NT atoms (NT * 24 elements = NT * 6 float4) and
// reads grad, m, v and the latent once and writes m, v and the latent once,
// all as float4 streams in which consecutive lanes touch consecutive 16-byte
// pieces (thread t moves pieces t, t+NT, ..., t+5NT), so every wave access is
// 1 KiB contiguous.  The streams are nontemporal (each byte is touched once:
// loads and stores that do not claim cache lines for reuse), which took the
// 4608x1152 update from 33.5 to 26.3 us.  NT = 64 for large launches (4x the
// blocks of NT = 256 balance better: 26.3 against 28.5 us), 256 below ~100K
// atoms (fewer, fuller blocks: 10.7 against 11.6 us at 55,296 atoms).  The
// elementwise part runs on those pieces; the capped step s goes through LDS,
// where thread t computes atom t's norm in the reference's order and its cap
// factor, which the latent update reads back per piece.
// Every operation reproduces one torch op of the reference and
// its rounding (fp32 tensors, Python floats entering as fp32, as torch
// evaluates them on the CPU):
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

constexpr int kOptSmall = 256;        // atoms (= threads) per block below kOptLargeAtoms
constexpr int kOptLarge = 64;         // ... and from there on
constexpr int64_t kOptLargeAtoms = 98304;
constexpr int kEnergyThreads = 256;

typedef float f32x4_nt __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 load_nt(const float4 *p) {
  const f32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_nt *>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store_nt(float4 *p, float a, float b, float c, float d) {
  __builtin_nontemporal_store(f32x4_nt{a, b, c, d}, reinterpret_cast<f32x4_nt *>(p));
}

template <int NT>
__global__ __launch_bounds__(NT) void adam_h24_kernel(const float *__restrict__ grad, float *__restrict__ m,
                                                      float *__restrict__ v, float *__restrict__ latent,
                                                      int64_t n_atoms, const float *__restrict__ scal,
                                                      float *__restrict__ partial) {
  // no contraction: a multiply feeding an add (latent * wdf + s) stays two
  // roundings, as in the reference; every FMA below is an explicit __fmaf_rn
#pragma clang fp contract(off)
  constexpr int kPieces = NT * kDim / 4;        // float4 pieces per block
  constexpr int kPerThread = kPieces / NT;      // 6
  __shared__ __align__(16) float sl[NT * kDim];  // the block's capped-step inputs s, atom-major
  __shared__ float fac_s[NT];                    // per atom: min(cap / (|s| + eps), 1)
  __shared__ float red[NT];
  const int tid = threadIdx.x;
  const int64_t a0 = static_cast<int64_t>(blockIdx.x) * NT;
  const int64_t pieces = min(static_cast<int64_t>(kPieces), (n_atoms - a0) * (kDim / 4));  // whole atoms
  const float4 *g4 = reinterpret_cast<const float4 *>(grad + a0 * kDim);
  float4 *m4 = reinterpret_cast<float4 *>(m + a0 * kDim);
  float4 *v4 = reinterpret_cast<float4 *>(v + a0 * kDim);
  float4 *l4 = reinterpret_cast<float4 *>(latent + a0 * kDim);
  const float b1 = scal[0], omb1 = scal[1], b2 = scal[2], omb2 = scal[3];
  const float bc1 = scal[4], bc2 = scal[5], neg_scale = scal[6], wdf = scal[7], cap = scal[8];
  const float eps = __uint_as_float(kEpsBits);

  float4 lat[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int i = tid + j * NT;
    if (i >= pieces) continue;
    const float4 g = load_nt(g4 + i), mm = load_nt(m4 + i), vv = load_nt(v4 + i);
    lat[j] = load_nt(l4 + i);
    float gv[4] = {g.x, g.y, g.z, g.w}, mv[4] = {mm.x, mm.y, mm.z, mm.w}, vw[4] = {vv.x, vv.y, vv.z, vv.w};
    float sv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      mv[c] = __fmaf_rn(gv[c], omb1, mv[c] * b1);
      vw[c] = __fmaf_rn(omb2 * gv[c], gv[c], vw[c] * b2);
      const float mu = mv[c] / bc1;
      const float den = sqrtf(vw[c] / bc2) + eps;
      sv[c] = neg_scale * (mu / den);
    }
    store_nt(m4 + i, mv[0], mv[1], mv[2], mv[3]);
    store_nt(v4 + i, vw[0], vw[1], vw[2], vw[3]);
    reinterpret_cast<float4 *>(sl)[i] = make_float4(sv[0], sv[1], sv[2], sv[3]);
  }
  __syncthreads();
  // atom tid: torch.linalg.vector_norm over its 24 values (8 FMA accumulators,
  // lane i taking coordinates i, i+8, i+16, then summed in lane order)
  if (a0 + tid < n_atoms) {
    const float *sa = sl + tid * kDim;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = __fmaf_rn(sa[i + 16], sa[i + 16], __fmaf_rn(sa[i + 8], sa[i + 8], sa[i] * sa[i]));
    float n2 = acc[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) n2 = n2 + acc[i];
    // torch evaluates `cap / t` (a Python float over a tensor) as reciprocal(t) * cap
    fac_s[tid] = fminf((1.0f / (sqrtf(n2) + eps)) * cap, 1.0f);
  }
  __syncthreads();
  float e2 = 0.f;  // this thread's sum of squared capped steps
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int i = tid + j * NT;
    if (i >= pieces) continue;
    const float fac = fac_s[i / (kDim / 4)];
    const float4 sv = reinterpret_cast<const float4 *>(sl)[i];
    const float sc[4] = {sv.x * fac, sv.y * fac, sv.z * fac, sv.w * fac};
    store_nt(l4 + i, lat[j].x * wdf + sc[0], lat[j].y * wdf + sc[1], lat[j].z * wdf + sc[2], lat[j].w * wdf + sc[3]);
#pragma unroll
    for (int c = 0; c < 4; ++c) e2 = __fmaf_rn(sc[c], sc[c], e2);
  }
  red[tid] = e2;
  __syncthreads();
#pragma unroll
  for (int w = NT / 2; w > 0; w >>= 1) {
    if (tid < w) red[tid] = red[tid] + red[tid + w];
    __syncthreads();
  }
  if (tid == 0) partial[blockIdx.x] = red[0];
}

// norm_out[0] = sqrt(sum of the block partials), summed in a fixed order.
__global__ __launch_bounds__(kEnergyThreads) void energy_kernel(const float *__restrict__ partial, int64_t n,
                                                             float *__restrict__ norm_out) {
  __shared__ float red[kEnergyThreads];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += kEnergyThreads) s = __fadd_rn(s, partial[i]);
  red[threadIdx.x] = s;
  __syncthreads();
#pragma unroll
  for (int w = kEnergyThreads / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] = __fadd_rn(red[threadIdx.x], red[threadIdx.x + w]);
    __syncthreads();
  }
  if (threadIdx.x == 0) norm_out[0] = sqrtf(red[0]);
}

int opt_threads(int64_t n_atoms) { return n_atoms >= kOptLargeAtoms ? kOptLarge : kOptSmall; }
int64_t opt_blocks(int64_t n_atoms) { return (n_atoms + opt_threads(n_atoms) - 1) / opt_threads(n_atoms); }

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
  profile_before(s, PLX_PROF_ADAM);
  if (opt_threads(n_atoms) == kOptLarge)
    hipLaunchKernelGGL((adam_h24_kernel<kOptLarge>), dim3(static_cast<unsigned>(blocks)), dim3(kOptLarge), 0, s, grad, m,
                       v, latent, n_atoms, scalars, partial);
  else
    hipLaunchKernelGGL((adam_h24_kernel<kOptSmall>), dim3(static_cast<unsigned>(blocks)), dim3(kOptSmall), 0, s, grad, m,
                       v, latent, n_atoms, scalars, partial);
  profile_after(s, PLX_PROF_ADAM);
  int st = check_launch("adam_h24_kernel");
  if (st != PLX_OK) return st;
  if (adam_norm_out) {
    hipLaunchKernelGGL(energy_kernel, dim3(1), dim3(kEnergyThreads), 0, s, partial, blocks, adam_norm_out);
    st = check_launch("energy_kernel");
  }
  return st;
}

}  // namespace plx

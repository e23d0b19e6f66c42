// Row RMS norm and the one-token attention step of the packed Pollux decoder
// (pollux.py:566-626 evaluated for one new position per sequence).
//
// rmsnorm_kernel: y = x * rsqrt(mean(x^2) + eps) * w over rows of d fp32
//   values (RMSNorm.forward, pollux.py:580-582); one wave per row, float4
//   loads (all of a row's issued at once up to 2,048 values), the sum of
//   squares reduced across the wave with shuffles.
//
// decode_attention_kernel: one block per (sequence, head).  For the new token
//   it RMS-normalises q and k over the head's 24 values (q_ln / k_ln,
//   pollux.py:615-620), writes k and v into the caches at the position read
//   from device memory, then computes softmax_j<=pos(q . K_j / sqrt 24) V_j
//   over the cached positions (the causal scaled_dot_product_attention of
//   pollux.py:624 for the last query): scores in LDS, block max and sum, the
//   24 outputs accumulated per thread over its positions and reduced in LDS.
//   Reading the position from device memory lets a captured graph replay the
//   step while the position advances on the device; a position outside the
//   cache writes nothing and yields NaN outputs.

#include "plx_device.h"

namespace plx {
namespace {

constexpr int kNormRowsPerBlock = 4;  // one wave per row
constexpr int kNormRegVec = 8;        // float4 per lane held in registers (rows of <= 2,048 values)
constexpr int kAttnThreads = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// REG: rows of up to kNormRegVec float4 per lane (d <= 2,048) are held in
// registers, so every load of the row is in flight before the reduction (a
// loop of dependent trips through memory costs ~1 us per trip at one row).
template <bool REG>
__global__ __launch_bounds__(64 * kNormRowsPerBlock) void rmsnorm_kernel(const float *__restrict__ x,
                                                                        const float *__restrict__ w,
                                                                        float *__restrict__ y, int64_t rows, int d,
                                                                        float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kNormRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float4 *xr = reinterpret_cast<const float4 *>(x + row * d);
  const float4 *wr = reinterpret_cast<const float4 *>(w);
  float4 *yr = reinterpret_cast<float4 *>(y + row * d);
  const int n4 = d >> 2;
  float ss = 0.f;
  if constexpr (REG) {
    float4 v[kNormRegVec], g[kNormRegVec];
#pragma unroll
    for (int k = 0; k < kNormRegVec; ++k) {
      const int i = lane + 64 * k;
      v[k] = i < n4 ? xr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      g[k] = i < n4 ? wr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int k = 0; k < kNormRegVec; ++k) {
      ss = fmaf(v[k].x, v[k].x, ss);
      ss = fmaf(v[k].y, v[k].y, ss);
      ss = fmaf(v[k].z, v[k].z, ss);
      ss = fmaf(v[k].w, v[k].w, ss);
    }
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
#pragma unroll
    for (int k = 0; k < kNormRegVec; ++k) {
      const int i = lane + 64 * k;
      if (i < n4)
        yr[i] = make_float4(v[k].x * r * g[k].x, v[k].y * r * g[k].y, v[k].z * r * g[k].z, v[k].w * r * g[k].w);
    }
  } else {
    for (int i = lane; i < n4; i += 64) {
      const float4 v = xr[i];
      ss = fmaf(v.x, v.x, ss);
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
    }
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
    for (int i = lane; i < n4; i += 64) {
      const float4 v = xr[i], g = wr[i];
      yr[i] = make_float4(v.x * r * g.x, v.y * r * g.y, v.z * r * g.z, v.w * r * g.w);
    }
  }
}

// q, k, v: [b, H, 24] projections of the new token; caches [b, H, max_len, 24];
// out [b, H, 24].  Dynamic LDS: max_len floats of scores.
__global__ __launch_bounds__(kAttnThreads) void decode_attention_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ q_w, const float *__restrict__ k_w, float eps, float *__restrict__ k_cache,
    float *__restrict__ v_cache, const int64_t *__restrict__ pos_ptr, int64_t max_len, float scale,
    float *__restrict__ out) {
  extern __shared__ float scores[];
  __shared__ float qn[kDim];
  __shared__ float red[kAttnThreads / 64][kDim + 1];
  __shared__ float stat[2];
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.x;  // sequence * H + head
  const int64_t pos = *pos_ptr;
  if (pos < 0 || pos >= max_len) {  // the caller's position is outside the cache: write nothing
    if (tid < kDim) out[bh * kDim + tid] = __builtin_nanf("");
    return;
  }
  const float *qh = q + bh * kDim;
  float *kc = k_cache + bh * max_len * kDim;
  float *vc = v_cache + bh * max_len * kDim;

  // wave 0: per-head RMS norms of q and k (24 values each), write k and v at pos
  if (tid < 64) {
    const int c = tid < kDim ? tid : 0;
    const float qv = tid < kDim ? qh[c] : 0.f, kv = tid < kDim ? k[bh * kDim + c] : 0.f;
    const float qs = wave_sum(qv * qv), ks = wave_sum(kv * kv);
    const float rq = 1.0f / sqrtf(qs / static_cast<float>(kDim) + eps);
    const float rk = 1.0f / sqrtf(ks / static_cast<float>(kDim) + eps);
    if (tid < kDim) {
      qn[c] = qv * rq * q_w[c];
      kc[pos * kDim + c] = kv * rk * k_w[c];
      vc[pos * kDim + c] = v[bh * kDim + c];
    }
  }
  __syncthreads();  // the new row is visible to the block (global and LDS)

  // scores of positions 0..pos
  float qr[kDim];
#pragma unroll
  for (int c = 0; c < kDim; ++c) qr[c] = qn[c];
  float mx = -INFINITY;
  for (int64_t j = tid; j <= pos; j += kAttnThreads) {
    const float4 *kr = reinterpret_cast<const float4 *>(kc + j * kDim);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kDim / 4; ++i) {
      const float4 t = kr[i];
      s = fmaf(qr[4 * i], t.x, s);
      s = fmaf(qr[4 * i + 1], t.y, s);
      s = fmaf(qr[4 * i + 2], t.z, s);
      s = fmaf(qr[4 * i + 3], t.w, s);
    }
    s *= scale;
    scores[j] = s;
    mx = fmaxf(mx, s);
  }
  // block max
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((tid & 63) == 0) red[tid >> 6][0] = mx;
  __syncthreads();
  if (tid == 0) {
    float m = red[0][0];
    for (int w = 1; w < kAttnThreads / 64; ++w) m = fmaxf(m, red[w][0]);
    stat[0] = m;
  }
  __syncthreads();
  const float m = stat[0];
  // exp, weighted V sum per thread
  float acc[kDim];
#pragma unroll
  for (int c = 0; c < kDim; ++c) acc[c] = 0.f;
  float se = 0.f;
  for (int64_t j = tid; j <= pos; j += kAttnThreads) {
    const float p = expf(scores[j] - m);
    se += p;
    const float4 *vr = reinterpret_cast<const float4 *>(vc + j * kDim);
#pragma unroll
    for (int i = 0; i < kDim / 4; ++i) {
      const float4 t = vr[i];
      acc[4 * i] = fmaf(p, t.x, acc[4 * i]);
      acc[4 * i + 1] = fmaf(p, t.y, acc[4 * i + 1]);
      acc[4 * i + 2] = fmaf(p, t.z, acc[4 * i + 2]);
      acc[4 * i + 3] = fmaf(p, t.w, acc[4 * i + 3]);
    }
  }
  __syncthreads();  // red[] is reused
  se = wave_sum(se);
#pragma unroll
  for (int c = 0; c < kDim; ++c) acc[c] = wave_sum(acc[c]);
  if ((tid & 63) == 0) {
#pragma unroll
    for (int c = 0; c < kDim; ++c) red[tid >> 6][c] = acc[c];
    red[tid >> 6][kDim] = se;
  }
  __syncthreads();
  if (tid < kDim) {
    float s = 0.f, e = 0.f;
    for (int w = 0; w < kAttnThreads / 64; ++w) {
      s += red[w][tid];
      e += red[w][kDim];
    }
    out[bh * kDim + tid] = s / e;
  }
}

}  // namespace

int launch_rms_norm(const float *x, const float *w, float *y, int64_t rows, int64_t d, float eps, hipStream_t s) {
  if (rows <= 0) return PLX_OK;
  if (d <= 0 || d % 4 != 0 || d > (1 << 24))
    return fail(PLX_EINVAL, "rms_norm: row length %lld must be a positive multiple of 4", static_cast<long long>(d));
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(y);
  if ((al & 15u) != 0) return fail(PLX_EINVAL, "rms_norm: x, w and y must be 16-byte aligned");
  const int64_t blocks = (rows + kNormRowsPerBlock - 1) / kNormRowsPerBlock;
  if (blocks > 0x7FFFFFFFll) return fail(PLX_EINVAL, "rms_norm: too many rows");
  if (d <= 64 * 4 * kNormRegVec)
    hipLaunchKernelGGL((rmsnorm_kernel<true>), dim3(static_cast<unsigned>(blocks)), dim3(64 * kNormRowsPerBlock), 0, s,
                       x, w, y, rows, static_cast<int>(d), eps);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<false>), dim3(static_cast<unsigned>(blocks)), dim3(64 * kNormRowsPerBlock), 0, s,
                       x, w, y, rows, static_cast<int>(d), eps);
  return check_launch("rmsnorm_kernel");
}

int launch_decode_attention(const float *q, const float *k, const float *v, const float *q_w, const float *k_w,
                            float eps, float *k_cache, float *v_cache, const int64_t *pos, int64_t seqs_heads,
                            int64_t max_len, float *out, hipStream_t s) {
  if (seqs_heads <= 0) return PLX_OK;
  if (max_len <= 0 || max_len > 16384)
    return fail(PLX_EINVAL, "decode_attention: cache length %lld outside 1..16384", static_cast<long long>(max_len));
  if (seqs_heads > 0x7FFFFFFFll) return fail(PLX_EINVAL, "decode_attention: too many heads");
  const uintptr_t al = reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache);
  if ((al & 15u) != 0) return fail(PLX_EINVAL, "decode_attention: caches must be 16-byte aligned");
  hipLaunchKernelGGL(decode_attention_kernel, dim3(static_cast<unsigned>(seqs_heads)), dim3(kAttnThreads),
                     static_cast<size_t>(max_len) * sizeof(float), s, q, k, v, q_w, k_w, eps, k_cache, v_cache, pos,
                     max_len, 1.0f / sqrtf(static_cast<float>(kDim)), out);
  return check_launch("decode_attention_kernel");
}

}  // namespace plx

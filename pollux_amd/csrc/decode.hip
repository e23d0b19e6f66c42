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
//   pollux.py:624 for the last query): an online softmax per group of four
//   lanes over its positions, combined across the block at the end.
//   Reading the position from device memory lets a captured graph replay the
//   step while the position advances on the device; a position outside the
//   cache writes nothing and yields NaN outputs.
//
// prefill_attention_kernel: the same for a chunk of up to 256 new positions
//   p .. p+tc-1 of every sequence (the prompt of a prefill, pollux.py:615-626
//   with is_causal over the cached prefix): one block per (head, sequence)
//   normalises the chunk's q and k rows (a thread per row), writes k and v
//   into the caches and keeps all three in LDS; then 16 lanes per query i
//   (keys j = lane, lane + 16, ... <= p + i; cached ones from the caches, the
//   chunk's from LDS) run an online softmax each and combine by DPP within
//   their row of 16 lanes.  Chunks of a longer prompt are consecutive launches,
//   so each one reads the previous chunks' rows from the caches.

#include "plx_device.h"

namespace plx {
namespace {

constexpr int kNormRowsPerBlock = 4;  // one wave per row
constexpr int kNormRegVec = 8;        // float4 per lane held in registers (rows of <= 2,048 values)
constexpr int kAttnThreads = 256;
constexpr int kArgThreads = 1024;
constexpr int kArgRegs = 16;  // float4 per thread held in registers (rows of <= 65,536 values)

__device__ __forceinline__ float wave_sum(float v) { return wave_reduce_sum(v); }

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
// out [b, H, 24].  Four lanes share a position: lane l of wave w holds dims
// 6(l & 3) .. +6 of the K and V rows of positions 64r + 16w + (l >> 2),
// r = 0, 1, ..., so one wave load covers 16 consecutive rows (1.5 KB) where a
// row per lane touched 64 cache lines per instruction.  Each group of four
// runs an online softmax over its positions (the score: its partial dot
// products summed over the four lanes, the same bits in each); the groups
// combine within the wave by DPP / shuffles over lanes of equal dims, the
// waves through LDS.  The positions' K / V rows are loaded kAttnRounds rounds
// of 64 at a time, from clamped addresses (no branch holds a load); round 0
// before the position is read (rows clamped to the cache), so those loads
// and the position's are in flight together.  The new position's normalised
// k and its v stand in for its (not yet written) cache rows.  3 rounds per
// trip (90 VGPRs; 5 waves per SIMD: 16 sequences x 80 heads are resident at
// once) measured 1% faster than 4 at batch 16 and 0.3% at batch 1.
constexpr int kAttnRounds = 3;
__global__ __launch_bounds__(kAttnThreads, 5) void decode_attention_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v, int64_t heads,
    int64_t in_stride, const float *__restrict__ q_w, const float *__restrict__ k_w, float eps,
    float *__restrict__ k_cache, float *__restrict__ v_cache, const int64_t *__restrict__ pos_ptr, int64_t max_len,
    float scale, float *__restrict__ out) {
  constexpr int kSub = kDim / 4;  // dims per lane
  __shared__ float red[kAttnThreads / 64][kDim + 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int d0 = (lane & 3) * kSub;
  const int grp = wave * 16 + (lane >> 2);  // position within a round of 64
  const int64_t bh = blockIdx.x;            // sequence * H + head
  float *kc = k_cache + bh * max_len * kDim + d0;
  float *vc = v_cache + bh * max_len * kDim + d0;
  float kr[kAttnRounds][kSub], vr[kAttnRounds][kSub];
  auto load_row = [&](int r, int64_t j) {
    const float2 *a = reinterpret_cast<const float2 *>(kc + j * kDim);
    const float2 *b = reinterpret_cast<const float2 *>(vc + j * kDim);
#pragma unroll
    for (int i = 0; i < kSub / 2; ++i) {
      const float2 x = a[i], y = b[i];
      kr[r][2 * i] = x.x; kr[r][2 * i + 1] = x.y;
      vr[r][2 * i] = y.x; vr[r][2 * i + 1] = y.y;
    }
  };
  load_row(0, grp < max_len ? grp : max_len - 1);
  // q, k, v rows of `heads` heads, in_stride floats apart per sequence
  const int64_t in = (bh / heads) * in_stride + (bh % heads) * kDim + d0;
  float qv[kSub], kv[kSub], vn[kSub], qw[kSub], kw[kSub];
#pragma unroll
  for (int i = 0; i < kSub / 2; ++i) {
    const float2 a = reinterpret_cast<const float2 *>(q + in)[i], b = reinterpret_cast<const float2 *>(k + in)[i];
    const float2 c = reinterpret_cast<const float2 *>(v + in)[i];
    const float2 e = reinterpret_cast<const float2 *>(q_w + d0)[i], f = reinterpret_cast<const float2 *>(k_w + d0)[i];
    qv[2 * i] = a.x; qv[2 * i + 1] = a.y; kv[2 * i] = b.x; kv[2 * i + 1] = b.y;
    vn[2 * i] = c.x; vn[2 * i + 1] = c.y; qw[2 * i] = e.x; qw[2 * i + 1] = e.y;
    kw[2 * i] = f.x; kw[2 * i + 1] = f.y;
  }
  const int64_t pos = *pos_ptr;
  if (pos < 0 || pos >= max_len) {  // the caller's position is outside the cache: write nothing
    if (tid < kDim) out[bh * kDim + tid] = __builtin_nanf("");
    return;
  }
#pragma unroll
  for (int r = 1; r < kAttnRounds; ++r) {
    const int64_t j = 64 * r + grp;
    load_row(r, j < pos ? j : pos);
  }

  // per-head RMS norms of q and k: 6 squares per lane, summed over the four lanes
  float sq[2] = {0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    sq[0] = fmaf(qv[i], qv[i], sq[0]);
    sq[1] = fmaf(kv[i], kv[i], sq[1]);
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) sq[u] += dpp_f32<0xB1>(sq[u]);
#pragma unroll
  for (int u = 0; u < 2; ++u) sq[u] += dpp_f32<0x4E>(sq[u]);
  const float rq = 1.0f / sqrtf(sq[0] / static_cast<float>(kDim) + eps);
  const float rk = 1.0f / sqrtf(sq[1] / static_cast<float>(kDim) + eps);
  float qn[kSub], kn[kSub];
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    qn[i] = qv[i] * rq * qw[i];
    kn[i] = kv[i] * rk * kw[i];
  }
  if (tid < 4) {  // the new row into the caches
#pragma unroll
    for (int i = 0; i < kSub / 2; ++i) {
      reinterpret_cast<float2 *>(kc + pos * kDim)[i] = make_float2(kn[2 * i], kn[2 * i + 1]);
      reinterpret_cast<float2 *>(vc + pos * kDim)[i] = make_float2(vn[2 * i], vn[2 * i + 1]);
    }
  }

  float m = -INFINITY, l = 0.f, acc[kSub];
#pragma unroll
  for (int i = 0; i < kSub; ++i) acc[i] = 0.f;
  // online softmax step of this group with key row kk and value row vv (all four lanes take it)
  auto step = [&](const float *kk, const float *vv) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kSub; ++i) s = fmaf(qn[i], kk[i], s);
    s += dpp_f32<0xB1>(s);
    s += dpp_f32<0x4E>(s);
    s *= scale;
    const float mn = fmaxf(m, s);
    const float a = expf(m - mn), p = expf(s - mn);  // m = -inf at the first step: a = 0
    l = fmaf(l, a, p);
#pragma unroll
    for (int i = 0; i < kSub; ++i) acc[i] = fmaf(acc[i], a, p * vv[i]);
    m = mn;
  };
  const int64_t n_rounds = pos / 64 + 1;  // positions 0 .. pos
  for (int64_t r0 = 0; r0 < n_rounds; r0 += kAttnRounds) {
    if (r0 > 0) {
#pragma unroll
      for (int r = 0; r < kAttnRounds; ++r) {
        const int64_t j = 64 * (r0 + r) + grp;
        load_row(r, j < pos ? j : pos);
      }
    }
#pragma unroll
    for (int r = 0; r < kAttnRounds; ++r) {
      if (r0 + r >= n_rounds) break;
      const int64_t j = 64 * (r0 + r) + grp;
      if (j < pos) {
        step(kr[r], vr[r]);
      } else if (j == pos) {
        step(kn, vn);
      }
    }
  }

  // the wave's maximum, every group's state rescaled to it and summed over the
  // groups (lanes of equal dims: DPP row rotations by 4 and 8, then shuffles)
  float bmv[1] = {m};
  group_reduce<64, true>(bmv);
  const float bm = bmv[0];
  const float f = m == -INFINITY ? 0.f : expf(m - bm);
  float part[kSub + 1];
#pragma unroll
  for (int i = 0; i < kSub; ++i) part[i] = acc[i] * f;
  part[kSub] = l * f;
#pragma unroll
  for (int i = 0; i <= kSub; ++i) part[i] += dpp_f32<0x124>(part[i]);
#pragma unroll
  for (int i = 0; i <= kSub; ++i) part[i] += dpp_f32<0x128>(part[i]);
#pragma unroll
  for (int i = 0; i <= kSub; ++i) part[i] += __shfl_xor(part[i], 16, 64);
#pragma unroll
  for (int i = 0; i <= kSub; ++i) part[i] += __shfl_xor(part[i], 32, 64);
  if (lane < 4) {
#pragma unroll
    for (int i = 0; i < kSub; ++i) red[wave][d0 + i] = part[i];
    if (lane == 0) {
      red[wave][kDim] = part[kSub];
      red[wave][kDim + 1] = bm;
    }
  }
  __syncthreads();
  if (tid < kDim) {
    float gm = red[0][kDim + 1];
#pragma unroll
    for (int w = 1; w < kAttnThreads / 64; ++w) gm = fmaxf(gm, red[w][kDim + 1]);
    float sacc = 0.f, sl = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnThreads / 64; ++w) {
      const float mw = red[w][kDim + 1];
      const float g = mw == -INFINITY ? 0.f : expf(mw - gm);
      sacc = fmaf(red[w][tid], g, sacc);
      sl = fmaf(red[w][kDim], g, sl);
    }
    out[bh * kDim + tid] = sacc / sl;
  }
}

constexpr int kPrefillChunk = 256;  // new positions per launch (q, k, v rows of the chunk in LDS: 72 KB)

// q, k, v, out: [b, t, H, 24] (rows of the whole prompt; this launch takes rows
// c0 .. c0+tc-1 of each sequence at cache positions p .. p+tc-1); caches
// [b, H, max_len, 24].
__global__ __launch_bounds__(kAttnThreads) void prefill_attention_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ q_w, const float *__restrict__ k_w, float eps, float *__restrict__ k_cache,
    float *__restrict__ v_cache, int64_t heads, int64_t in_stride, int64_t t_total, int64_t c0, int tc, int64_t p,
    int64_t max_len, float scale, float *__restrict__ out) {
  __shared__ __align__(16) float qs[kPrefillChunk][kDim];
  __shared__ __align__(16) float ks[kPrefillChunk][kDim];
  __shared__ __align__(16) float vs[kPrefillChunk][kDim];
  const int tid = threadIdx.x;
  const int64_t h = blockIdx.x, bb = blockIdx.y;
  const int64_t row_stride = heads * kDim;                           // out: between positions of one sequence
  const int64_t in0 = (bb * t_total + c0) * in_stride + h * kDim;    // q, k, v: row c0 of this (sequence, head)
  const int64_t out0 = (bb * t_total + c0) * row_stride + h * kDim;
  float *kc = k_cache + (bb * heads + h) * max_len * kDim;
  float *vc = v_cache + (bb * heads + h) * max_len * kDim;

  // the chunk's rows: RMS norms of q and k (q_ln / k_ln), k and v into the caches
  for (int r = tid; r < tc; r += kAttnThreads) {
    const float4 *q4 = reinterpret_cast<const float4 *>(q + in0 + r * in_stride);
    const float4 *k4 = reinterpret_cast<const float4 *>(k + in0 + r * in_stride);
    const float4 *v4 = reinterpret_cast<const float4 *>(v + in0 + r * in_stride);
    float qv[kDim], kv[kDim], vv[kDim];
#pragma unroll
    for (int i = 0; i < kDim / 4; ++i) {
      const float4 a = q4[i], b = k4[i], c = v4[i];
      qv[4 * i] = a.x; qv[4 * i + 1] = a.y; qv[4 * i + 2] = a.z; qv[4 * i + 3] = a.w;
      kv[4 * i] = b.x; kv[4 * i + 1] = b.y; kv[4 * i + 2] = b.z; kv[4 * i + 3] = b.w;
      vv[4 * i] = c.x; vv[4 * i + 1] = c.y; vv[4 * i + 2] = c.z; vv[4 * i + 3] = c.w;
    }
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int i = 0; i < kDim; ++i) {
      sq = fmaf(qv[i], qv[i], sq);
      sk = fmaf(kv[i], kv[i], sk);
    }
    const float rq = 1.0f / sqrtf(sq / static_cast<float>(kDim) + eps);
    const float rk = 1.0f / sqrtf(sk / static_cast<float>(kDim) + eps);
    float4 *kd = reinterpret_cast<float4 *>(kc + (p + r) * kDim);
    float4 *vd = reinterpret_cast<float4 *>(vc + (p + r) * kDim);
#pragma unroll
    for (int i = 0; i < kDim / 4; ++i) {
      const float4 qn = make_float4(qv[4 * i] * rq * q_w[4 * i], qv[4 * i + 1] * rq * q_w[4 * i + 1],
                                    qv[4 * i + 2] * rq * q_w[4 * i + 2], qv[4 * i + 3] * rq * q_w[4 * i + 3]);
      const float4 kn = make_float4(kv[4 * i] * rk * k_w[4 * i], kv[4 * i + 1] * rk * k_w[4 * i + 1],
                                    kv[4 * i + 2] * rk * k_w[4 * i + 2], kv[4 * i + 3] * rk * k_w[4 * i + 3]);
      const float4 vn = make_float4(vv[4 * i], vv[4 * i + 1], vv[4 * i + 2], vv[4 * i + 3]);
      reinterpret_cast<float4 *>(qs[r])[i] = qn;
      reinterpret_cast<float4 *>(ks[r])[i] = kn;
      reinterpret_cast<float4 *>(vs[r])[i] = vn;
      kd[i] = kn;
      vd[i] = vn;
    }
  }
  __syncthreads();

  // 16 lanes (one DPP row) per query; a row whose query is past the chunk
  // skips the round as a whole, so every DPP exchange sees its full row
  const int grp = tid >> 4, l16 = tid & 15;
  for (int i = grp; i < tc; i += kAttnThreads / 16) {
    const int64_t last = p + i;  // the query's own position: keys 0 .. last
    float qr[kDim];
#pragma unroll
    for (int c = 0; c < kDim; ++c) qr[c] = qs[i][c];
    float m = -INFINITY, l = 0.f, acc[kDim];
#pragma unroll
    for (int c = 0; c < kDim; ++c) acc[c] = 0.f;
    auto step = [&](const float4 *k4, const float4 *v4) {
      float kr[kDim], vr[kDim];
#pragma unroll
      for (int c = 0; c < kDim / 4; ++c) {
        const float4 a = k4[c], b = v4[c];
        kr[4 * c] = a.x; kr[4 * c + 1] = a.y; kr[4 * c + 2] = a.z; kr[4 * c + 3] = a.w;
        vr[4 * c] = b.x; vr[4 * c + 1] = b.y; vr[4 * c + 2] = b.z; vr[4 * c + 3] = b.w;
      }
      float sc = 0.f;
#pragma unroll
      for (int c = 0; c < kDim; ++c) sc = fmaf(qr[c], kr[c], sc);
      sc *= scale;
      const float mn = fmaxf(m, sc);
      const float a = expf(m - mn), pr = expf(sc - mn);  // m = -inf at a lane's first key: a = 0
      l = fmaf(l, a, pr);
#pragma unroll
      for (int c = 0; c < kDim; ++c) acc[c] = fmaf(acc[c], a, pr * vr[c]);
      m = mn;
    };
    // keys j = l16 + 16n in increasing order: the cached ones, then the chunk's
    int64_t j = l16;
    for (; j < p; j += 16)
      step(reinterpret_cast<const float4 *>(kc + j * kDim), reinterpret_cast<const float4 *>(vc + j * kDim));
    for (; j <= last; j += 16)
      step(reinterpret_cast<const float4 *>(ks[j - p]), reinterpret_cast<const float4 *>(vs[j - p]));
    // the row's maximum, every lane's state rescaled to it, then the sums
    float bmv[1] = {m};
    group_reduce<16, true>(bmv);
    const float f = m == -INFINITY ? 0.f : expf(m - bmv[0]);
    float part[kDim + 1];
#pragma unroll
    for (int c = 0; c < kDim; ++c) part[c] = acc[c] * f;
    part[kDim] = l * f;
    group_reduce<16>(part);
    float *o = out + out0 + static_cast<int64_t>(i) * row_stride;
    const float inv = part[kDim];
    // lane c writes coordinate c, lanes 0..7 also c + 16 (static indices: no scratch)
    float v0 = part[0], v1 = part[16];
#pragma unroll
    for (int c = 1; c < 16; ++c) v0 = l16 == c ? part[c] : v0;
#pragma unroll
    for (int c = 17; c < kDim; ++c) v1 = l16 == c - 16 ? part[c] : v1;
    o[l16] = v0 / inv;
    if (l16 < kDim - 16) o[16 + l16] = v1 / inv;
  }
}

// torch.argmax's order: a NaN beats every number; among equal values (or
// NaNs) the lowest index wins.
__device__ __forceinline__ bool arg_better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

// One block per row of cols values; each thread scans its strided share
// (increasing indices), then the block reduces (value, index) pairs.
template <bool VEC>
__global__ __launch_bounds__(kArgThreads) void argmax_rows_kernel(const float *__restrict__ x, int cols,
                                                                  int64_t *__restrict__ out) {
  __shared__ float sv[kArgThreads / 64];
  __shared__ int si[kArgThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float *r = x + static_cast<int64_t>(blockIdx.x) * cols;
  float bv = -INFINITY;
  int bi = cols;  // beyond every index: the first -inf wins when all are -inf
  if constexpr (VEC) {
    const float4 *r4 = reinterpret_cast<const float4 *>(r);
    const int n4 = cols / 4;
    auto take = [&](const float4 &v, int i) {
      if (arg_better(v.x, 4 * i, bv, bi)) { bv = v.x; bi = 4 * i; }
      if (arg_better(v.y, 4 * i + 1, bv, bi)) { bv = v.y; bi = 4 * i + 1; }
      if (arg_better(v.z, 4 * i + 2, bv, bi)) { bv = v.z; bi = 4 * i + 2; }
      if (arg_better(v.w, 4 * i + 3, bv, bi)) { bv = v.w; bi = 4 * i + 3; }
    };
    if (n4 <= kArgThreads * kArgRegs) {
      // the whole row in flight at once (clamped indices: no branch holds a load)
      float4 v[kArgRegs];
#pragma unroll
      for (int k = 0; k < kArgRegs; ++k) {
        const int i = tid + kArgThreads * k;
        v[k] = r4[i < n4 ? i : 0];
      }
#pragma unroll
      for (int k = 0; k < kArgRegs; ++k)
        if (tid + kArgThreads * k < n4) take(v[k], tid + kArgThreads * k);
    } else {
#pragma unroll 4
      for (int i = tid; i < n4; i += kArgThreads) take(r4[i], i);
    }
  } else {
#pragma unroll 4
    for (int i = tid; i < cols; i += kArgThreads) {
      const float v = r[i];
      if (arg_better(v, i, bv, bi)) { bv = v; bi = i; }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (arg_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgThreads / 64; ++w)
      if (arg_better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
    out[blockIdx.x] = bi < cols ? bi : 0;
  }
}

}  // namespace

int launch_argmax_rows(const float *x, int64_t rows, int64_t cols, int64_t *out, hipStream_t s) {
  if (rows <= 0) return PLX_OK;
  if (cols <= 0 || cols > 0x7FFFFFFFll || rows > 0x7FFFFFFFll)
    return fail(PLX_EINVAL, "argmax_rows: shape (%lld, %lld)", static_cast<long long>(rows), static_cast<long long>(cols));
  const bool vec = cols % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
  if (vec)
    hipLaunchKernelGGL((argmax_rows_kernel<true>), dim3(static_cast<unsigned>(rows)), dim3(kArgThreads), 0, s, x,
                       static_cast<int>(cols), out);
  else
    hipLaunchKernelGGL((argmax_rows_kernel<false>), dim3(static_cast<unsigned>(rows)), dim3(kArgThreads), 0, s, x,
                       static_cast<int>(cols), out);
  return check_launch("argmax_rows_kernel");
}

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

int launch_decode_attention(const float *q, const float *k, const float *v, int64_t qkv_stride, int64_t heads,
                            const float *q_w, const float *k_w, float eps, float *k_cache, float *v_cache,
                            const int64_t *pos, int64_t seqs_heads, int64_t max_len, float *out, hipStream_t s) {
  if (seqs_heads <= 0) return PLX_OK;
  if (max_len <= 0 || max_len > (1 << 24))
    return fail(PLX_EINVAL, "decode_attention: cache length %lld outside 1..2^24", static_cast<long long>(max_len));
  if (seqs_heads > 0x7FFFFFFFll) return fail(PLX_EINVAL, "decode_attention: too many heads");
  const uintptr_t al = reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache);
  if ((al & 15u) != 0) return fail(PLX_EINVAL, "decode_attention: caches must be 16-byte aligned");
  if (qkv_stride == 0) {  // contiguous [seqs_heads, 24]
    heads = 1;
    qkv_stride = kDim;
  }
  if (heads <= 0 || seqs_heads % heads != 0 || qkv_stride < heads * kDim)
    return fail(PLX_EINVAL, "decode_attention: rows of %lld heads %lld floats apart do not tile %lld head rows",
                static_cast<long long>(heads), static_cast<long long>(qkv_stride), static_cast<long long>(seqs_heads));
  // the kernel reads q, k, v and the norm weights as float2
  const uintptr_t al8 = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                        reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(q_w) |
                        reinterpret_cast<uintptr_t>(k_w);
  if ((al8 & 7u) != 0 || (qkv_stride & 1) != 0)
    return fail(PLX_EINVAL, "decode_attention: q, k, v and the norm weights must be 8-byte aligned, the row stride even");
  hipLaunchKernelGGL(decode_attention_kernel, dim3(static_cast<unsigned>(seqs_heads)), dim3(kAttnThreads), 0, s, q, k,
                     v, heads, qkv_stride, q_w, k_w, eps, k_cache, v_cache, pos, max_len,
                     1.0f / sqrtf(static_cast<float>(kDim)), out);
  return check_launch("decode_attention_kernel");
}

int launch_prefill_attention(const float *q, const float *k, const float *v, int64_t qkv_stride, const float *q_w,
                             const float *k_w, float eps, float *k_cache, float *v_cache, int64_t b, int64_t heads,
                             int64_t t, int64_t p0, int64_t max_len, float *out, hipStream_t s) {
  if (b <= 0 || heads <= 0 || t <= 0) return PLX_OK;
  if (max_len <= 0 || max_len > (1 << 24))
    return fail(PLX_EINVAL, "prefill_attention: cache length %lld outside 1..2^24", static_cast<long long>(max_len));
  if (p0 < 0 || p0 + t > max_len)
    return fail(PLX_EINVAL, "prefill_attention: positions %lld..%lld outside the cache of %lld", static_cast<long long>(p0),
                static_cast<long long>(p0 + t - 1), static_cast<long long>(max_len));
  if (heads > 0xFFFFll || b > 0xFFFFll) return fail(PLX_EINVAL, "prefill_attention: too many heads or sequences");
  const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                       reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache) |
                       reinterpret_cast<uintptr_t>(out);
  if ((al & 15u) != 0) return fail(PLX_EINVAL, "prefill_attention: q, k, v, caches and out must be 16-byte aligned");
  if (qkv_stride == 0) qkv_stride = heads * kDim;  // contiguous rows
  if (qkv_stride < heads * kDim || qkv_stride % 4 != 0)
    return fail(PLX_EINVAL, "prefill_attention: q, k, v rows %lld floats apart (at least %lld, a multiple of 4)",
                static_cast<long long>(qkv_stride), static_cast<long long>(heads * kDim));
  const float scale = 1.0f / sqrtf(static_cast<float>(kDim));
  for (int64_t c0 = 0; c0 < t; c0 += kPrefillChunk) {
    const int tc = static_cast<int>(t - c0 < kPrefillChunk ? t - c0 : kPrefillChunk);
    hipLaunchKernelGGL(prefill_attention_kernel, dim3(static_cast<unsigned>(heads), static_cast<unsigned>(b)),
                       dim3(kAttnThreads), 0, s, q, k, v, q_w, k_w, eps, k_cache, v_cache, heads, qkv_stride, t, c0, tc,
                       p0 + c0, max_len, scale, out);
    const int st = check_launch("prefill_attention_kernel");
    if (st != PLX_OK) return st;
  }
  return PLX_OK;
}

}  // namespace plx

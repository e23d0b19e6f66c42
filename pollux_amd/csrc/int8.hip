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
//
// int8_linear_kernel: y[m, r] = sum_j n(x)[m, j] * w_j of row r, fp32
//   accumulation of exact products with the fp16 weights above, never stored
//   (PackedInt8Linear.forward, pollux.py:562-563: F.linear(x, W.to(x.dtype)),
//   W fp16 and x fp32); n = identity or the final RMSNorm ln_f
//   (pollux.py:699-700) applied to x in registers.  One wave per run of rows;
//   lane l holds x of the 16-column chunks l, l + 64, ... for MB tokens in
//   registers and streams the same chunks of 4 rows at a time (16-byte loads).
//   Weights: the 4 bytes of a dword, offset by 128 (xor 0x80), become the low
//   bytes of fp16 values 1024 + u (v_perm_b32 with 0x64 high bytes), minus
//   1152 gives q exactly, and one fp16 multiply by s16 rounds q * s16 once -
//   the same value as fp16(fp32(q) * fp32(s16)), whose fp32 product is exact.
//
// int8mm_kernel: the same product for two or more tokens on MFMA.  A block
//   owns 64 rows x 16*MT tokens and its 4 waves split K (each wave a
//   contiguous run of 32-column steps).  Per step a lane decodes 8 weights of
//   one row per row tile (the fp16 values above, split exactly into bf16
//   hi + lo: lo = W - bf16(W) has at most 3 significant bits) and splits 8
//   activations of one token per token tile exactly into three bf16 parts
//   (x = h + m + l), so six v_mfma_f32_16x16x32_bf16 per tile pair (h, m, l
//   times hi and times lo) form the exact products of fp32 x with the fp16
//   weights in fp32 accumulation.  The
//   waves' tiles are summed through LDS in wave order.  With ln_f the
//   activations enter as x * w (the norm weight) and each token's sum is
//   scaled by rsqrt(mean(x^2) + eps) at the end, the sums of squares taken
//   from the same loads.  With keys, each block's best argmax key per token.
//
// int8_embed_kernel: out[b, i, :] = fp32(w[idx[b, i], :]) + pos_w[p0 + i, :]
//   (PackedInt8Embedding.forward + the position embedding, pollux.py:532-533,
//   691-693), p0 read from device memory (a captured graph replays it while
//   the position advances); an id or position out of range yields a NaN row.

#include <algorithm>
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
  const float s = __half2float(__float2half_rn(f32_kept(__half2float(__ushort_as_half(mu16[row])) * inv127)));
  const int8_t *qr = q + row * cols;
  uint16_t *out = w16 + row * cols;
  auto one = [&](int8_t v) { return __half_as_ushort(__float2half_rn(f32_kept(static_cast<float>(v) * s))); };
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

constexpr int kLinWaves = 4;   // waves per block of int8_linear_kernel
constexpr int kEmbedRegs = 8;  // 4-byte pieces per lane held in registers by int8_embed_kernel (rows <= 2,048)

__device__ __forceinline__ float wave_sum64(float v) { return wave_reduce_sum(v); }

// s16 of a row as fp32 (fp16(fp32(mu16) * fp32(1/127)))
__device__ __forceinline__ float int8_row_scale(uint16_t mu) {
  return __half2float(__float2half_rn(f32_kept(__half2float(__ushort_as_half(mu)) * (1.0f / 127.0f))));
}

// the fp16 weights of bytes 0,1 (lo) and 2,3 (hi) of d, each pair times s2
__device__ __forceinline__ void int8x4_weights(uint32_t d, __half2 s2, __half2 &lo, __half2 &hi) {
  const uint32_t u = d ^ 0x80808080u;
  const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // 1024 + u0, 1024 + u1
  const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // 1024 + u2, 1024 + u3
  const __half2 off = __halves2half2(__ushort_as_half(0x6480), __ushort_as_half(0x6480));  // 1152
  lo = __hmul2(__hsub2(*reinterpret_cast<const __half2 *>(&a), off), s2);
  hi = __hmul2(__hsub2(*reinterpret_cast<const __half2 *>(&b), off), s2);
}

// The argmax key of value v at index i: unsigned order of the keys is
// torch.argmax's order (a NaN above every number, +0 and -0 equal, the lower
// index winning among equal values): the value's bits made monotone in the
// high word (NaNs as one positive quiet NaN, -0 as +0), ~i in the low word.
// No key is 0.
__device__ __forceinline__ uint64_t arg_key(float v, uint32_t i) {
  uint32_t b = __float_as_uint(v);
  b = v != v ? 0x7FC00000u : v == 0.0f ? 0u : b;
  b ^= (b & 0x80000000u) ? 0xFFFFFFFFu : 0x80000000u;
  return (static_cast<uint64_t>(b) << 32) | static_cast<uint64_t>(~i);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m, 64);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m, 64);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// ARG: also the block's largest arg_key per token into keys[m, gridDim.x]
// (every wave then runs the token loop, the ones past the rows with no rows,
// for the block barrier each token group ends with).
template <int CPL, int MB, bool NORM, bool ARG>
__global__ __launch_bounds__(64 * kLinWaves) void int8_linear_kernel(
    const int8_t *__restrict__ q, const uint16_t *__restrict__ mu16, int64_t rows, int cols,
    const float *__restrict__ x, int64_t m_total, const float *__restrict__ norm_w, float eps, int rows_per_wave,
    float *__restrict__ y, uint64_t *__restrict__ keys) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kLinWaves + (threadIdx.x >> 6);
  const int64_t r_begin = wave * rows_per_wave;
  if (!ARG && r_begin >= rows) return;  // the whole wave (no block barriers without ARG)
  const int64_t r_end = min(rows, r_begin + rows_per_wave);
  const int nch = cols >> 4;
  __shared__ uint64_t best[2][kLinWaves][MB];
  for (int64_t m0 = 0; m0 < m_total; m0 += MB) {
    uint64_t kb = 0;  // ARG: this lane's best key, token m0 + lane % MB (lanes < 4 * MB)
    const int mb_here = static_cast<int>(min(static_cast<int64_t>(MB), m_total - m0));
    // Every load below comes from a clamped address with no branch around it
    // (a load under a divergent branch is waited for at once when the other
    // path writes the same register); out-of-range values are zeroed after.
    float xr[MB][CPL][16];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        const bool ok = c < nch && mb < mb_here;
        const float4 *src =
            reinterpret_cast<const float4 *>(x + (m0 + (mb < mb_here ? mb : 0)) * cols + 16 * (c < nch ? c : 0));
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float4 v = src[k];
          xr[mb][j][4 * k] = ok ? v.x : 0.f;
          xr[mb][j][4 * k + 1] = ok ? v.y : 0.f;
          xr[mb][j][4 * k + 2] = ok ? v.z : 0.f;
          xr[mb][j][4 * k + 3] = ok ? v.w : 0.f;
        }
      }
    if constexpr (NORM) {
      // x * rsqrt(mean(x^2) + eps) * w per token (pollux.py:580-582); every wave sums alike
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) ss = fmaf(xr[mb][j][e], xr[mb][j][e], ss);
        ss = wave_sum64(ss);
        const float r = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          const int c = lane + 64 * j;
          const float4 *g4 = reinterpret_cast<const float4 *>(norm_w + 16 * (c < nch ? c : 0));
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const float4 g = g4[k];  // lanes past the row scale zeros
            xr[mb][j][4 * k] = xr[mb][j][4 * k] * r * g.x;
            xr[mb][j][4 * k + 1] = xr[mb][j][4 * k + 1] * r * g.y;
            xr[mb][j][4 * k + 2] = xr[mb][j][4 * k + 2] * r * g.z;
            xr[mb][j][4 * k + 3] = xr[mb][j][4 * k + 3] * r * g.w;
          }
        }
      }
    }
    for (int64_t r0 = r_begin; r0 < r_end; r0 += 4) {
      uint4 qv[4][CPL];
      float sc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = r0 + i < r_end ? r0 + i : r_end - 1;  // rows past the end: loaded, never stored
        sc[i] = int8_row_scale(mu16[row]);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          const int c = lane + 64 * j;  // chunks past the row: loaded, never used
          qv[i][j] = *reinterpret_cast<const uint4 *>(q + row * cols + 16 * (c < nch ? c : 0));
        }
      }
      float acc[4][MB];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[i][mb] = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const __half2 s2 = __float2half2_rn(sc[i]);  // exact: sc is an fp16 value
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          if (lane + 64 * j >= nch) continue;
          const uint32_t d[4] = {qv[i][j].x, qv[i][j].y, qv[i][j].z, qv[i][j].w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            __half2 lo, hi;
            int8x4_weights(d[k], s2, lo, hi);
            const float w0 = __low2float(lo), w1 = __high2float(lo), w2 = __low2float(hi), w3 = __high2float(hi);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
              float a = acc[i][mb];
              a = fmaf(w0, xr[mb][j][4 * k], a);
              a = fmaf(w1, xr[mb][j][4 * k + 1], a);
              a = fmaf(w2, xr[mb][j][4 * k + 2], a);
              a = fmaf(w3, xr[mb][j][4 * k + 3], a);
              acc[i][mb] = a;
            }
          }
        }
      }
      float flat[4 * MB];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) flat[i * MB + mb] = acc[i][mb];
      group_reduce<64>(flat);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          if (lane == i * MB + mb && r0 + i < r_end && mb < mb_here) {
            y[(m0 + mb) * rows + r0 + i] = flat[i * MB + mb];
            if constexpr (ARG) {
              const uint64_t k = arg_key(flat[i * MB + mb], static_cast<uint32_t>(r0 + i));
              kb = k > kb ? k : kb;
            }
          }
    }
    if constexpr (ARG) {
      // lanes mb, MB + mb, 2 MB + mb, 3 MB + mb hold token mb's keys
      uint64_t o = shfl_xor_u64(kb, MB);
      kb = o > kb ? o : kb;
      o = shfl_xor_u64(kb, 2 * MB);
      kb = o > kb ? o : kb;
      const int par = static_cast<int>((m0 / MB) & 1);  // a buffer per parity: one barrier per token group
      if (lane < MB) best[par][threadIdx.x >> 6][lane] = kb;
      __syncthreads();
      if (threadIdx.x < MB && static_cast<int>(threadIdx.x) < mb_here) {
        uint64_t b = best[par][0][threadIdx.x];
#pragma unroll
        for (int w = 1; w < kLinWaves; ++w) b = best[par][w][threadIdx.x] > b ? best[par][w][threadIdx.x] : b;
        keys[(m0 + threadIdx.x) * gridDim.x + blockIdx.x] = b;
      }
    }
  }
}

typedef __bf16 bf16x8_i8 __attribute__((ext_vector_type(8)));
typedef float f32x4_i8 __attribute__((ext_vector_type(4)));

constexpr int kI8mmRows = 64;     // output rows per block (four MFMA row tiles)
constexpr int kI8mmWaves = 4;     // waves per block, splitting K
constexpr int kI8mmRedStride = 68; // floats per token row of the cross-wave sum (64 rows + pad)

// Two fp32 values rounded to bf16 (RNE) by one v_cvt_pk_bf16_f32, low half first.
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  typedef __bf16 bf16x2_i8 __attribute__((ext_vector_type(2)));
  const bf16x2_i8 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf16_lo_f32(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi_f32(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }

// 8 fp32 values split exactly into three bf16 parts (v = h + m + l while the
// parts stay normal; inf / nan go to h alone), packed as bf16x8 each
__device__ __forceinline__ void split3_bf16x8(const float (&v)[8], bf16x8_i8 &h, bf16x8_i8 &m, bf16x8_i8 &l) {
  uint32_t ph[4], pm[4], pl[4];
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const bool fa = fabsf(v[e]) <= 3.0e38f, fb = fabsf(v[e + 1]) <= 3.0e38f;
    ph[e / 2] = pk_bf16(v[e], v[e + 1]);
    const float ra = fa ? v[e] - bf16_lo_f32(ph[e / 2]) : 0.f, rb = fb ? v[e + 1] - bf16_hi_f32(ph[e / 2]) : 0.f;
    pm[e / 2] = pk_bf16(ra, rb);
    pl[e / 2] = pk_bf16(ra - bf16_lo_f32(pm[e / 2]), rb - bf16_hi_f32(pm[e / 2]));
  }
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  h = __builtin_bit_cast(bf16x8_i8, u4{ph[0], ph[1], ph[2], ph[3]});
  m = __builtin_bit_cast(bf16x8_i8, u4{pm[0], pm[1], pm[2], pm[3]});
  l = __builtin_bit_cast(bf16x8_i8, u4{pl[0], pl[1], pl[2], pl[3]});
}

// the 8 fp16 weights of 8 int8 values (bytes of d0, d1) times s2, split
// exactly into bf16 hi + lo (inf / nan weights, from an fp16 overflow of
// q * s16 or a nan scale, go to hi alone)
__device__ __forceinline__ void int8x8_hilo(uint32_t d0, uint32_t d1, __half2 s2, bf16x8_i8 &hi, bf16x8_i8 &lo) {
  __half2 w[4];
  int8x4_weights(d0, s2, w[0], w[1]);
  int8x4_weights(d1, s2, w[2], w[3]);
  uint32_t ph[4], pl[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = __low2float(w[i]), b = __high2float(w[i]);
    ph[i] = pk_bf16(a, b);
    const float ra = fabsf(a) <= 65504.0f ? a - bf16_lo_f32(ph[i]) : 0.f;
    const float rb = fabsf(b) <= 65504.0f ? b - bf16_hi_f32(ph[i]) : 0.f;
    pl[i] = pk_bf16(ra, rb);
  }
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  hi = __builtin_bit_cast(bf16x8_i8, u4{ph[0], ph[1], ph[2], ph[3]});
  lo = __builtin_bit_cast(bf16x8_i8, u4{pl[0], pl[1], pl[2], pl[3]});
}

template <int MT, bool NORM, bool ARG>
__global__ __launch_bounds__(64 * kI8mmWaves, 2) void int8mm_kernel(
    const int8_t *__restrict__ q, const uint16_t *__restrict__ mu16, int64_t rows, int cols,
    const float *__restrict__ x, int64_t m_total, const float *__restrict__ norm_w, float eps, float *__restrict__ y,
    uint64_t *__restrict__ keys) {
  constexpr int TOK = 16 * MT;
  __shared__ __align__(16) float red[kI8mmWaves][TOK][kI8mmRedStride];
  __shared__ float sq[kI8mmWaves][TOK];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, qd = lane >> 4;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kI8mmRows;
  const int64_t tok0 = static_cast<int64_t>(blockIdx.y) * TOK;
  const int nsteps = (cols + 31) / 32;
  const int sb = nsteps / kI8mmWaves, sx = nsteps % kI8mmWaves;
  const int s0 = wave * sb + min(wave, sx), sn = sb + (wave < sx ? 1 : 0);

  // per row tile: this lane's row scale (a row past the end takes the last row's: decoded, never stored)
  __half2 s2[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t row = row0 + 16 * r + j < rows ? row0 + 16 * r + j : rows - 1;
    s2[r] = __float2half2_rn(int8_row_scale(mu16[row]));  // exact: an fp16 value
  }
  // Raw buffer loads over the block's rows of q and tokens of x: a row or
  // token past the end, a column past the row and a step past the wave's
  // share fall outside the ranges and read as zeros (weight 0, activation 0),
  // so no load sits under a branch or feeds a select, and the ring below keeps
  // D steps of loads in flight (with the selects at load time every step
  // waited for its own loads).
  const int64_t rows_b = rows - row0 < kI8mmRows ? rows - row0 : kI8mmRows;
  const int64_t toks_b = m_total - tok0 < TOK ? m_total - tok0 : TOK;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t *>(q + row0 * cols), static_cast<short>(0), static_cast<int>(rows_b * cols), kBufferFlags);
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(x + tok0 * cols), static_cast<short>(0),
                                        static_cast<int>(toks_b * cols * 4), kBufferFlags);
  const __amdgpu_buffer_rsrc_t grs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(NORM ? norm_w : x), static_cast<short>(0), NORM ? cols * 4 : 0, kBufferFlags);

  f32x4_i8 acc[MT][4];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[t][r] = f32x4_i8{0.f, 0.f, 0.f, 0.f};
  float ssq[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) ssq[t] = 0.f;

  // Raw operands of one step (activations: 8 per token tile; weights: 8 bytes
  // per row tile; NORM: 8 norm weights) in a ring of D steps: the loads of
  // step i + D go out as step i is computed, so a wave keeps several HBM round
  // trips in flight (one step's work is far shorter than one trip).
  constexpr int D = 2;  // 2 measured faster than 3 or 4 at 5..256 tokens (fewer VGPRs: 3 waves per SIMD)
  uint4 xv[D][MT][2];
  uint2 wv[D][4];
  uint4 gv[D][NORM ? 2 : 1];
  auto load_step = [&](int step, uint4 (&xs)[MT][2], uint2 (&ws)[4], uint4 (&gs)[NORM ? 2 : 1]) {
    const int k = 32 * step + 8 * qd;
    const bool kok = k < cols && step < s0 + sn;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int off = kok ? (16 * r + j) * cols + k : kBufferOutOfRange;
      asm("" : "+v"(off));
      ws[r] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(wrs, off, 0, 0));
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      int off = kok ? ((16 * t + j) * cols + k) * 4 : kBufferOutOfRange;
      asm("" : "+v"(off));
      xs[t][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
      xs[t][1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 16, 0));
    }
    if constexpr (NORM) {
      int off = kok ? 4 * k : kBufferOutOfRange;
      asm("" : "+v"(off));
      gs[0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(grs, off, 0, 0));
      gs[1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(grs, off, 16, 0));
    }
  };
  auto compute_step = [&](const uint4 (&xs)[MT][2], const uint2 (&ws)[4], const uint4 (&gs)[NORM ? 2 : 1]) {
    float g[8];
    if constexpr (NORM) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        g[4 * h] = __uint_as_float(gs[h].x);
        g[4 * h + 1] = __uint_as_float(gs[h].y);
        g[4 * h + 2] = __uint_as_float(gs[h].z);
        g[4 * h + 3] = __uint_as_float(gs[h].w);
      }
    }
    bf16x8_i8 wh[4], wl[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) int8x8_hilo(ws[r].x, ws[r].y, s2[r], wh[r], wl[r]);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      float v[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        v[4 * h] = __uint_as_float(xs[t][h].x);
        v[4 * h + 1] = __uint_as_float(xs[t][h].y);
        v[4 * h + 2] = __uint_as_float(xs[t][h].z);
        v[4 * h + 3] = __uint_as_float(xs[t][h].w);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (NORM) {
          ssq[t] = fmaf(v[e], v[e], ssq[t]);
          v[e] = v[e] * g[e];
        }
      }
      bf16x8_i8 xh, xm, xl;
      split3_bf16x8(v, xh, xm, xl);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, wh[r], acc[t][r], 0, 0, 0);
        acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xm, wh[r], acc[t][r], 0, 0, 0);
        acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, wh[r], acc[t][r], 0, 0, 0);
        acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, wl[r], acc[t][r], 0, 0, 0);
        acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xm, wl[r], acc[t][r], 0, 0, 0);
        acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, wl[r], acc[t][r], 0, 0, 0);
      }
    }
  };
#pragma unroll
  for (int u = 0; u < D; ++u) load_step(s0 + u, xv[u], wv[u], gv[u]);
  for (int i = 0; i < sn; i += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      if (i + u < sn) {  // wave-uniform
        compute_step(xv[u], wv[u], gv[u]);
        load_step(s0 + i + u + D, xv[u], wv[u], gv[u]);  // past the wave's steps: out of range, zeros
      }
    }
  }

  // ---- epilogue: C[token 16t + 4qd + e][row 16r + j] of every wave into LDS, summed in wave order ----
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave][16 * t + 4 * qd + e][16 * r + j] = acc[t][r][e];
  if constexpr (NORM) {
    // token 16t + j: the four lane groups' sums, then the waves' (below)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      float v = ssq[t];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      if (qd == 0) sq[wave][16 * t + j] = v;
    }
  }
  __syncthreads();
  constexpr int kTpt = 64 * kI8mmWaves / TOK;  // threads per token
  constexpr int kRpt = kI8mmRows / kTpt;        // rows per thread
  const int tl = tid / kTpt, part = tid % kTpt;
  const int64_t tok = tok0 + tl;
  float rs = 1.0f;
  if constexpr (NORM) {
    float t2 = sq[0][tl];
#pragma unroll
    for (int w = 1; w < kI8mmWaves; ++w) t2 += sq[w][tl];
    rs = 1.0f / sqrtf(t2 / static_cast<float>(cols) + eps);
  }
  uint64_t kb = 0;
#pragma unroll
  for (int i = 0; i < kRpt; ++i) {
    const int rr = part + kTpt * i;
    float sum = red[0][tl][rr];
#pragma unroll
    for (int w = 1; w < kI8mmWaves; ++w) sum += red[w][tl][rr];
    if constexpr (NORM) sum *= rs;
    const int64_t row = row0 + rr;
    if (tok < m_total && row < rows) {
      y[tok * rows + row] = sum;
      if constexpr (ARG) {
        const uint64_t k = arg_key(sum, static_cast<uint32_t>(row));
        kb = k > kb ? k : kb;
      }
    }
  }
  if constexpr (ARG) {
#pragma unroll
    for (int d = 1; d < kTpt; d <<= 1) {
      const uint64_t o = shfl_xor_u64(kb, d);
      kb = o > kb ? o : kb;
    }
    if (part == 0 && tok < m_total) keys[tok * gridDim.x + blockIdx.x] = kb;
  }
}

constexpr int kPickThreads = 1024;
constexpr int kPickRegs = 8;  // keys in flight per lane and round

// The argmax of each token from the int8_linear_kernel blocks' keys
// [m, parts], in one block: R = min(16, pow2 >= m) tokens at a time, 16 / R
// waves per token.  ids[t] = the winning index; with pos, history[t, *pos + 1]
// = ids[t] (when inside [0, hist_len)) and then *pos += 1.
__global__ __launch_bounds__(kPickThreads) void argmax_pick_kernel(const uint64_t *__restrict__ keys, int parts,
                                                                   int64_t m, int rsh, int64_t *__restrict__ ids,
                                                                   int64_t *__restrict__ history, int64_t hist_len,
                                                                   int64_t *__restrict__ pos) {
  __shared__ uint64_t wbest[kPickThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int R = 1 << rsh, G = (kPickThreads / 64) >> rsh;  // tokens at a time, waves per token
  const int slot = wave / G, gw = wave % G;
  const int64_t p0 = pos ? pos[0] : 0;
  for (int64_t base = 0; base < m; base += R) {
    const int64_t t = base + slot;
    const uint64_t *kt = keys + (t < m ? t : 0) * parts;
    uint64_t kb = 0;
    for (int p = gw * 64 + lane; p < parts; p += G * 64 * kPickRegs) {
      uint64_t v[kPickRegs];
#pragma unroll
      for (int k = 0; k < kPickRegs; ++k) {
        const int pk = p + k * G * 64;
        v[k] = kt[pk < parts ? pk : 0];  // clamped: every load unconditional
      }
#pragma unroll
      for (int k = 0; k < kPickRegs; ++k) kb = v[k] > kb ? v[k] : kb;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint64_t o = shfl_xor_u64(kb, off);
      kb = o > kb ? o : kb;
    }
    if (lane == 0) wbest[wave] = kb;
    __syncthreads();
    if (gw == 0 && lane == 0 && t < m) {
      for (int w = 1; w < G; ++w) kb = wbest[wave + w] > kb ? wbest[wave + w] : kb;
      const int64_t id = static_cast<int64_t>(~static_cast<uint32_t>(kb));
      ids[t] = id;
      if (pos && history && p0 + 1 >= 0 && p0 + 1 < hist_len) history[t * hist_len + p0 + 1] = id;
    }
    __syncthreads();
  }
  if (pos && tid == 0) pos[0] = p0 + 1;
}

// one wave per token; cols % 4 == 0, q rows 4-byte aligned, pos_w / out 16-byte aligned
__global__ __launch_bounds__(256) void int8_embed_kernel(const int8_t *__restrict__ q,
                                                         const uint16_t *__restrict__ mu16, int64_t vocab, int cols,
                                                         const int64_t *__restrict__ idx, int64_t n, int64_t t,
                                                         const float *__restrict__ pos_w, int64_t pos_rows,
                                                         const int64_t *__restrict__ pos0, float *__restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t tok = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (tok >= n) return;
  const int64_t id = idx[tok];
  const int64_t p = pos_w ? (pos0 ? *pos0 : 0) + tok % t : 0;
  float4 *o = reinterpret_cast<float4 *>(out + tok * cols);
  if (id < 0 || id >= vocab || (pos_w && (p < 0 || p >= pos_rows))) {
    const float nan = __builtin_nanf("");
    for (int i = lane; i < cols / 4; i += 64) o[i] = make_float4(nan, nan, nan, nan);
    return;
  }
  const uint16_t mu = mu16[id];
  const uint32_t *qr = reinterpret_cast<const uint32_t *>(q + id * cols);
  const float4 *pr = pos_w ? reinterpret_cast<const float4 *>(pos_w + p * cols) : nullptr;
  const int n4 = cols / 4;
  auto emit = [&](int i, uint32_t b, float4 g, float s) {
    auto one = [&](int8_t v) { return __half2float(__float2half_rn(f32_kept(static_cast<float>(v) * s))); };
    float4 v = make_float4(one(static_cast<int8_t>(b)), one(static_cast<int8_t>(b >> 8)),
                           one(static_cast<int8_t>(b >> 16)), one(static_cast<int8_t>(b >> 24)));
    if (pr) v = make_float4(v.x + g.x, v.y + g.y, v.z + g.z, v.w + g.w);
    o[i] = v;
  };
  if (n4 <= 64 * kEmbedRegs) {
    // the whole row's loads in flight at once (clamped indices: no branch holds a load)
    uint32_t b[kEmbedRegs];
    float4 g[kEmbedRegs];
#pragma unroll
    for (int k = 0; k < kEmbedRegs; ++k) {
      const int i = lane + 64 * k < n4 ? lane + 64 * k : 0;
      b[k] = qr[i];
      g[k] = pr ? pr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float s = int8_row_scale(mu);
#pragma unroll
    for (int k = 0; k < kEmbedRegs; ++k)
      if (lane + 64 * k < n4) emit(lane + 64 * k, b[k], g[k], s);
  } else {
    const float s = int8_row_scale(mu);
    for (int i = lane; i < n4; i += 64) emit(i, qr[i], pr ? pr[i] : make_float4(0.f, 0.f, 0.f, 0.f), s);
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

int int8_linear_blocks(int64_t rows, int64_t *rows_per_wave) {
  // about 8 waves of 4-row groups per SIMD over the chip (1,024 SIMDs)
  int64_t rpw = (rows + 8 * 1024 - 1) / (8 * 1024);
  rpw = rpw < 4 ? 4 : (rpw + 3) / 4 * 4;
  if (rows_per_wave) *rows_per_wave = rpw;
  const int64_t waves = (rows + rpw - 1) / rpw;
  return static_cast<int>(std::min<int64_t>((waves + kLinWaves - 1) / kLinWaves, 0x7FFFFFFFll));
}

// From this many tokens the MFMA kernel runs: it reads the weights once for up
// to 64 tokens, the GEMV once per 4 tokens.  Measured on the Pollux head
// (50,688 x 1,920): GEMV 20.8 / 25.8 / 47.4 / 79.2 us at 1 / 2 / 4 / 5 tokens;
// MFMA 52-54 us at 5..16 tokens (VALU-bound by the weight decode and the exact
// bf16 splits: ~10 VALU instructions per weight), 67 at 17, 99 at 33, 170 at
// 65, 373 at 256 (torch F.linear on the cached fp32 cast: 70-73, 76, 95, 162,
// 392).
constexpr int64_t kI8mmMinTokens = 5;

int64_t int8mm_row_blocks(int64_t rows) { return (rows + kI8mmRows - 1) / kI8mmRows; }

int launch_int8mm(const int8_t *q, const uint16_t *mu16, int64_t rows, int cols, const float *x, int64_t m,
                  const float *norm_w, float eps, float *y, uint64_t *keys, hipStream_t s) {
  const int mt = m <= 16 ? 1 : m <= 32 ? 2 : 4;
  const int64_t slabs = (m + 16 * mt - 1) / (16 * mt);
  if (slabs > 0xFFFFll) return fail(PLX_EINVAL, "int8_linear: %lld tokens", static_cast<long long>(m));
  const dim3 g(static_cast<unsigned>(int8mm_row_blocks(rows)), static_cast<unsigned>(slabs)), b(64 * kI8mmWaves);
#define PLX_I8MM_K(MT, NORM)                                                                                        \
  do {                                                                                                              \
    if (keys)                                                                                                       \
      hipLaunchKernelGGL((int8mm_kernel<MT, NORM, true>), g, b, 0, s, q, mu16, rows, cols, x, m, norm_w, eps, y, keys); \
    else                                                                                                            \
      hipLaunchKernelGGL((int8mm_kernel<MT, NORM, false>), g, b, 0, s, q, mu16, rows, cols, x, m, norm_w, eps, y,    \
                         keys);                                                                                     \
  } while (0)
#define PLX_I8MM(MT)              \
  do {                            \
    if (norm_w)                   \
      PLX_I8MM_K(MT, true);       \
    else                          \
      PLX_I8MM_K(MT, false);      \
  } while (0)
  if (mt == 1)
    PLX_I8MM(1);
  else if (mt == 2)
    PLX_I8MM(2);
  else
    PLX_I8MM(4);
#undef PLX_I8MM
#undef PLX_I8MM_K
  return check_launch("int8mm_kernel");
}

// blocks of the kernel a call at m tokens launches (the argmax keys' parts)
int64_t int8_linear_parts(int64_t rows, int64_t m) {
  return m >= kI8mmMinTokens ? int8mm_row_blocks(rows) : int8_linear_blocks(rows, nullptr);
}

int launch_int8_linear(const int8_t *q, const uint16_t *mu16, int64_t rows, int64_t cols, const float *x, int64_t m,
                       const float *norm_w, float eps, float *y, uint64_t *keys, hipStream_t s) {
  if (rows == 0 || m == 0) return PLX_OK;
  if (cols <= 0 || cols % 16 != 0 || cols > 64 * 16 * 4)
    return fail(PLX_EINVAL, "int8_linear: %lld columns (a multiple of 16 up to 4,096)", static_cast<long long>(cols));
  const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(x) |
                       reinterpret_cast<uintptr_t>(norm_w);
  if ((al & 15u) != 0) return fail(PLX_EINVAL, "int8_linear: q, x and the norm weight must be 16-byte aligned");
  if (rows > 0x7FFFFFFFll) return fail(PLX_EINVAL, "int8_linear: too many rows");
  if (m >= kI8mmMinTokens) return launch_int8mm(q, mu16, rows, static_cast<int>(cols), x, m, norm_w, eps, y, keys, s);
  int64_t rpw = 0;
  const int blocks = int8_linear_blocks(rows, &rpw);
  const int cpl = static_cast<int>((cols / 16 + 63) / 64);
  const int mb = m >= 4 ? 4 : m >= 2 ? 2 : 1;
  const dim3 g(static_cast<unsigned>(blocks)), b(64 * kLinWaves);
  const int ci = static_cast<int>(cols);
  const int ri = static_cast<int>(rpw);
#define PLX_I8L_K(CPL, MB, NORM)                                                                                \
  do {                                                                                                          \
    if (keys)                                                                                                   \
      hipLaunchKernelGGL((int8_linear_kernel<CPL, MB, NORM, true>), g, b, 0, s, q, mu16, rows, ci, x, m, norm_w, \
                         eps, ri, y, keys);                                                                     \
    else                                                                                                        \
      hipLaunchKernelGGL((int8_linear_kernel<CPL, MB, NORM, false>), g, b, 0, s, q, mu16, rows, ci, x, m, norm_w, \
                         eps, ri, y, keys);                                                                     \
  } while (0)
#define PLX_I8L(CPL, MB)        \
  do {                          \
    if (norm_w)                 \
      PLX_I8L_K(CPL, MB, true); \
    else                        \
      PLX_I8L_K(CPL, MB, false); \
  } while (0)
#define PLX_I8L_MB(CPL)  \
  do {                   \
    if (mb == 4)         \
      PLX_I8L(CPL, 4);   \
    else if (mb == 2)    \
      PLX_I8L(CPL, 2);   \
    else                 \
      PLX_I8L(CPL, 1);   \
  } while (0)
  if (cpl == 1)
    PLX_I8L_MB(1);
  else if (cpl == 2)
    PLX_I8L_MB(2);
  else
    PLX_I8L_MB(4);
#undef PLX_I8L_MB
#undef PLX_I8L
#undef PLX_I8L_K
  return check_launch("int8_linear_kernel");
}

int launch_int8_linear_argmax(const int8_t *q, const uint16_t *mu16, int64_t rows, int64_t cols, const float *x,
                              int64_t m, const float *norm_w, float eps, float *y, int64_t *ids, int64_t *history,
                              int64_t hist_len, int64_t *pos, void *workspace, size_t workspace_bytes, hipStream_t s) {
  if (m == 0) return PLX_OK;
  if (rows <= 0 || rows > 0x7FFFFFFFll) return fail(PLX_EINVAL, "int8_linear_argmax: %lld rows", static_cast<long long>(rows));
  const int64_t parts = int8_linear_parts(rows, m);
  const size_t need = static_cast<size_t>(m) * static_cast<size_t>(parts) * sizeof(uint64_t);
  if (workspace == nullptr || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 7u) != 0)
    return fail(PLX_EINVAL, "int8_linear_argmax: workspace of %zu bytes (8-byte aligned) needed", need);
  uint64_t *keys = static_cast<uint64_t *>(workspace);
  const int st = launch_int8_linear(q, mu16, rows, cols, x, m, norm_w, eps, y, keys, s);
  if (st != PLX_OK) return st;
  int rsh = 0;
  while ((int64_t{1} << rsh) < m && rsh < 4) ++rsh;
  hipLaunchKernelGGL(argmax_pick_kernel, dim3(1), dim3(kPickThreads), 0, s, keys, static_cast<int>(parts), m, rsh, ids,
                     history, hist_len, pos);
  return check_launch("argmax_pick_kernel");
}

size_t int8_linear_argmax_workspace_bytes(int64_t rows, int64_t m) {
  if (rows <= 0 || m <= 0 || rows > 0x7FFFFFFFll) return 0;
  return static_cast<size_t>(m) * static_cast<size_t>(int8_linear_parts(rows, m)) * sizeof(uint64_t);
}

int launch_int8_embed(const int8_t *q, const uint16_t *mu16, int64_t vocab, int64_t cols, const int64_t *idx,
                      int64_t n, int64_t t, const float *pos_w, int64_t pos_rows, const int64_t *pos0, float *out,
                      hipStream_t s) {
  if (n == 0) return PLX_OK;
  if (cols <= 0 || cols % 4 != 0 || cols > (1 << 24) || t <= 0)
    return fail(PLX_EINVAL, "int8_embed: %lld columns (a positive multiple of 4), %lld tokens per row",
                static_cast<long long>(cols), static_cast<long long>(t));
  const uintptr_t al = reinterpret_cast<uintptr_t>(pos_w) | reinterpret_cast<uintptr_t>(out);
  if ((reinterpret_cast<uintptr_t>(q) & 3u) != 0 || (al & 15u) != 0)
    return fail(PLX_EINVAL, "int8_embed: q must be 4-byte and pos_w / out 16-byte aligned");
  const int64_t blocks = (n + 3) / 4;
  if (blocks > 0x7FFFFFFFll) return fail(PLX_EINVAL, "int8_embed: too many tokens");
  hipLaunchKernelGGL(int8_embed_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, q, mu16, vocab,
                     static_cast<int>(cols), idx, n, t, pos_w, pos_rows, pos0, out);
  return check_launch("int8_embed_kernel");
}

}  // namespace plx

// Leech nearest-neighbour quantizer on CDNA4 MFMA (replaces castor.py:374-560).
//
// Scores x.c of every atom against all 196,560 kissing points as a dense bf16
// contraction on v_mfma_f32_16x16x32_bf16 (K = 24 coordinates + 8 zero pad),
// keeping only a running maximum per (atom, lane) and the index of the code
// group where it was reached; no score is ever written to memory.
//
// Decomposition.
//   grid.x = atom_blocks * n_slices; block b works on atom block b / n_slices
//   and codebook slice b % n_slices.  Work-groups are dispatched round-robin
//   over the 8 XCDs, so with 8 (or 16) slices each XCD only ever streams its
//   own 1.18 (2.36) MB of the 9.4 MB bf16 codebook and serves it from its
//   4 MB L2.
//   A block is 4 waves; a wave holds 8 atom tiles of 16 atoms as MFMA B
//   operands in registers (512 atoms per block) and sweeps its slice, staged
//   through LDS 32 code tiles (24 KB) at a time, double buffered, with the
//   next stage streamed by global_load_lds while the current one is scored.
//   MFMA A operand = 16 codes x 32 K from LDS (lanes 48-63 re-read plane 0:
//   their K = 24..31 meet zero B entries).  Lane l of the 16x16 result holds
//   atom l%16 against codes 4*(l/16)..+3 of the tile.
//
// Selection semantics (per atom, codes in ascending index order).
//   NN-B (castor.py:549-557): bucket(s) = bf16_rne(s); winner = lowest code
//     with the maximal bucket M; origin iff 2*M < 0x407FFFFF, i.e. M < 2.0.
//   NN-T (castor.py:419-460): winner = lowest code with the maximal fp32
//     score S; origin iff 2*S < 0x407FFFFF.
//   Both are tracked with one integer threshold R per (atom, lane): a group of
//   4 tiles (16 codes per lane) improves when its max score, as an int bit
//   pattern, exceeds R (positive floats order like ints; negative scores can
//   only lose to the origin threshold R starts at).  NN-B raises R to the
//   largest fp32 that still rounds to the new bucket, so later codes in the
//   same bucket never displace the earlier group; NN-T raises R to the score.
//   At the end each lane that holds its atom's best R rescans its best group
//   exactly (fp64 sum of exact bf16 products, rounded to fp32 then bf16) to
//   pick the lowest code, and the lanes / slices merge through a 64-bit
//   atomicMax on (score bits << 32 | ~code).  MFMA's fp32 sum differs from the
//   exact one by < 2^-22 * sum|x_i c_i| (measured), so the result equals the
//   exact-score answer on every atom that is not a near-tie within that
//   envelope.

#include "plx_device.h"

namespace plx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kAT = 8;                                  // atom tiles per wave
constexpr int kG = 4;                                   // code tiles per tracking group
constexpr int kST = 32;                                 // code tiles per LDS stage
constexpr int kAtomsPerBlock = kWaves * kAT * 16;       // 512
constexpr int kStageBytes = kST * kTileBytes;           // 24,576
constexpr int kStageVecs = kStageBytes / 16;            // 1,536 uint4
constexpr int kLoadsPerThread = kStageVecs / kThreads;  // 6
static_assert(kStageVecs % kThreads == 0, "stage must split evenly over the block");
static_assert(kST % kG == 0, "groups must not straddle stages");

constexpr int kModeB = PLX_NN_BF16_SCORES;

template <int MODE>
__device__ __forceinline__ int initial_threshold() {
  // NN-B: largest fp32 whose bf16 rounding is below 2.0 (bf16 0x3FFF is odd).
  // NN-T: largest fp32 s with 2*s < 0x407FFFFF.
  return MODE == kModeB ? 0x3FFF7FFF : 0x3FFFFFFE;
}

template <int MODE>
__device__ __forceinline__ int raised_threshold(int gm) {
  if (MODE != kModeB) return gm;
  const uint32_t b = bf16_rne_bits(__int_as_float(gm));
  return static_cast<int>((b << 16) + 0x8000u - (b & 1u));
}

// Lattice coordinates 8q..8q+7 of atom a (zeros past the end / for q == 3).
// FUSED: x = (w / max(sigma[row], 1e-8)) / fp32(1/sqrt 2) (castor.py:332-333,
// pollux.py:882), both IEEE divisions.
template <bool FUSED>
__device__ __forceinline__ void load_coords8(const float *__restrict__ src, const float *__restrict__ sigma,
                                             int64_t atoms_per_row, int64_t n_atoms, int64_t a, int q, float *v) {
  if (a >= n_atoms || q >= 3) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.f;
    return;
  }
  const float4 *p = reinterpret_cast<const float4 *>(src + a * kDim + 8 * q);
  const float4 u0 = p[0], u1 = p[1];
  v[0] = u0.x; v[1] = u0.y; v[2] = u0.z; v[3] = u0.w;
  v[4] = u1.x; v[5] = u1.y; v[6] = u1.z; v[7] = u1.w;
  if (FUSED) {
    const float s = fmaxf(sigma[a / atoms_per_row], __uint_as_float(kEpsBits));
    const float sl = __uint_as_float(kSLatticeBits);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (v[e] / s) / sl;
  }
}

template <int MODE, bool FUSED>
__global__ __launch_bounds__(kThreads, 2) void nn_kernel(const float *__restrict__ src,
                                                          const float *__restrict__ sigma, int64_t atoms_per_row,
                                                          int64_t n_atoms, const uint8_t *__restrict__ tiles,
                                                          const int8_t *__restrict__ cb_raw, int n_slices,
                                                          int tiles_per_slice,
                                                          unsigned long long *__restrict__ keys) {
  __shared__ __align__(16) uint8_t lds[2][kStageBytes];

  const int slice = static_cast<int>(blockIdx.x % static_cast<unsigned>(n_slices));
  const int64_t ablock = blockIdx.x / static_cast<unsigned>(n_slices);
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, q = lane >> 4, j = lane & 15;
  const int64_t wave_atom0 = ablock * kAtomsPerBlock + static_cast<int64_t>(wave) * (kAT * 16);

  // B operands: 8 atom tiles, lane holds coordinates 8q..8q+7 of atom j.
  bf16x8 b[kAT];
#pragma unroll
  for (int at = 0; at < kAT; ++at) {
    float v[8];
    load_coords8<FUSED>(src, sigma, atoms_per_row, n_atoms, wave_atom0 + at * 16 + j, q, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) b[at][e] = __builtin_bit_cast(__bf16, static_cast<uint16_t>(bf16_rne_bits(v[e])));
  }

  int R[kAT], best[kAT];
#pragma unroll
  for (int at = 0; at < kAT; ++at) {
    R[at] = initial_threshold<MODE>();
    best[at] = -1;
  }

  const int t0 = slice * tiles_per_slice;
  const int n_stages = tiles_per_slice / kST;
  const uint4 *gsrc = reinterpret_cast<const uint4 *>(tiles + static_cast<size_t>(t0) * kTileBytes);
  // Stage s is copied HBM/L2 -> LDS by global_load_lds_dwordx4 (no VGPR
  // staging): wave w, lane l moves vector i*256 + 64w + l, so each wave fills
  // a contiguous KiB of the buffer.
  auto stage_copy = [&](int stage, int dst_buf) {
#pragma unroll
    for (int i = 0; i < kLoadsPerThread; ++i) {
      const uint4 *g = gsrc + static_cast<size_t>(stage) * kStageVecs + i * kThreads + tid;
      uint8_t *d = lds[dst_buf] + (i * kThreads + wave * 64) * 16;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(g),
                                       (__attribute__((address_space(3))) void *)(d), 16, 0, 0);
    }
  };
  stage_copy(0, 0);
  __syncthreads();

  const int a_off = (q < 3 ? q : 0) * 256 + j * 16;
  for (int st = 0; st < n_stages; ++st) {
    const int buf = st & 1;
    if (st + 1 < n_stages) stage_copy(st + 1, buf ^ 1);
    const uint8_t *L = lds[buf] + a_off;
    const int group0 = (t0 + st * kST) / kG;
#pragma unroll 1
    for (int g = 0; g < kST / kG; ++g) {
      int gm[kAT];
#pragma unroll
      for (int at = 0; at < kAT; ++at) gm[at] = INT_MIN;
#pragma unroll
      for (int t = 0; t < kG; ++t) {
        const bf16x8 a = *reinterpret_cast<const bf16x8 *>(L + (g * kG + t) * kTileBytes);
#pragma unroll
        for (int at = 0; at < kAT; ++at) {
          const f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[at], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          // written as a chain so each pair folds into one v_max3_i32
          gm[at] = max(max(gm[at], __float_as_int(c[0])), __float_as_int(c[1]));
          gm[at] = max(max(gm[at], __float_as_int(c[2])), __float_as_int(c[3]));
        }
      }
      // Improvements get rare once the running maxima settle: test all atom
      // tiles, and take the update path only when some lane of the wave needs it.
      bool any_up = false;
#pragma unroll
      for (int at = 0; at < kAT; ++at) any_up |= gm[at] > R[at];
      if (__builtin_expect(__ballot(any_up) != 0ull, 0)) {
#pragma unroll
        for (int at = 0; at < kAT; ++at) {
          if (gm[at] > R[at]) {
            R[at] = raised_threshold<MODE>(gm[at]);
            best[at] = group0 + g;
          }
        }
      }
    }
    __syncthreads();
  }

  // ---- resolve: exact rescan of the best group of each candidate lane ----
  const double s1 = static_cast<double>(bf16_bits_to_float(bf16_rne_bits(raw_value_f32(1))));
  const double s2 = static_cast<double>(bf16_bits_to_float(bf16_rne_bits(raw_value_f32(2))));
  const double s3 = static_cast<double>(bf16_bits_to_float(bf16_rne_bits(raw_value_f32(3))));
  const double s4 = static_cast<double>(bf16_bits_to_float(bf16_rne_bits(raw_value_f32(4))));
#pragma unroll 1
  for (int at = 0; at < kAT; ++at) {
    int Rm = R[at];
    Rm = max(Rm, __shfl_xor(Rm, 16, 64));
    Rm = max(Rm, __shfl_xor(Rm, 32, 64));
    const int64_t a = wave_atom0 + at * 16 + j;
    uint32_t key_hi = 0, key_lo = 0;
    if (best[at] >= 0 && R[at] == Rm && a < n_atoms) {
      double xs[kDim];
#pragma unroll
      for (int qq = 0; qq < 3; ++qq) {
        float v[8];
        load_coords8<FUSED>(src, sigma, atoms_per_row, n_atoms, a, qq, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) xs[8 * qq + e] = static_cast<double>(bf16_bits_to_float(bf16_rne_bits(v[e])));
      }
      const uint32_t target = MODE == kModeB ? (static_cast<uint32_t>(R[at]) >> 16) : 0u;
      bool found = false;
      uint32_t found_code = 0;
      float best_v = -__builtin_inff();
      uint32_t best_code = 0;
      for (int t = 0; t < kG; ++t) {
        for (int e = 0; e < 4; ++e) {
          const int code = (best[at] * kG + t) * kTileCodes + 4 * q + e;  // kissing index
          if (code >= kKissing) continue;
          const int8_t *cr = cb_raw + static_cast<size_t>(code + 1) * kDim;
          double s = 0.0;
#pragma unroll
          for (int k = 0; k < kDim; ++k) {
            const int r = cr[k];
            const int m = r < 0 ? -r : r;
            double c = m == 1 ? s1 : m == 2 ? s2 : m == 3 ? s3 : m == 4 ? s4 : 0.0;
            c = r < 0 ? -c : c;
            s = fma(xs[k], c, s);
          }
          const float s32 = static_cast<float>(s);
          float v = s32;
          if (MODE == kModeB) {
            const uint32_t bk = bf16_rne_bits(s32);
            v = bf16_bits_to_float(bk);
            if (!found && bk == target) {
              found = true;
              found_code = static_cast<uint32_t>(code);
            }
          }
          if (v > best_v) {
            best_v = v;
            best_code = static_cast<uint32_t>(code);
          }
        }
      }
      uint32_t code = best_code;
      float v = best_v;
      if (MODE == kModeB && found) {
        code = found_code;
        v = bf16_bits_to_float(target);
      }
      if (v > 0.f) {
        key_hi = MODE == kModeB ? (__float_as_uint(v) >> 16) : __float_as_uint(v);
        key_lo = 0xFFFFFFFFu - code;
      }
    }
    // merge the four lanes of atom j: max of (key_hi, key_lo) lexicographically
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
      const uint32_t oh = static_cast<uint32_t>(__shfl_xor(static_cast<int>(key_hi), off, 64));
      const uint32_t ol = static_cast<uint32_t>(__shfl_xor(static_cast<int>(key_lo), off, 64));
      if (oh > key_hi || (oh == key_hi && ol > key_lo)) {
        key_hi = oh;
        key_lo = ol;
      }
    }
    if (q == 0 && a < n_atoms && (key_hi | key_lo) != 0u)
      atomicMax(keys + a, (static_cast<unsigned long long>(key_hi) << 32) | key_lo);
  }
}

__global__ void fill_u64_kernel(unsigned long long *__restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0ull;
}

// keys -> int32 indices (and optionally the packed 9-byte groups); one thread per group of 4 atoms.
template <int MODE>
__global__ __launch_bounds__(256) void finalize_kernel(const unsigned long long *__restrict__ keys, int64_t n,
                                                       int32_t *__restrict__ idx_out,
                                                       uint8_t *__restrict__ packed_out, int64_t n_groups) {
  __shared__ __align__(16) uint8_t lds[256 * 9];
  const int64_t g0 = static_cast<int64_t>(blockIdx.x) * 256;
  const int64_t g = g0 + threadIdx.x;
  if (g < n_groups) {
    int32_t v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int64_t a = g * 4 + k;
      int32_t id = 0;
      if (a < n) {
        const unsigned long long key = keys[a];
        const uint32_t hi = static_cast<uint32_t>(key >> 32);
        const uint32_t code = 0xFFFFFFFFu - static_cast<uint32_t>(key);
        bool snap = key == 0ull;
        if (!snap) {
          if (MODE == kModeB)
            snap = hi < 0x4000u;  // bf16 max below 2.0
          else
            snap = 2.0f * __uint_as_float(hi) < __uint_as_float(kCSqNormBits);
        }
        id = snap ? 0 : static_cast<int32_t>(code) + 1;
        idx_out[a] = id;
      }
      v[k] = id;
    }
    if (packed_out) group_to_bytes(v[0], v[1], v[2], v[3], lds + threadIdx.x * 9);
  }
  if (!packed_out) return;
  __syncthreads();
  const int64_t groups_here = min(static_cast<int64_t>(256), n_groups - g0);
  uint8_t *dst = packed_out + g0 * 9;
  if (groups_here == 256 && aligned16(packed_out)) {
    if (threadIdx.x < 144) reinterpret_cast<uint4 *>(dst)[threadIdx.x] = reinterpret_cast<const uint4 *>(lds)[threadIdx.x];
  } else {
    const int nb = static_cast<int>(groups_here * 9);
    for (int i = threadIdx.x; i < nb; i += 256) dst[i] = lds[i];
  }
}

// out[a*24 + c] = value(codebook[idx[a]][c]); SCALE: (v * sigma[row]) * fp32(1/sqrt 2).
// One thread per 4 consecutive elements (never straddles an atom).
template <int OUT, bool SCALE>  // OUT: 0 fp32, 1 fp16, 2 bf16
__global__ __launch_bounds__(256) void gather_kernel(const int32_t *__restrict__ idx, int64_t n_atoms,
                                                     const int8_t *__restrict__ cb_raw,
                                                     const float *__restrict__ sigma, int64_t atoms_per_row,
                                                     void *__restrict__ out) {
  const int64_t e4 = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e4 >= n_atoms * 6) return;
  const int64_t a = e4 / 6;
  const int c0 = static_cast<int>(e4 % 6) * 4;
  int32_t code = idx[a];
  if (static_cast<uint32_t>(code) > static_cast<uint32_t>(kKissing)) code = 0;  // memory safety for bad input
  const uint32_t packed4 = *reinterpret_cast<const uint32_t *>(cb_raw + static_cast<size_t>(code) * kDim + c0);
  float v[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = raw_value_f32(static_cast<int8_t>((packed4 >> (8 * k)) & 0xFFu));
  if (SCALE) {
    const float s = sigma[a / atoms_per_row];
    const float sl = __uint_as_float(kSLatticeBits);
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = (v[k] * s) * sl;
  }
  if (OUT == 0) {
    reinterpret_cast<float4 *>(out)[e4] = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    uint32_t h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) h[k] = OUT == 1 ? __half_as_ushort(__float2half_rn(v[k])) : bf16_rne_bits(v[k]);
    reinterpret_cast<uint2 *>(out)[e4] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
  }
}

int choose_slices(int64_t ablocks) {
  int s = 8;
  while (s < 64 && ablocks * s < 2048) s *= 2;
  return s;
}

}  // namespace

size_t quantize_workspace_bytes(int64_t n_atoms) {
  return static_cast<size_t>((n_atoms * 8 + 255) / 256 * 256);
}

int launch_quantize(const float *x, const float *sigma, int64_t rows, int64_t cols, int64_t n_atoms, int mode,
                    int32_t *idx_out, uint8_t *packed_out, float *weight_out, void *workspace,
                    size_t workspace_bytes, hipStream_t s) {
  if (n_atoms <= 0) return PLX_OK;
  if (workspace == nullptr || workspace_bytes < quantize_workspace_bytes(n_atoms))
    return fail(PLX_EINVAL, "quantize: workspace of %zu bytes is smaller than the %zu needed for %lld atoms",
                workspace_bytes, quantize_workspace_bytes(n_atoms), static_cast<long long>(n_atoms));
  if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0)
    return fail(PLX_EINVAL, "quantize: input must be 16-byte aligned");
  const DeviceTables *tab = nullptr;
  int st = get_tables(&tab);
  if (st != PLX_OK) return st;

  unsigned long long *keys = static_cast<unsigned long long *>(workspace);
  hipLaunchKernelGGL(fill_u64_kernel, dim3(static_cast<unsigned>((n_atoms + 255) / 256)), dim3(256), 0, s, keys,
                     n_atoms);
  if ((st = check_launch("fill_u64_kernel")) != PLX_OK) return st;

  const int64_t ablocks = (n_atoms + kAtomsPerBlock - 1) / kAtomsPerBlock;
  const int n_slices = choose_slices(ablocks);
  const int tiles_per_slice = kPaddedTiles / n_slices;
  const int64_t grid = ablocks * n_slices;
  if (grid > 0x7FFFFFFFll) return fail(PLX_EINVAL, "quantize: %lld atoms exceed one launch", static_cast<long long>(n_atoms));
  const bool fused = sigma != nullptr;
  const int64_t apr = cols / kDim;
  const dim3 g(static_cast<unsigned>(grid)), b(kThreads);
  profile_before(s);
  if (mode == PLX_NN_BF16_SCORES) {
    if (fused)
      hipLaunchKernelGGL((nn_kernel<PLX_NN_BF16_SCORES, true>), g, b, 0, s, x, sigma, apr, n_atoms, tab->kp_bf16_tiles,
                         tab->cb_raw, n_slices, tiles_per_slice, keys);
    else
      hipLaunchKernelGGL((nn_kernel<PLX_NN_BF16_SCORES, false>), g, b, 0, s, x, sigma, apr, n_atoms,
                         tab->kp_bf16_tiles, tab->cb_raw, n_slices, tiles_per_slice, keys);
  } else {
    if (fused)
      hipLaunchKernelGGL((nn_kernel<PLX_NN_FP32_SCORES, true>), g, b, 0, s, x, sigma, apr, n_atoms, tab->kp_bf16_tiles,
                         tab->cb_raw, n_slices, tiles_per_slice, keys);
    else
      hipLaunchKernelGGL((nn_kernel<PLX_NN_FP32_SCORES, false>), g, b, 0, s, x, sigma, apr, n_atoms,
                         tab->kp_bf16_tiles, tab->cb_raw, n_slices, tiles_per_slice, keys);
  }
  if ((st = check_launch("nn_kernel")) != PLX_OK) return st;
  profile_after(s);

  const int64_t n_groups = (n_atoms + 3) / 4;
  const dim3 fg(static_cast<unsigned>((n_groups + 255) / 256));
  if (mode == PLX_NN_BF16_SCORES)
    hipLaunchKernelGGL(finalize_kernel<PLX_NN_BF16_SCORES>, fg, dim3(256), 0, s, keys, n_atoms, idx_out, packed_out,
                       n_groups);
  else
    hipLaunchKernelGGL(finalize_kernel<PLX_NN_FP32_SCORES>, fg, dim3(256), 0, s, keys, n_atoms, idx_out, packed_out,
                       n_groups);
  if ((st = check_launch("finalize_kernel")) != PLX_OK) return st;

  if (weight_out) {
    const dim3 gg(static_cast<unsigned>((n_atoms * 6 + 255) / 256));
    hipLaunchKernelGGL((gather_kernel<0, true>), gg, dim3(256), 0, s, idx_out, n_atoms, tab->cb_raw, sigma, apr,
                       static_cast<void *>(weight_out));
    if ((st = check_launch("gather_kernel")) != PLX_OK) return st;
  }
  (void)rows;
  return PLX_OK;
}

int launch_gather(const int32_t *idx, int64_t n, int out_dtype, void *out, hipStream_t s) {
  const DeviceTables *tab = nullptr;
  int st = get_tables(&tab);
  if (st != PLX_OK) return st;
  const dim3 gg(static_cast<unsigned>((n * 6 + 255) / 256));
  if (out_dtype == 0)
    hipLaunchKernelGGL((gather_kernel<0, false>), gg, dim3(256), 0, s, idx, n, tab->cb_raw, nullptr, int64_t{1}, out);
  else if (out_dtype == 1)
    hipLaunchKernelGGL((gather_kernel<1, false>), gg, dim3(256), 0, s, idx, n, tab->cb_raw, nullptr, int64_t{1}, out);
  else
    hipLaunchKernelGGL((gather_kernel<2, false>), gg, dim3(256), 0, s, idx, n, tab->cb_raw, nullptr, int64_t{1}, out);
  return check_launch("gather_kernel");
}

}  // namespace plx

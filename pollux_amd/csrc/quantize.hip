// Leech nearest-neighbour quantizer on CDNA4 MFMA (replaces castor.py:374-560).
//
// Scores x.c of every atom against the 196,560 kissing points as a dense bf16
// contraction on v_mfma_f32_16x16x32_bf16 (K = 24 coordinates + 8 zero pad),
// keeping only a running maximum per (atom, lane) and the index of the code
// group where it was reached; no score is ever written to memory.  The sweep
// covers 147,432 codes: the 98,304 type-3 codes and one representative per
// antipodal pair of the type-1/2 codes, whose |score| stands for both members
// (plx_internal.h).
//
// nn_kernel -- the scoring sweep.
//   grid.x = atom_blocks * n_slices; block b works on atom block b / n_slices
//   and codebook slice b % n_slices.  Large launches use one slice: every
//   block sweeps the whole 7.1 MB bf16 sweep table and reads its atoms' bf16
//   planes once; the blocks resident on an XCD sweep the table at nearby
//   positions and share its 4 MB L2 (~97% hits), the rest comes from MALL.
//   Small launches split the table into slices so the grid fills the chip.
//   A block is 4 waves; a wave holds 12 atom tiles of 16 atoms as MFMA B
//   operands in registers (768 atoms per block) and sweeps its slice, staged
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
//   NN-P (pack.py:167-177): fp32 atom against the fp32 codebook, winner =
//     lowest code with the maximal score; origin iff |x|_2 < 1e-8.  The atom
//     is split exactly into three bf16 parts (x = h + m + l up to 2^-27|x|)
//     and scored against the raw integer codes (exact in bf16) by three
//     chained MFMAs per tile; the fp32 codebook is the raw table times
//     fp32(1/sqrt 8) (3s rounded), so these scores order the codes like the
//     fp32 ones up to 2^-21 * sum|x_i c_i|, inside the near-tie envelope.
//   Both are tracked with one integer threshold R per (atom, lane): a group of
//   kG tiles (4 kG codes per lane) improves when its max score, as an int bit
//   pattern, exceeds R (positive floats order like ints; negative scores can
//   only lose to the origin threshold R starts at).  NN-B raises R to the
//   largest fp32 that still rounds to the new bucket, so later codes in the
//   same bucket never displace the earlier group; NN-T raises R to the score.
//   Each (atom, slice) ends as one atomic max into the atom's key word:
//   (best bucket or score, 1023 - earliest group reaching it, mask of the
//   atom's four lanes whose earliest group that is), 32 bits for NN-B
//   (bucket << 16 | (1023 - g) << 6 | mask << 2), 64 bits for NN-T / NN-P
//   (score << 32 | (1023 - g) << 4 | mask).  Slices own disjoint groups, so
//   the maximum over slices is the highest bucket / score, then the earliest
//   group holding it -- the group of the lowest code the selection rule
//   wants -- and no two slices write the same (score, group).  prep_kernel
//   (NN-P: clear_keys_kernel) zeroes the keys; 0 means the origin threshold
//   was never beaten.
//
// resolve_kernel -- per atom its key, then an exact-product rescan
//   (v_dot2_f32_bf16; NN-P: fp64 dot products of the fp32 atom and the fp32
//   codebook rows, exact up to 2^-48) of the key's group in the lanes of its
//   mask to find the lowest code, 4 lanes per (group, lane) with coalesced
//   table reads, then the index and the packed 9-byte groups.  Both fp32 sums
//   (MFMA, dot2) lie within 24 * 2^-24 * sum|x_i c_i| of the exact score
//   (MFMA measured at < 2^-22), so the result equals the exact-score answer
//   on every atom that is not a near-tie within that envelope.

#include <mutex>
#include <type_traits>

#include "plx_device.h"

namespace plx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kAT = 12;                                 // atom tiles per wave
constexpr int kG = 16;                                  // code tiles per tracking group
constexpr int kST = 32;                                 // code tiles per LDS stage
constexpr int kAtomsPerBlock = kWaves * kAT * 16;       // 768
constexpr int kStageBytes = kST * kTileBytes;           // 24,576
constexpr int kStageVecs = kStageBytes / 16;            // 1,536 uint4
constexpr int kLoadsPerThread = kStageVecs / kThreads;  // 6
static_assert(kStageVecs % kThreads == 0, "stage must split evenly over the block");
static_assert(kST % kG == 0 && kG >= 8 && kG <= 64 && (kG & (kG - 1)) == 0, "whole groups per LDS stage");

constexpr int kModeB = PLX_NN_BF16_SCORES;
constexpr int kModeP = PLX_NN_PACK_FP32;

// bf16 parts per atom coordinate: NN-P carries the fp32 value as h + m + l.
template <int MODE>
constexpr int n_splits() {
  return MODE == kModeP ? 3 : 1;
}

template <int MODE>
__device__ __forceinline__ int initial_threshold() {
  // NN-B: the largest group key of bucket 0x3FFF (bf16 max below 2.0); any
  //       group reaching bucket 0x4000 has a larger key (group_key).
  // NN-T: largest fp32 s with 2*s < 0x407FFFFF.
  // NN-P: +0.0 -- no score threshold (every nonzero atom has a positive
  //       maximum: the best +-4 pair scores 4s(|x_i| + |x_j|)).
  return MODE == kModeB ? 0x3FFFFFFF : MODE == kModeP ? 0 : 0x3FFFFFFE;
}

// New threshold after a group whose maximum is gm.  NN-T: gm itself.  NN-B:
// the largest fp32 bit pattern in gm's bf16 bucket, with the bucket taken by
// round-half-up ((gm + 0x8000) >> 16) -- two VALU ops instead of five.  It
// differs from round-to-nearest-even only when gm's low 16 bits are exactly
// 0x8000, a score sitting exactly on a bf16 rounding midpoint, which the
// parity oracle classifies as a near-tie.
template <int MODE>
__device__ __forceinline__ int raised_threshold(int gm) {
  if (MODE != kModeB) return gm;
  return static_cast<int>(((static_cast<uint32_t>(gm) + 0x8000u) & 0xFFFF0000u) | 0x7FFFu);
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

// bf16 lattice coordinates of every atom, row-major [n_atoms][24] (one
// 16-byte plane of 8 per thread), written once per launch so the scoring
// blocks of all slices load ready-made MFMA B operands instead of each
// repeating the row-scale divisions.  NN-B / NN-T only.
// Also clears the atoms' 16-byte key slots before nn_kernel merges its
// slices into them.
template <bool FUSED>
__global__ __launch_bounds__(256) void prep_kernel(const float *__restrict__ src, const float *__restrict__ sigma,
                                                   int64_t atoms_per_row, int64_t n_atoms, uint4 *__restrict__ xb,
                                                   uint4 *__restrict__ keys) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // plane i % 3 of atom i / 3
  if (i >= n_atoms * 3) return;
  const int64_t a = i / 3;
  if (i == 3 * a) keys[a] = make_uint4(0u, 0u, 0u, 0u);
  float v[8];
  load_coords8<FUSED>(src, sigma, atoms_per_row, n_atoms, a, static_cast<int>(i - 3 * a), v);
  uint4 w;
  w.x = bf16_rne_bits(v[0]) | (bf16_rne_bits(v[1]) << 16);
  w.y = bf16_rne_bits(v[2]) | (bf16_rne_bits(v[3]) << 16);
  w.z = bf16_rne_bits(v[4]) | (bf16_rne_bits(v[5]) << 16);
  w.w = bf16_rne_bits(v[6]) | (bf16_rne_bits(v[7]) << 16);
  xb[i] = w;
}

// NN-P has no prep pass: its key slots are cleared here.
__global__ __launch_bounds__(256) void clear_keys_kernel(uint4 *__restrict__ keys, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) keys[i] = make_uint4(0u, 0u, 0u, 0u);
}

// NN-B tracking key of a type-3 group: bucket (round-half-up, see
// raised_threshold) in the high half, 0xFFFF - group in the low half, so one
// signed max keeps the highest bucket and, within it, the earliest group.
// v_perm_b32 takes bytes 2-3 of the rounded score and bytes 0-1 of the
// (uniform) group field in one instruction.
__device__ __forceinline__ int group_key(int gm, int group) {
  return static_cast<int>(__builtin_amdgcn_perm(static_cast<uint32_t>(gm) + 0x8000u,
                                                static_cast<uint32_t>(0xFFFF - group) & 0xFFFFu, 0x07060100u));
}

// NN-B tracking of a pair group g (index within the slice's pair range,
// < 256) whose max |score| is gm, in one unsigned word: bucket << 17 | many <<
// 16 | (255 - first) << 8 | last -- the earliest and the latest group at the
// highest bucket, and whether a third group reached it.  A higher bucket
// replaces the word (first = last = g); the same bucket keeps first, moves
// last to g and sets `many` if first != last already.  The resolve then
// knows every group at the best bucket (first and last of each lane) unless
// `many` is set.  The bucket of a positive score (< 0x8000) fits 15 bits;
// kPairInit (bucket 0x3FFF) is below every hit (bucket >= 0x4000).
constexpr uint32_t kPairInit = 0x7FFFFFFFu;
__device__ __forceinline__ uint32_t pair_key(uint32_t R, int gm, int g) {
  const uint32_t gf = static_cast<uint32_t>(g) & 0xFFu;
  const uint32_t bk = (static_cast<uint32_t>(gm) + 0x8000u) >> 16;  // bucket, round half up
  const uint32_t nk = (bk << 17) | ((255u - gf) << 8) | gf;
  const uint32_t t = max(R, nk);
  // (255 - first) + last + 1 is 0 mod 256 exactly when first == last
  const uint32_t many = (((t >> 8) + t + 1u) & 0xFFu) != 0u ? 0x10000u : 0u;
  return ((t ^ nk) >> 17) == 0u ? (t & 0xFFFFFF00u) | many | gf : t;
}

// Lane mask (bit k = lane j + 16k, the four lanes of atom j) from a wave ballot.
__device__ __forceinline__ uint32_t atom_lanes(uint64_t bal, int j) {
  return static_cast<uint32_t>(((bal >> j) & 1u) | ((bal >> (j + 15)) & 2u) | ((bal >> (j + 30)) & 4u) |
                               ((bal >> (j + 45)) & 8u));
}

// src: NN-P: the fp32 atoms; NN-B / NN-T: xb, the bf16 planes of prep_kernel.
// tiles: the sweep-order tiles (type-3 codes, then pair representatives).
// recs (NN-B): one record per (atom, slice >= s0, the slices holding pair
// tiles), [slice - s0][n_atoms].
// NN-B: at most 168 VGPRs (3 waves per SIMD; the MFMA issue rate needs the
// third wave), which costs two 8-byte spills outside the scoring loops;
// NN-T / NN-P keep 2 waves per SIMD (their wider keys and split operands
// would spill inside the loops at 168).
template <int MODE>
__global__ __launch_bounds__(kThreads, MODE == kModeB ? 3 : 2) void nn_kernel(const void *__restrict__ src,
                                                                             int64_t n_atoms,
                                                          const uint8_t *__restrict__ tiles, int n_slices,
                                                          int tiles_per_slice, uint4 *__restrict__ keys,
                                                          uint64_t *__restrict__ recs, int s0) {
  __shared__ __align__(16) uint8_t lds[2][kStageBytes];

  const int slice = static_cast<int>(blockIdx.x % static_cast<unsigned>(n_slices));
  const int64_t ablock = blockIdx.x / static_cast<unsigned>(n_slices);
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, q = lane >> 4, j = lane & 15;
  const int64_t wave_atom0 = ablock * kAtomsPerBlock + static_cast<int64_t>(wave) * (kAT * 16);

  // B operands: kAT atom tiles, lane holds coordinates 8q..8q+7 of atom j
  // (NN-P: as three bf16 parts, b[0] + b[1] + b[2]).
  constexpr int NS = n_splits<MODE>();
  bf16x8 b[NS][kAT];
#pragma unroll
  for (int at = 0; at < kAT; ++at) {
    const int64_t a = wave_atom0 + at * 16 + j;
    if constexpr (NS == 1) {
      uint4 w = make_uint4(0u, 0u, 0u, 0u);
      if (a < n_atoms && q < 3) w = static_cast<const uint4 *>(src)[a * 3 + q];
      b[0][at] = __builtin_bit_cast(bf16x8, w);
      continue;
    }
    float v[8];
    load_coords8<false>(static_cast<const float *>(src), nullptr, 1, n_atoms, a, q, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t h = bf16_rne_bits(v[e]);
      b[0][at][e] = __builtin_bit_cast(__bf16, static_cast<uint16_t>(h));
      if constexpr (NS == 3) {
        const float r1 = v[e] - bf16_bits_to_float(h);  // exact
        const uint32_t m = bf16_rne_bits(r1);
        const float r2 = r1 - bf16_bits_to_float(m);    // exact
        b[1][at][e] = __builtin_bit_cast(__bf16, static_cast<uint16_t>(m));
        b[2][at][e] = __builtin_bit_cast(__bf16, static_cast<uint16_t>(bf16_rne_bits(r2)));
      }
    }
  }

  const int t0 = slice * tiles_per_slice;
  const int n_stages = tiles_per_slice / kST;
  // stages [0, n_t) hold type-3 tiles, [n_t, n_stages) pair representatives
  // (the region boundary falls on a stage boundary)
  const int n_t = min(max(kType3Tiles - t0, 0) / kST, n_stages);
  const uint4 *gsrc = reinterpret_cast<const uint4 *>(tiles + static_cast<size_t>(t0) * kTileBytes);
  // Stage s is copied L2 -> LDS by global_load_lds_dwordx4 (no VGPR staging):
  // wave w, lane l moves vector i*256 + 64w + l, so each wave fills a
  // contiguous KiB of the buffer.
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
  int R[kAT], best[kAT];

  // Stages [st0, st1) of one region.  PAIR: the fold takes max |score| (the
  // antipode of each representative scores exactly its negation), and NN-B
  // tracks the first and last group at the best bucket (pair_key).
  // Software pipeline: the MFMA result of tile k for atom tile `at` is folded
  // into the group maximum while tile k+1's MFMAs issue, and tile k+1's A
  // operand is read from LDS right after tile k's first MFMA.  A group of kG
  // tiles is compared against the threshold once its last tile has been
  // folded, i.e. during the next group's first tile (NN-B: the next group's
  // tile at % 8); the region's last tile is folded after its loop.
  auto run = [&](auto pair_tag, int st0, int st1) {
    constexpr bool PAIR = decltype(pair_tag)::value;
    const int g_base = (t0 + st0 * kST) / kG;  // global group of the region's first group in this slice
#pragma unroll
    for (int at = 0; at < kAT; ++at) {
      R[at] = PAIR && MODE == kModeB ? static_cast<int>(kPairInit) : initial_threshold<MODE>();
      best[at] = -1;
    }
    int gm[kAT];
    f32x4 acc[kAT], part[kAT];
#pragma unroll
    for (int at = 0; at < kAT; ++at) {
      gm[at] = INT_MIN;
      acc[at] = f32x4{-0.f, -0.f, -0.f, -0.f};  // INT_MIN bit patterns: neutral for the fold
    }
    int group_prev = -1;  // global id of the group whose compare is pending
    for (int st = st0; st < st1; ++st) {
      const int buf = st & 1;
      if (st + 1 < n_stages) stage_copy(st + 1, buf ^ 1);
      const uint8_t *L = lds[buf] + a_off;
      bf16x8 a = *reinterpret_cast<const bf16x8 *>(L);
      bool up[kAT];
      int gdone[kAT];
      // One group of kG tiles: tile 0 closes the previous group, tile 1 starts
      // this group's maximum.
      auto group_tiles = [&](int k0) {
#pragma unroll
        for (int t = 0; t < kG; ++t) {
          const int k = k0 + t;
          bf16x8 an;
#pragma unroll
          for (int at = 0; at < kAT; ++at) {
            const f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[0][at], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            if (at == 0) {
              // the LDS wait that guards `a` must not also wait for this read
              __builtin_amdgcn_sched_barrier(0);
              an = *reinterpret_cast<const bf16x8 *>(L + (k + 1 < kST ? k + 1 : k) * kTileBytes);
            }
            int m;
            if constexpr (PAIR) {
              // v_max3_f32 with |.| source modifiers: the same two VALU ops
              float mf;
              if (t == 1) {
                mf = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(acc[at][0]), __builtin_fabsf(acc[at][1])),
                                     __builtin_fabsf(acc[at][2]));
                mf = __builtin_fmaxf(mf, __builtin_fabsf(acc[at][3]));
              } else {
                mf = __builtin_fmaxf(__builtin_fmaxf(__int_as_float(gm[at]), __builtin_fabsf(acc[at][0])),
                                     __builtin_fabsf(acc[at][1]));
                mf = __builtin_fmaxf(__builtin_fmaxf(mf, __builtin_fabsf(acc[at][2])), __builtin_fabsf(acc[at][3]));
              }
              m = __float_as_int(mf);
            } else {
              if (t == 1) {
                m = max(max(__float_as_int(acc[at][0]), __float_as_int(acc[at][1])), __float_as_int(acc[at][2]));
                m = max(m, __float_as_int(acc[at][3]));
              } else {
                m = max(max(gm[at], __float_as_int(acc[at][0])), __float_as_int(acc[at][1]));
                m = max(max(m, __float_as_int(acc[at][2])), __float_as_int(acc[at][3]));
              }
            }
            // The empty asm pins the fold next to this MFMA (IR passes would
            // otherwise sink the chain to the group end) and the sched_barrier
            // stops the machine scheduler from hoisting every MFMA, so the
            // matrix pipe and the VALU work in parallel.
            asm volatile("" : "+v"(m));
            if (t == 0) {
              gdone[at] = m;
              if constexpr (MODE != kModeB) up[at] = m > R[at];
            }
            // NN-B: the closed group's key enters R in tile at % 8 of the next
            // group, one atom tile per code tile, so the key's VALU work is
            // spread evenly under the MFMAs instead of piling up in tile 0.
            if (MODE == kModeB && at % 8 == t) {
              if constexpr (PAIR)
                R[at] = static_cast<int>(pair_key(static_cast<uint32_t>(R[at]), gdone[at], group_prev - g_base));
              else
                R[at] = max(R[at], group_key(gdone[at], group_prev));
            }
            gm[at] = m;
            if constexpr (NS == 1)
              acc[at] = c;
            else
              part[at] = c;
            __builtin_amdgcn_sched_barrier(0);
          }
          if constexpr (NS == 3) {
#pragma unroll
            for (int at = 0; at < kAT; ++at)
              part[at] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[1][at], part[at], 0, 0, 0);
#pragma unroll
            for (int at = 0; at < kAT; ++at)
              acc[at] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[2][at], part[at], 0, 0, 0);
          }
          a = an;
        }
      };
#pragma unroll 1
      for (int k0 = 0; k0 < kST; k0 += kG) {
        group_tiles(k0);
        if constexpr (MODE != kModeB) {
#pragma unroll
          for (int at = 0; at < kAT; ++at) {
            if (up[at]) {
              R[at] = raised_threshold<MODE>(gdone[at]);
              best[at] = group_prev;
            }
          }
        }
        group_prev = (t0 + st * kST + k0) / kG;
      }
      __syncthreads();
    }
    // fold the region's last tile and close its last group
#pragma unroll
    for (int at = 0; at < kAT; ++at) {
      int m;
      if constexpr (PAIR) {
        float mf = __builtin_fmaxf(__builtin_fmaxf(__int_as_float(gm[at]), __builtin_fabsf(acc[at][0])),
                                   __builtin_fabsf(acc[at][1]));
        mf = __builtin_fmaxf(__builtin_fmaxf(mf, __builtin_fabsf(acc[at][2])), __builtin_fabsf(acc[at][3]));
        m = __float_as_int(mf);
      } else {
        m = max(max(gm[at], __float_as_int(acc[at][0])), __float_as_int(acc[at][1]));
        m = max(max(m, __float_as_int(acc[at][2])), __float_as_int(acc[at][3]));
      }
      if constexpr (MODE == kModeB) {
        if constexpr (PAIR)
          R[at] = static_cast<int>(pair_key(static_cast<uint32_t>(R[at]), m, group_prev - g_base));
        else
          R[at] = max(R[at], group_key(m, group_prev));
      } else if (m > R[at]) {
        R[at] = raised_threshold<MODE>(m);
        best[at] = group_prev;
      }
    }

    // ---- merge this region of the slice into the atom's keys ----
    // The four lanes of atom j (j, j+16, j+32, j+48) hold the slice's best per
    // lane; their maximum is the slice's best (score, group) and the mask
    // names the lanes that reached it there.  A lane without a hit merges 0 (a
    // select, not a branch: a conditional atomic here costs the main loop
    // ~20 VGPRs).
#pragma unroll
    for (int at = 0; at < kAT; ++at) {
      const int64_t a = wave_atom0 + at * 16 + j;
      const bool mine = q == 0 && a < n_atoms;
      if constexpr (MODE == kModeB && !PAIR) {
        int Rm = R[at];
        Rm = max(Rm, __shfl_xor(Rm, 16, 64));
        Rm = max(Rm, __shfl_xor(Rm, 32, 64));
        const uint32_t mask = atom_lanes(__ballot(R[at] == Rm), j);
        const uint32_t g = 0xFFFFu - (static_cast<uint32_t>(Rm) & 0xFFFFu);
        const uint32_t key = Rm != initial_threshold<MODE>()
                                 ? (static_cast<uint32_t>(Rm) & 0xFFFF0000u) | ((0x3FFu - g) << 6) | (mask << 2)
                                 : 0u;
        if (mine) atomicMax(&keys[a].x, key);
      } else if constexpr (MODE == kModeB) {
        // This slice's record: the best bucket Bm over the atom's lanes; among
        // the lanes at Bm, the earliest first group F and the latest last
        // group L (pair-region indices), the lanes with a hit in F and in L,
        // and `many` when some group at Bm is neither F nor L.
        const uint32_t r = static_cast<uint32_t>(R[at]);
        const bool hit = r >= 0x80000000u;  // bucket >= 0x4000
        const uint32_t bkt = hit ? r >> 17 : 0u;
        uint32_t bm = max(bkt, static_cast<uint32_t>(__shfl_xor(static_cast<int>(bkt), 16, 64)));
        bm = max(bm, static_cast<uint32_t>(__shfl_xor(static_cast<int>(bm), 32, 64)));
        const bool at_m = hit && bkt == bm;
        const uint32_t fl = 255u - ((r >> 8) & 0xFFu), ll = r & 0xFFu;
        uint32_t F = at_m ? fl : 255u, Lg = at_m ? ll : 0u;
        F = min(F, static_cast<uint32_t>(__shfl_xor(static_cast<int>(F), 16, 64)));
        F = min(F, static_cast<uint32_t>(__shfl_xor(static_cast<int>(F), 32, 64)));
        Lg = max(Lg, static_cast<uint32_t>(__shfl_xor(static_cast<int>(Lg), 16, 64)));
        Lg = max(Lg, static_cast<uint32_t>(__shfl_xor(static_cast<int>(Lg), 32, 64)));
        const uint32_t mf = atom_lanes(__ballot(at_m && (fl == F || ll == F)), j);
        const uint32_t ml = atom_lanes(__ballot(at_m && (fl == Lg || ll == Lg)), j);
        const bool odd = at_m && (((r >> 16) & 1u) != 0u || (fl != F && fl != Lg) || (ll != F && ll != Lg));
        const uint32_t many = atom_lanes(__ballot(odd), j) != 0u ? 1u : 0u;
        const uint64_t pb = static_cast<uint64_t>(g_base - kType3Tiles / kG);
        const uint64_t rec = bm != 0u ? (static_cast<uint64_t>(bm) << 48) | (static_cast<uint64_t>(many) << 40) |
                                            ((pb + F) << 32) | ((pb + Lg) << 24) | (mf << 4) | ml
                                      : 0ull;
        if (mine) recs[static_cast<int64_t>(slice - s0) * n_atoms + a] = rec;
      } else {
        // (score, 1023 - group) as one 64-bit value (pair groups counted from
        // the pair region's start), lanes that never beat the threshold 0
        const bool hit = best[at] >= 0;
        const uint32_t g = static_cast<uint32_t>(best[at] - (PAIR ? kType3Tiles / kG : 0));
        const uint64_t v = hit ? (static_cast<uint64_t>(static_cast<uint32_t>(R[at])) << 32) |
                                     (static_cast<uint64_t>(0x3FFu - g) << 4)
                               : 0ull;
        uint64_t vm = v;
        uint64_t o = static_cast<uint64_t>(__shfl_xor(static_cast<long long>(vm), 16, 64));
        vm = o > vm ? o : vm;
        o = static_cast<uint64_t>(__shfl_xor(static_cast<long long>(vm), 32, 64));
        vm = o > vm ? o : vm;
        const uint64_t mask = atom_lanes(__ballot(v == vm), j);
        const uint64_t key = vm != 0ull ? vm | mask : 0ull;
        if (mine)
          atomicMax(reinterpret_cast<unsigned long long *>(&keys[a]) + (PAIR ? 1 : 0),
                    static_cast<unsigned long long>(key));
      }
    }
  };
  if (n_t > 0) run(std::integral_constant<bool, false>{}, 0, n_t);
  if (n_t < n_stages) run(std::integral_constant<bool, true>{}, n_t, n_stages);
}

// Structured type-3 scoring (NN-B; replaces the sweep's 6,144 type-3 tiles).
//
// A type-3 code (w, p) is the sign pattern P(w) of a Golay word w (-s where
// w has a 1, +s elsewhere) with coordinate p replaced by -3s, so with the
// bf16 values s = 0.353515625 and 3s = 1.0625 its score is
//   score(w, p) = S(w) - x_p (1.0625 + s P_p(w)),   S(w) = s P(w).x,
// i.e. S(w) - x_p * (alpha = 1.416015625 where w_p = 0, beta = 0.708984375
// where w_p = 1); both products are exact in fp32 (8 x 8 significant bits).
// The best code of a word is S(w) + bonus(w) with bonus(w) = max_p of
// -x_p (alpha or beta).  With p1, p2 the positions of the two largest terms
// t_p = max(-alpha x_p, -beta x_p) and m3 the largest elsewhere, bonus(w) <=
// e(b1, b2) = max(c1(b1), c2(b2), m3) for the word's bits b1, b2 at p1, p2
// (c(0) = -alpha x, c(1) = -beta x there), and the least additive bound
// eb + k1 P_p1(w) + k2 P_p2(w) >= e(b1, b2) is solved per atom.  The MFMA's
// B operand is the atom with x_p1, x_p2 raised by k1 / s, k2 / s, so it gives
// T(w) = S(w) + k1 P_p1(w) + k2 P_p2(w), and S(w) + e(w) <= T(w) + eb: a test
// on T bounds each word by its own bits at p1, p2 (about 8x fewer candidates
// than one bound max_p t_p for all words).  The Golay code holds the
// complement of every word, S(~w) = -S(w) and T(~w) = -T(w), so one MFMA per
// 16 representative words tests 32 words: 128 tiles instead of 6,144.
// p1, p2, the raised coordinates, m3, eb and the margin come per atom from
// t12_kernel (T3Setup), which ran first.
// A block of 4 waves holds AT atom tiles of 16 atoms per wave as MFMA B
// operands and streams the 128 pattern tiles through LDS once (a second time
// only if a survivor list overflows):
//   pass 1  every lane whose four outputs hold a word that could reach the
//           lowest bucket still possible -- the pair key of t12_kernel (the
//           best pair bucket, or a type-3 code's bucket above it), 2.0 (the
//           origin rule) and the best type-3
//           bucket found so far, whichever is highest: |T| >= lo(bucket) -
//           eb - margin -- appends one 4-byte entry (atom, tile, lane
//           quarter, 4-bit mask of its outputs) to the wave's list in LDS;
//           when the list is nearly full and at the end of the pass the wave
//           evaluates it, one flagged word per lane per round (an entry with
//           work left goes back on the list): each flagged representative gets S recomputed from the atom's
//           bf16 coordinates, and it and its complement, each when its S +
//           e(w) reaches the floor, get their 24 positions scored,
//           the best bucket M3 per atom is kept by an LDS atomic max, words
//           at or above the running best go onto a survivor list, and the
//           thresholds rise to the new best buckets;
//   rows    every word at the final M3 was at or above the running best when
//           it was evaluated, so the survivors give every (w, p) at bucket M3
//           and its codebook row (t3_rows); the lowest is kept by an LDS
//           atomic min;
//   pass 2  (only after a survivor list lost entries) the rows of the atoms
//           whose entries were lost, from a second sweep with their
//           thresholds at M3 (the other atoms' thresholds: +inf).
// The atom's key gets (M3 << 16, lowest row at M3), or 0 when no type-3 code
// reaches 2.0; pick_kernel compares it with the pair key.  (An atom with a NaN
// or infinite coordinate carries t12_kernel's marker pair key, whose NaN
// threshold leaves it no candidates here.)
// Buckets are taken by round-half-up like the dense sweep's, and every score
// is an fp32 sum of exact products plus one rounding for the bonus, so the
// answer equals the exact-score answer off near-ties (oracle/nn.py).
constexpr int kT3ST = 16;                          // pattern tiles per LDS stage (8: 3.47 -> 3.39 ms)
constexpr int kT3Stages = kT3Tiles / kT3ST;        // 8 per pass
constexpr int kT3StageBytes = kT3ST * kTileBytes;  // 12,288
constexpr int kT3StageVecs = kT3StageBytes / 16;   // 768
constexpr int kT3Cap = 200;                        // candidate entries per wave (4 bytes each)
constexpr int kT3Surv = 384;                       // survivor words per wave (4 bytes each)
constexpr float kT3Alpha = 1.416015625f;           // bf16(3s) + bf16(s)
constexpr float kT3Beta = 0.708984375f;            // bf16(3s) - bf16(s)
constexpr float kT3S = 0.353515625f;               // bf16(s)
static_assert(kT3StageVecs % 64 == 0, "type-3 stage splits into whole wave loads");
static_assert(kT3Tiles % kT3ST == 0, "whole type-3 stages");

__device__ __forceinline__ uint32_t t3_bucket(float v) { return (__float_as_uint(v) + 0x8000u) >> 16; }

// S of representative word wb: sum over the 24 coordinates of (-s where wb has a 1, else +s) * x,
// in coordinate order (exact products, fp32 sums); xr: the atom's 12 words of bf16 pairs.
__device__ __forceinline__ float t3_dot(const uint32_t *xr, uint32_t wb) {
  float S = 0.f;
#pragma unroll
  for (int d = 0; d < 12; ++d) {
    const uint32_t xx = xr[d];
    const float x0 = __uint_as_float((xx << 16) ^ ((wb >> (2 * d)) & 1u) << 31);
    const float x1 = __uint_as_float((xx & 0xFFFF0000u) ^ ((wb >> (2 * d + 1)) & 1u) << 31);
    S = fmaf(x0, kT3S, S);
    S = fmaf(x1, kT3S, S);
  }
  return S;
}

// t3_kernel's per-atom set-up, made by t12_kernel (one lane per atom: 64 atoms per wave instruction
// instead of t3_kernel's 16) and handed over as a 16-byte record.  Position terms t_p = max(-alpha x_p,
// -beta x_p): the two largest at p1, p2 (ties: the lower position first), x there (x1, x2), the third
// largest m3.  A word w with bits b1, b2 at p1, p2 has bonus(w) <= e(b1, b2) = max(c1(b1), c2(b2), m3),
// c(0) = -alpha x, c(1) = -beta x there.  The additive bound eb + k1 P1(w) + k2 P2(w) >= e(b1, b2)
// (P = +1 for bit 0) with the least eb: eb = max((e00 + e11) / 2, (e01 + e10) / 2), k1 + k2 = (e00 -
// e11) / 2, k1 - k2 = (e01 - e10) / 2.  The MFMA with x_p1, x_p2 raised by k1 / s, k2 / s (rounded to
// bf16: h1, h2) gives T(w) = S(w) + k1 P1(w) + k2 P2(w) (and T(~w) = -T(w)), so |T| >= lo(floor) - eb -
// dl - mg flags every word whose S(w) + e(w) reaches the floor; dl: what the bf16 rounding of the raised
// coordinates adds; mg = (s sum |x| + |t_p1|) 2^-14: the MFMA's fp32 summation order of T and the score
// roundings.  Record: ra = (h1 | h2 << 16, p1 | p2 << 8 | mg's bf16 bits rounded up << 16) in the type-3
// half of the atom's key (t3_kernel reads it, then writes its result there), rb = (m3, eb + dl).
// add() takes the coordinates in ascending order, record() gives the record.
struct T3Setup {
  float m1 = -__builtin_inff(), m2 = -__builtin_inff(), m3 = -__builtin_inff(), x1 = 0.f, x2 = 0.f, ax = 0.f;
  uint32_t p1 = 0u, p2 = 1u;
  // coordinate i (ascending) of the atom
  __device__ __forceinline__ void add(float x, uint32_t i) {
    const float t = fmaxf(-x * kT3Alpha, -x * kT3Beta);
    const bool a1 = t > m1, a2 = t > m2;
    m3 = a2 ? m2 : fmaxf(m3, t);
    m2 = a1 ? m1 : (a2 ? t : m2);
    x2 = a1 ? x1 : (a2 ? x : x2);
    p2 = a1 ? p1 : (a2 ? i : p2);
    m1 = a1 ? t : m1;
    x1 = a1 ? x : x1;
    p1 = a1 ? i : p1;
    ax += fabsf(x);
  }
  __device__ __forceinline__ void record(uint2 &ra, uint2 &rb) const {
    const float a1 = -x1 * kT3Alpha, b1 = -x1 * kT3Beta, a2 = -x2 * kT3Alpha, b2 = -x2 * kT3Beta;
    const float e00 = fmaxf(fmaxf(a1, a2), m3), e11 = fmaxf(fmaxf(b1, b2), m3);
    const float e01 = fmaxf(fmaxf(a1, b2), m3), e10 = fmaxf(fmaxf(b1, a2), m3);
    const float ebar = fmaxf((e00 + e11) * 0.5f, (e01 + e10) * 0.5f);
    const float sgm = (e00 - e11) * 0.5f, dlt = (e01 - e10) * 0.5f;
    const float k1 = (sgm + dlt) * 0.5f, k2 = (sgm - dlt) * 0.5f;
    const uint32_t h1 = bf16_rne_bits(x1 + k1 / kT3S), h2 = bf16_rne_bits(x2 + k2 / kT3S);
    const float dl =
        fabsf((bf16_bits_to_float(h1) - x1) * kT3S - k1) + fabsf((bf16_bits_to_float(h2) - x2) * kT3S - k2);
    const float mg = (ax * kT3S + fabsf(m1)) * 0x1p-14f;
    const uint32_t mgb = (__float_as_uint(mg) + 0xFFFFu) >> 16;  // (mg >= 0: rounded up)
    ra = make_uint2(h1 | h2 << 16, p1 | p2 << 8 | mgb << 16);
    rb = make_uint2(__float_as_uint(m3), __float_as_uint(ebar + dl));
  }
};

template <int AT>
__global__ __launch_bounds__(kThreads, 4) void t3_kernel(const uint4 *__restrict__ xb, int64_t n_atoms,
                                                         const uint8_t *__restrict__ t3_tiles,
                                                         const uint32_t *__restrict__ t3_words,
                                                         const uint32_t *__restrict__ t3_rows,
                                                         uint4 *__restrict__ keys, const uint2 *__restrict__ rec,
                                                         int rows_by_sweep) {
  constexpr int NA = AT * 16;  // atoms per wave
  static_assert(NA <= 128, "entry layout: 7 bits of atom");
  __shared__ __align__(16) uint8_t stg[2][kT3StageBytes];
  __shared__ uint32_t cand[kWaves][kT3Cap];  // atom | tile << 7 | quarter << 14 | output mask << 16 | done << 20
  __shared__ uint32_t surv[kWaves][kT3Surv];  // atom | pattern id << 7: words at or above the atom's running best
  __shared__ uint32_t st_x[kWaves][NA];  // x at p1 | x at p2 << 16 (bf16 bits)
  __shared__ uint32_t st_m[kWaves][NA], st_r[kWaves][NA];
  __shared__ float st_t[kWaves][NA];    // lo(floor) less twice the margin: which signs of a word to evaluate
  __shared__ float st_m3[kWaves][NA];   // the third largest position term (the largest off p1, p2)
  __shared__ float st_mg[kWaves][NA];   // the atom's margin for summation orders
  __shared__ uint8_t st_p[kWaves][NA][2];  // p1, p2: the positions of the two largest position terms
  __shared__ uint32_t surv_n[kWaves];
  __shared__ uint32_t st_ovf[kWaves][2];   // atoms (bits) whose survivor list lost an entry: rows by pass 2

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, q = lane >> 4, j = lane & 15;
  const int64_t wave_atom0 = static_cast<int64_t>(blockIdx.x) * (kWaves * NA) + static_cast<int64_t>(wave) * NA;

  if (lane < 2) st_ovf[wave][lane] = 0u;
  if (lane == 0) surv_n[wave] = 0u;
  bf16x8 b[AT];
  float offs[AT];  // eb, the raised coordinate's rounding and the margin: thr = lo(floor) - offs
#pragma unroll
  for (int at = 0; at < AT; ++at) {
    const int64_t a = wave_atom0 + at * 16 + j;
    uint4 w = make_uint4(0u, 0u, 0u, 0u);
    if (a < n_atoms && q < 3) w = xb[a * 3 + q];
    // The atom's set-up record from t12_kernel (T3Setup: positions p1, p2 of the two largest
    // position terms, their raised bf16 coordinates, the third largest term m3, eb + dl and the margin);
    // an atom past the end: the record of a zero atom (p1 = 0, p2 = 1, the rest 0)
    uint2 ra = make_uint2(0u, 1u << 8), rb = make_uint2(0u, 0u);
    if (a < n_atoms) {
      ra = reinterpret_cast<const uint2 *>(&keys[a])[0];
      rb = rec[a];
    }
    const uint32_t p1 = min(ra.y & 31u, 23u), p2 = min((ra.y >> 8) & 31u, 23u);
    uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t pr = r ? p2 : p1, h = r ? ra.x >> 16 : ra.x & 0xFFFFu;
      if (q < 3 && (pr >> 3) == static_cast<uint32_t>(q)) {
        const uint32_t e = pr & 7u;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (static_cast<uint32_t>(k) == (e >> 1)) {
            reinterpret_cast<uint16_t *>(&st_x[wave][at * 16 + j])[r] =
                static_cast<uint16_t>((e & 1u) ? ww[k] >> 16 : ww[k] & 0xFFFFu);
            ww[k] = (e & 1u) ? (ww[k] & 0xFFFFu) | (h << 16) : (ww[k] & 0xFFFF0000u) | h;
          }
      }
    }
    b[at] = __builtin_bit_cast(bf16x8, make_uint4(ww[0], ww[1], ww[2], ww[3]));
    const float mg = __uint_as_float(ra.y & 0xFFFF0000u);
    offs[at] = __uint_as_float(rb.y) + mg;
    if (q == 0) {
      st_m3[wave][at * 16 + j] = __uint_as_float(rb.x);
      st_mg[wave][at * 16 + j] = mg;
      st_p[wave][at * 16 + j][0] = static_cast<uint8_t>(p1);
      st_p[wave][at * 16 + j][1] = static_cast<uint8_t>(p2);
    }
  }
  // the best pair bucket of each atom (the pair key of t12_kernel, which ran first): the type-3 best starts
  // there, so no word below it becomes a survivor (an atom whose type-3 codes all stay below it keeps no
  // row and gets key 0)
  uint32_t mp[AT];
#pragma unroll
  for (int at = 0; at < AT; ++at) {
    const int64_t a = wave_atom0 + at * 16 + j;
    uint32_t m = 0u;
    if (q == 0 && a < n_atoms) m = keys[a].z >> 16;
    if (q == 0) {
      st_m[wave][at * 16 + j] = m;
      st_r[wave][at * 16 + j] = 0xFFFFFFFFu;
    }
    mp[at] = static_cast<uint32_t>(__shfl(static_cast<int>(m), j, 64));
  }

  const uint4 *gsrc = reinterpret_cast<const uint4 *>(t3_tiles);
  auto stage_copy = [&](int g, int dst) {
    const int stage = g % kT3Stages;
#pragma unroll
    for (int i = 0; i < (kT3StageVecs + kThreads - 1) / kThreads; ++i) {
      if (i * kThreads + wave * 64 >= kT3StageVecs) break;  // (wave-uniform)
      int off = i * kThreads + tid;
      asm volatile("" : "+v"(off));  // (computed here: a per-thread pointer kept across the loop spills)
      const uint4 *src = gsrc + static_cast<size_t>(stage) * kT3StageVecs + off;
      uint8_t *d = stg[dst] + (i * kThreads + wave * 64) * 16;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(src),
                                       (__attribute__((address_space(3))) void *)(d), 16, 0, 0);
    }
  };

  // The scores of word wr (sg: its complement) of atom al at its 24 positions, through f(p, t).
  auto word_scores = [&](const uint32_t *xr, uint32_t wr, int sg, float D, auto f) {
    const uint32_t wb = sg ? wr ^ 0xFFFFFFu : wr;
    const float S = sg ? -D : D;
#pragma unroll
    for (int d = 0; d < 12; ++d) {
      const uint32_t xx = xr[d];
      f(2 * d, fmaf(-__uint_as_float(xx << 16), ((wb >> (2 * d)) & 1u) ? kT3Beta : kT3Alpha, S));
      f(2 * d + 1, fmaf(-__uint_as_float(xx & 0xFFFF0000u), ((wb >> (2 * d + 1)) & 1u) ? kT3Beta : kT3Alpha, S));
    }
  };

  int cnt = 0;  // entries in this wave's candidate list (wave-uniform)
  // One flagged word and sign per lane per round: the list is worked as a stack and an entry with work left
  // goes back on it, so every lane is busy while 64 or more words are listed.
  // pass 1: the best bucket of each word -> st_m (atomic max), and the word onto the survivor list when it
  //         is at or above the atom's running best; pass 2: the lowest row at the atom's st_m -> st_r.
  bool flushed = false;  // (wave-uniform) a flush ran since the thresholds were last set
  auto flush = [&](int pass) {
    flushed |= cnt > 0;
    while (cnt > 0) {  // (wave-uniform)
      const int n = min(cnt, 64);
      cnt -= n;
      const bool act = lane < n;
      const uint32_t ce = act ? cand[wave][cnt + lane] : 0u;
      const uint32_t mask = (ce >> 16) & 0xFu;
      uint32_t back = 0u;  // the entry as it goes back on the list (0: done)
      if (act && mask != 0u) {  // (every appended entry has an output bit; the test keeps rep in the table)
        const int al = static_cast<int>(ce & 0x7Fu);
        const uint32_t rep = ((ce >> 7) & 0x7Fu) * kTileCodes + 4 * ((ce >> 14) & 3u) +
                             static_cast<uint32_t>(__builtin_ctz(mask));
        // (the atom's coordinates from its bf16 planes in global memory; an entry's atom is in range)
        const uint32_t *xr = reinterpret_cast<const uint32_t *>(xb + min(wave_atom0 + al, n_atoms - 1) * 3);
        const float tlo = st_t[wave][al];
        // the bound on the bonus of a word by its bits at p1, p2 (as at set-up)
        const uint32_t pa = st_p[wave][al][0], pb = st_p[wave][al][1];
        const float m3v = st_m3[wave][al];
        const uint32_t xab = st_x[wave][al];
        const float xa1 = __uint_as_float(xab << 16);
        const float xa2 = __uint_as_float(xab & 0xFFFF0000u);
        const uint32_t wr = t3_words[rep];
        const float D = t3_dot(xr, wr);
        const uint32_t ba = (wr >> pa) & 1u, bb = (wr >> pb) & 1u;
        // the representative (S = D) and its complement (S = -D, the other bits at p1, p2), each when its
        // S + e(word) can reach the floor; one of them per round (bit 20: the representative is done)
        const float ew0 = fmaxf(fmaxf(-xa1 * (ba ? kT3Beta : kT3Alpha), -xa2 * (bb ? kT3Beta : kT3Alpha)), m3v);
        const float ew1 = fmaxf(fmaxf(-xa1 * (ba ? kT3Alpha : kT3Beta), -xa2 * (bb ? kT3Alpha : kT3Beta)), m3v);
        const bool q0 = ((ce >> 20) & 1u) == 0u && D + ew0 >= tlo, q1 = -D + ew1 >= tlo;
        const uint32_t rest = mask & (mask - 1u);
        back = q0 && q1 ? ce | 1u << 20 : rest != 0u ? (ce & ~0x1F0000u) | rest << 16 : 0u;
        if (q0 || q1) {
          const int sg = q0 ? 0 : 1;
          const uint32_t wid = rep + (sg ? static_cast<uint32_t>(kT3Reps) : 0u);
          if (pass == 1) {
            float best = -__builtin_inff();
            word_scores(xr, wr, sg, D, [&](int, float t) { best = fmaxf(best, t); });
            const uint32_t bk = best > 0.f ? t3_bucket(best) : 0u;
            if (bk >= 0x4000u) {
              const uint32_t old = atomicMax(&st_m[wave][al], bk);
              if (bk >= old) {
                const uint32_t slot = atomicAdd(&surv_n[wave], 1u);
                if (slot < static_cast<uint32_t>(kT3Surv))
                  surv[wave][slot] = static_cast<uint32_t>(al) | wid << 7;
                else
                  atomicOr(&st_ovf[wave][al >> 5], 1u << (al & 31));
              }
            }
          } else {
            const uint32_t M = st_m[wave][al];
            uint32_t rmin = 0xFFFFFFFFu;
            word_scores(xr, wr, sg, D, [&](int p, float t) {
              if (t > 0.f && t3_bucket(t) == M) rmin = min(rmin, t3_rows[wid * kDim + p]);
            });
            if (rmin != 0xFFFFFFFFu) atomicMin(&st_r[wave][al], rmin);
          }
        }
      }
      // the entries with work left go back on the list (every lane read its entry above)
      const uint64_t bm = __ballot(back != 0u);
      if (back != 0u)
        cand[wave][cnt + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bm >> 32),
                                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bm), 0u))] = back;
      cnt += __popcll(bm);
    }
  };

  // The threshold on |T|: a word can reach bucket B only if S + e(w) >= lo(B) - margin, i.e.
  // T >= lo(B) - eb - margin, and no bucket below the lowest that can still win counts: the best pair
  // bucket (the pair key), 2.0 (the origin rule), and -- raised at every stage end -- the best type-3
  // bucket found so far.
  float thr[AT];
  auto set_thr = [&](int at, uint32_t mlow) {
    mlow = max(mlow, max(mp[at], 0x4000u));
    const float lo = __uint_as_float((mlow << 16) - 0x8000u);
    thr[at] = lo - offs[at];
    if (q == 0) st_t[wave][at * 16 + j] = lo - 2.f * st_mg[wave][at * 16 + j];
  };
#pragma unroll
  for (int at = 0; at < AT; ++at) set_thr(at, 0u);

  const int a_off = (q < 3 ? q : 0) * 256 + j * 16;
  const uint32_t ebase = static_cast<uint32_t>(j) | static_cast<uint32_t>(q) << 14;  // the lane's entry bits
  stage_copy(0, 0);
  __syncthreads();
  // pass 1 (the candidates); pass 2 only when some wave's survivor list overflowed
  int g_end = kT3Stages;
  for (int g = 0; g < g_end; ++g) {
    const int pass = 1 + g / kT3Stages, buf = g & 1;
    if (g + 1 < g_end) stage_copy(g + 1, buf ^ 1);  // (pass 2's first stage: after the decision below)
    if (g == kT3Stages) {
      // pass 2 (a survivor list lost entries): thresholds at the final best buckets of the atoms concerned
#pragma unroll
      for (int at = 0; at < AT; ++at) {
        const int al = at * 16 + j;
        const bool redo = rows_by_sweep != 0 || ((st_ovf[wave][al >> 5] >> (al & 31)) & 1u) != 0u;
        const uint32_t M = st_m[wave][al];
        const float lo = redo && M >= 0x4000u ? __uint_as_float((M << 16) - 0x8000u) : __builtin_inff();
        thr[at] = lo - offs[at];
        if (q == 0) st_t[wave][at * 16 + j] = lo - 2.f * st_mg[wave][at * 16 + j];
      }
    }
    const uint8_t *L = stg[buf] + a_off;
    const int tile0 = (g % kT3Stages) * kT3ST;
    // (unrolled by 8: the A tiles' LDS offsets and the entries' tile bits become constants; 3.83 -> 3.75
    // ms with 8-tile stages)
#pragma unroll 8
    for (int k = 0; k < kT3ST; ++k) {
      const bf16x8 a = *reinterpret_cast<const bf16x8 *>(L + k * kTileBytes);
      f32x4 c[AT];
#pragma unroll
      for (int at = 0; at < AT; ++at)
        c[at] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[at], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
      for (int at = 0; at < AT; ++at) {
        // each output's |T| against the atom's threshold (a word and its complement: one test): the
        // largest of the four against it, one compare and one wave mask; the four compares only on a hit
        // (IEEE maximum, v_maximum3_f32: a NaN output, only a non-finite atom's, makes the step a miss)
        const float mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(fabsf(c[at][0]), fabsf(c[at][1])),
                                                       __builtin_elementwise_maximum(fabsf(c[at][2]), fabsf(c[at][3])));
        const bool hit = mx >= thr[at];
        const uint64_t msk = __ballot(hit);
        if (msk == 0ull) continue;
        if (cnt > kT3Cap - 64) flush(pass);
        if (hit) {
          const bool h0 = fabsf(c[at][0]) >= thr[at], h1 = fabsf(c[at][1]) >= thr[at];
          const bool h2 = fabsf(c[at][2]) >= thr[at], h3 = fabsf(c[at][3]) >= thr[at];
          const uint32_t mask = (h0 ? 1u : 0u) | (h1 ? 2u : 0u) | (h2 ? 4u : 0u) | (h3 ? 8u : 0u);
          const uint32_t pos = static_cast<uint32_t>(cnt) +
                               __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(msk >> 32),
                                                         __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(msk), 0u));
          cand[wave][pos] = (ebase + static_cast<uint32_t>(at * 16)) | static_cast<uint32_t>(tile0 + k) << 7 | mask << 16;
        }
        cnt += __popcll(msk);
      }
    }
    // the list is evaluated when it is nearly full (in the tile loop) and at the end of each pass: the
    // floor from the pair key leaves little for rising thresholds to gain, and fuller rounds keep the
    // lanes busy and the block's waves in step at the barriers (4.93 -> 4.64 ms against a flush at
    // every stage end holding 64 entries, config 4)
    if (g == kT3Stages - 1 || g == 2 * kT3Stages - 1) flush(pass);
    if (pass == 1 && flushed) {
      // the thresholds rise with the best buckets found so far (this wave's own atoms: no barrier needed);
      // the buckets change only in a flush
      flushed = false;
#pragma unroll
      for (int at = 0; at < AT; ++at) set_thr(at, st_m[wave][at * 16 + j]);
    }
    if (g == kT3Stages - 1) {
      // pass 1 done: pass 2 only if a survivor list lost entries (all waves agree), for those atoms
      // (rows_by_sweep: pass 2 for every atom -- the path an overflow takes, for its tests)
      if (__syncthreads_or(rows_by_sweep != 0 || (st_ovf[wave][0] | st_ovf[wave][1]) != 0u)) {
        g_end = 2 * kT3Stages;
        stage_copy(g + 1, buf ^ 1);  // buffer buf ^ 1 was last read in stage g - 1, before the barrier
        __syncthreads();
      }
    } else {
      __syncthreads();
    }
  }
  {
    // the lowest row at each atom's best bucket, from its survivors (every word that reached the final
    // best bucket was at or above the running best when it was evaluated); pass 2 gave the others'
    const int ns = static_cast<int>(min(surv_n[wave], static_cast<uint32_t>(kT3Surv)));
    for (int i = lane; i < ns; i += 64) {
      const uint32_t se = surv[wave][i];
      const int al = static_cast<int>(se & 0x7Fu);
      if (rows_by_sweep != 0 || ((st_ovf[wave][al >> 5] >> (al & 31)) & 1u) != 0u) continue;
      const uint32_t wid = se >> 7;
      const uint32_t M = st_m[wave][al];
      const uint32_t *xr = reinterpret_cast<const uint32_t *>(xb + min(wave_atom0 + al, n_atoms - 1) * 3);
      const uint32_t wr = t3_words[wid & (kT3Reps - 1)];
      const int sg = wid >= static_cast<uint32_t>(kT3Reps) ? 1 : 0;
      const float D = t3_dot(xr, wr);
      uint32_t rmin = 0xFFFFFFFFu;
      word_scores(xr, wr, sg, D, [&](int p, float t) {
        if (t > 0.f && t3_bucket(t) == M) rmin = min(rmin, t3_rows[wid * kDim + p]);
      });
      if (rmin != 0xFFFFFFFFu) atomicMin(&st_r[wave][al], rmin);
    }
  }
  __syncthreads();
  if (q == 0) {
#pragma unroll
    for (int at = 0; at < AT; ++at) {
      const int64_t a = wave_atom0 + at * 16 + j;
      if (a >= n_atoms) continue;
      const uint32_t M = st_m[wave][at * 16 + j], r = st_r[wave][at * 16 + j];
      *reinterpret_cast<uint2 *>(&keys[a]) = M >= 0x4000u && r != 0xFFFFFFFFu ? make_uint2(M << 16, r) : make_uint2(0u, 0u);
    }
  }
}

// Structured pair scoring (NN-B; replaces the sweep's 3,072 pair tiles).
//
// A type-2 code is +-c2 on the 8 positions of an octad O (c2 = bf16(2s) =
// 0.70703125) with an even number of minus signs; its score is
// c2 sum_{i in O} e_i x_i (exact products, fp32 sums), at most
// U(O) = c2 sum_{i in O} |x_i|.  Relative to the signs of x, a code flips a set
// F of the octad's positions and scores c2 (sum_O |x_i| - 2 sum_F |x_i|), with
// |F| of the parity of x's negative coordinates on O: the best code of an
// octad flips nothing (even) or its smallest |x_i| (odd).  One MFMA with |x|
// as the B operand gives U for 16 octads and 16 atoms: 48 tiles for the 759
// octads.  A type-1 code is +-c1 on two positions (c1 = bf16(4s) =
// 1.4140625); the best is c1 times the two largest |x_i|.
// A block of 4 waves holds AT atom tiles of 16 atoms per wave as MFMA B
// operands and streams the 48 octad tiles through LDS once (a second time
// only if a survivor list overflows):
//   set-up  one lane per atom scores the octad holding its 5 largest |x|
//           and the one holding its 4 largest and 6th largest (every 5
//           positions lie in exactly one octad, t2_steiner): usually at or
//           near the atom's best octad, so the sweep starts from a high floor
//           (~3 octads evaluated per atom instead of ~24); it also decodes a
//           type-3 floor F3 (Chase decoding, t3_dec) and makes t3_kernel's
//           per-atom set-up record (T3Setup);
//   sweep   every lane whose outputs hold an octad with U >= lo(floor) - margin
//           appends one 4-byte entry (atom, tile, quarter, output mask) to the
//           wave's list; floor is the highest of 2.0 (the origin rule), the
//           atom's best type-1 bucket, F3 and the best octad bucket found so
//           far.  When the list is nearly full and at the end of the pass the
//           wave evaluates it, one flagged octad per lane per round: the
//           octads' best codes scored exactly, the best bucket per atom kept by
//           an LDS atomic max, octads at or above the running best onto a
//           survivor list, which is compacted to the octads at their atom's
//           current best (and the thresholds raised) at the next stage end;
//   rows    the survivors at the final best bucket M give every type-2 code at
//           M: the flip sets F of the positions whose 2 c2 |x_i| fits in
//           U - lo(M) are enumerated and scored exactly; type 1 the same way
//           from the atom's coordinates when its best type-1 bucket is M; the
//           lowest codebook row by LDS atomic min;
//   pass 2  (only after a survivor list lost entries) the rows of the atoms
//           whose entries were lost, from a second sweep with their
//           thresholds at M (the other atoms' thresholds: +inf).
// The atom's key gets (M << 16, lowest row at M) in its upper 8 bytes, or
// (F3 << 16, no row) when F3 is above M, or 0 when neither reaches 2.0;
// t3_kernel takes that bucket as its floor.
// Buckets are taken by round-half-up like the dense sweep's, every score is
// an fp32 sum of exact products in ascending position order, so the answer
// equals the exact-score answer off near-ties (oracle/nn.py).
constexpr int kT2ST = 8;                           // octad tiles per LDS stage
constexpr int kT2Stages = kT2Tiles / kT2ST;        // 6
constexpr int kT2StageBytes = kT2ST * kTileBytes;  // 6,144
constexpr int kT2StageVecs = kT2StageBytes / 16;   // 384
constexpr int kT2Cap = 384;                        // candidate entries per wave (4 bytes each)
constexpr int kT2Surv = 256;                       // survivor entries per wave (4 bytes each)
constexpr uint32_t kNonFinite = 0xFFFFFFFFu;       // pair key of an atom with a NaN or infinite coordinate
constexpr float kC1 = 1.4140625f;                  // bf16(4s)
constexpr float kC2 = 0.70703125f;                 // bf16(2s)
static_assert(kT2StageVecs % 64 == 0, "octad stage splits into whole wave loads");
static_assert(kT2Tiles % kT2ST == 0 && kT2Tiles * kTileCodes >= kT2Octads && kT2Tiles <= 64, "whole octad stages");

// |x| at octad o's 8 positions (pp: ascending, one byte each) of the atom whose bf16 coordinates are xr,
// and the sign bits there (bit k: x negative at the k-th position).
__device__ __forceinline__ uint32_t t2_load(const uint32_t *xr, uint2 pp, float *xa) {
  const uint16_t *xh = reinterpret_cast<const uint16_t *>(xr);
  uint32_t sg = 0u;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t p = ((k < 4 ? pp.x : pp.y) >> (8 * (k & 3))) & 0xFFu;
    const uint32_t h = xh[p];
    xa[k] = __uint_as_float((h & 0x7FFFu) << 16);
    sg |= (h >> 15) << k;
  }
  return sg;
}

// The exact score of the octad code with flips F (bit k: sign opposite to x's at the k-th position).
__device__ __forceinline__ float t2_score(const float *xa, uint32_t F) {
  float S = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) S = fmaf(xa[k], ((F >> k) & 1u) ? -kC2 : kC2, S);
  return S;
}

// The exact score of the octad's best code: no flip when x has an even number of negative coordinates there,
// else its smallest |x| flipped.
__device__ __forceinline__ float t2_best(const float *xa, uint32_t sg) {
  float mn = xa[0];
  int mi = 0;
#pragma unroll
  for (int k = 1; k < 8; ++k)
    if (xa[k] < mn) {
      mn = xa[k];
      mi = k;
    }
  return t2_score(xa, (__popc(sg) & 1) ? 1u << mi : 0u);
}

// Colex rank of the 5-subset p0 < p1 < ... < p4 of the positions: C(p0,1) + C(p1,2) + ... + C(p4,5).
__device__ __forceinline__ uint32_t subset5_rank(const uint32_t *p) {
  return p[0] + p[1] * (p[1] - 1u) / 2u + p[2] * (p[2] - 1u) * (p[2] - 2u) / 6u +
         p[3] * (p[3] - 1u) * (p[3] - 2u) * (p[3] - 3u) / 24u +
         p[4] * (p[4] - 1u) * (p[4] - 2u) * (p[4] - 3u) * (p[4] - 4u) / 120u;
}

// The lowest row among octad o's codes at bucket M: every flip set of the parity of sg whose flipped |x|
// can fit in U - lo(M) is scored.
__device__ __forceinline__ uint32_t t2_rows_at(const float *xa, uint32_t sg, uint32_t o, uint32_t M,
                                               const uint32_t *__restrict__ t2_rows) {
  float U = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) U = fmaf(xa[k], kC2, U);
  const float room = (U - __uint_as_float((M << 16) - 0x8000u)) + U * 0x1p-14f;
  uint32_t C = 0u;
#pragma unroll
  for (int k = 0; k < 8; ++k) C |= (xa[k] * (2.f * kC2) <= room ? 1u : 0u) << k;
  const uint32_t par = static_cast<uint32_t>(__popc(sg)) & 1u;
  uint32_t rmin = 0xFFFFFFFFu;
  for (uint32_t F = C;; F = (F - 1u) & C) {  // every subset of C, the empty one last
    if ((static_cast<uint32_t>(__popc(F)) & 1u) == par) {
      const float S = t2_score(xa, F);
      if (S > 0.f && t3_bucket(S) == M) rmin = min(rmin, t2_rows[o * 128u + ((sg ^ F) & 0x7Fu)]);
    }
    if (F == 0u) break;
  }
  return rmin;
}

// The lowest row among the type-1 codes at bucket M of the atom whose bf16 coordinates are xr (v1: its
// largest |x|): the positions i with c1 (|x_i| + v1) >= lo(M) - margin, every pair of them, all four signs.
__device__ uint32_t t1_rows_at(const uint32_t *xr, float v1, uint32_t M, const uint32_t *__restrict__ t1_rows) {
  const uint16_t *xh = reinterpret_cast<const uint16_t *>(xr);
  const float lo = __uint_as_float((M << 16) - 0x8000u);
  const float top = v1 * kC1;
  const float need = lo - top - top * 0x1p-13f;
  uint32_t C = 0u;
  for (int i = 0; i < kDim; ++i) {
    const float a = __uint_as_float((static_cast<uint32_t>(xh[i]) & 0x7FFFu) << 16);
    C |= (a * kC1 >= need ? 1u : 0u) << i;
  }
  uint32_t rmin = 0xFFFFFFFFu;
  for (uint32_t ci = C; ci != 0u; ci &= ci - 1u) {
    const int i = __builtin_ctz(ci);
    const float xi = __uint_as_float(static_cast<uint32_t>(xh[i]) << 16) * kC1;
    for (uint32_t cj = ci & (ci - 1u); cj != 0u; cj &= cj - 1u) {
      const int j = __builtin_ctz(cj);
      const float xj = __uint_as_float(static_cast<uint32_t>(xh[j]) << 16) * kC1;
#pragma unroll
      for (uint32_t e = 0; e < 4; ++e) {
        const float S = ((e & 1u) ? -xi : xi) + ((e & 2u) ? -xj : xj);
        if (S > 0.f && t3_bucket(S) == M) rmin = min(rmin, t1_rows[(static_cast<uint32_t>(i) * kDim + j) * 4u + e]);
      }
    }
  }
  return rmin;
}

// LOAD: 0 the bf16 planes from prep_kernel (xb); 1 the fp32 atoms (src), rounded here and written to xb
// for t3_kernel; 2 the same with the row scale applied first (src / sigma, as prep_kernel<true>).
template <int AT, int LOAD>
__global__ __launch_bounds__(kThreads, 4) void t12_kernel(uint4 *__restrict__ xb, const float *__restrict__ src,
                                                          const float *__restrict__ sigma, int64_t atoms_per_row,
                                                          int64_t n_atoms,
                                                          const uint8_t *__restrict__ t2_tiles,
                                                          const uint2 *__restrict__ t2_pos,
                                                          const uint32_t *__restrict__ t2_rows,
                                                          const uint32_t *__restrict__ t1_rows,
                                                          const uint16_t *__restrict__ t2_steiner,
                                                          const uint32_t *__restrict__ t3_dec,
                                                          uint4 *__restrict__ keys, uint2 *__restrict__ rec,
                                                          int rows_by_sweep) {
  constexpr int NA = AT * 16;  // atoms per wave
  static_assert(NA <= 128 && NA <= 64, "entry layout: 7 bits of atom; one lane per atom at set-up");
  __shared__ __align__(16) uint8_t stg[2][kT2StageBytes];
  __shared__ uint32_t cand[kWaves][kT2Cap];   // atom | tile << 7 | quarter << 13 | output mask << 16
  __shared__ uint32_t surv[kWaves][kT2Surv];  // atom | octad << 7 | (bucket - 0x4000) << 17
  __shared__ __align__(16) uint32_t xw[kWaves][NA][12];  // the atoms' bf16 coordinates (pairs)
  __shared__ uint32_t st_m[kWaves][NA], st_r[kWaves][NA];
  __shared__ uint32_t st_o[kWaves][NA];  // the octad of the atom's 5 largest |x| (scored at set-up)
  __shared__ uint32_t st_o2[kWaves][NA];  // the octad of its 4 largest and its 6th largest |x| (set-up)
  __shared__ uint32_t st_f[kWaves][NA];   // the type-3 floor: bucket of the best decoded type-3 code (or 0)
  __shared__ uint32_t surv_n[kWaves];
  __shared__ uint32_t st_ovf[kWaves][2];  // atoms (bits) whose survivor list lost an entry: rows by pass 2

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, q = lane >> 4, j = lane & 15;
  const int64_t wave_atom0 = static_cast<int64_t>(blockIdx.x) * (kWaves * NA) + static_cast<int64_t>(wave) * NA;

  if (lane < 2) st_ovf[wave][lane] = 0u;
  if (lane == 0) surv_n[wave] = 0u;
  bf16x8 b[AT];
  float mg[AT], v1[AT];
  uint32_t m1b[AT];  // the best type-1 bucket (0 below 2.0)
  uint32_t nonfinite = 0u;  // bit at: the atom has a NaN or infinite coordinate, or sum |x| overflows fp32
#pragma unroll
  for (int at = 0; at < AT; ++at) {
    const int64_t a = wave_atom0 + at * 16 + j;
    uint4 w = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (LOAD == 0) {
      if (a < n_atoms && q < 3) w = xb[a * 3 + q];
    } else {
      float v[8];
      load_coords8<LOAD == 2>(src, sigma, atoms_per_row, n_atoms, a, q, v);  // (zeros past the end, q == 3)
      w.x = bf16_rne_bits(v[0]) | (bf16_rne_bits(v[1]) << 16);
      w.y = bf16_rne_bits(v[2]) | (bf16_rne_bits(v[3]) << 16);
      w.z = bf16_rne_bits(v[4]) | (bf16_rne_bits(v[5]) << 16);
      w.w = bf16_rne_bits(v[6]) | (bf16_rne_bits(v[7]) << 16);
      if (a < n_atoms && q < 3) xb[a * 3 + q] = w;
    }
    if (q < 3) *reinterpret_cast<uint4 *>(&xw[wave][at * 16 + j][4 * q]) = w;
    const uint4 wa = make_uint4(w.x & 0x7FFF7FFFu, w.y & 0x7FFF7FFFu, w.z & 0x7FFF7FFFu, w.w & 0x7FFF7FFFu);
    b[at] = __builtin_bit_cast(bf16x8, wa);
    // the two largest |x| and sum |x| over this lane's 8 coordinates, then over the atom's lanes
    float t1 = 0.f, t2 = 0.f, ax = 0.f;
    const uint32_t ww[4] = {wa.x, wa.y, wa.z, wa.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = __uint_as_float(e & 1 ? ww[e / 2] & 0xFFFF0000u : ww[e / 2] << 16);
      t2 = fmaxf(t2, fminf(t1, v));
      t1 = fmaxf(t1, v);
      ax += v;
    }
#pragma unroll
    for (int sh = 16; sh <= 32; sh <<= 1) {
      const float o1 = __shfl_xor(t1, sh, 64), o2 = __shfl_xor(t2, sh, 64);
      t2 = fmaxf(fmaxf(t2, o2), fminf(t1, o1));
      t1 = fmaxf(t1, o1);
      ax += __shfl_xor(ax, sh, 64);
    }
    // sum |x| is NaN or infinite exactly when a coordinate is (or the sum overflows fp32): such an atom
    // goes to the origin
    nonfinite |= (ax <= 3.402823466e38f ? 0u : 1u) << at;
    const float s1 = t1 * kC1 + t2 * kC1;  // exact products, one rounding
    const uint32_t bk = s1 > 0.f ? t3_bucket(s1) : 0u;
    m1b[at] = bk >= 0x4000u ? bk : 0u;
    v1[at] = t1;
    // the margin for the MFMA's fp32 summation order of U
    mg[at] = ax * kC2 * 0x1p-14f;
  }
  for (int i = lane; i < NA; i += 64) st_r[wave][i] = 0xFFFFFFFFu;
#pragma unroll
  for (int at = 0; at < AT; ++at)
    if (q == 0) st_m[wave][at * 16 + j] = m1b[at];

  const uint4 *gsrc = reinterpret_cast<const uint4 *>(t2_tiles);
  auto stage_copy = [&](int g, int dst) {
    const int stage = g % kT2Stages;
#pragma unroll
    for (int i = 0; i < (kT2StageVecs + kThreads - 1) / kThreads; ++i) {
      if (i * kThreads + wave * 64 >= kT2StageVecs) break;  // (wave-uniform)
      const uint4 *src = gsrc + static_cast<size_t>(stage) * kT2StageVecs + i * kThreads + tid;
      uint8_t *d = stg[dst] + (i * kThreads + wave * 64) * 16;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(src),
                                       (__attribute__((address_space(3))) void *)(d), 16, 0, 0);
    }
  };

  int cnt = 0;  // entries in this wave's candidate list (wave-uniform)
  // One flagged octad per lane per round (the list is worked as a stack: an entry with flagged octads left
  // goes back on it).  pass 1: the octad's best code -> st_m (atomic max), and the octad onto the survivor
  // list when it is at or above the atom's running best; pass 2: the lowest row at st_m -> st_r.
  bool flushed = false;  // (wave-uniform) a flush ran since the last compaction
  auto flush = [&](int pass) {
    flushed |= cnt > 0;
    while (cnt > 0) {  // (wave-uniform)
      const int n = min(cnt, 64);
      cnt -= n;
      const bool act = lane < n;
      const uint32_t ce = act ? cand[wave][cnt + lane] : 0u;
      const uint32_t mask = (ce >> 16) & 0xFu;
      const uint32_t rest = mask & (mask - 1u);
      if (act) {
        const int al = static_cast<int>(ce & 0x7Fu);
        const uint32_t o = ((ce >> 7) & 0x3Fu) * kTileCodes + 4u * ((ce >> 13) & 3u) +
                           static_cast<uint32_t>(__builtin_ctz(mask));
        // (padding slots: U = 0 unless the margin is not finite; the set-up octads: scored already)
        if (o < static_cast<uint32_t>(kT2Octads) && (pass == 2 || (o != st_o[wave][al] && o != st_o2[wave][al]))) {
          float xa[8];
          const uint32_t sg = t2_load(xw[wave][al], t2_pos[o], xa);
          if (pass == 1) {
            const float S = t2_best(xa, sg);
            const uint32_t bk = S > 0.f ? t3_bucket(S) : 0u;
            if (bk >= 0x4000u) {
              const uint32_t old = atomicMax(&st_m[wave][al], bk);
              if (bk >= old) {
                const uint32_t slot = atomicAdd(&surv_n[wave], 1u);
                if (slot < static_cast<uint32_t>(kT2Surv))
                  surv[wave][slot] = static_cast<uint32_t>(al) | o << 7 | (bk - 0x4000u) << 17;
                else
                  atomicOr(&st_ovf[wave][al >> 5], 1u << (al & 31));
              }
            }
          } else {
            const uint32_t r = t2_rows_at(xa, sg, o, st_m[wave][al], t2_rows);
            if (r != 0xFFFFFFFFu) atomicMin(&st_r[wave][al], r);
          }
        }
      }
      // the entries with flagged octads left go back on the list (every lane read its entry above)
      const uint64_t bm = __ballot(rest != 0u);
      if (rest != 0u)
        cand[wave][cnt + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bm >> 32),
                                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bm), 0u))] =
            (ce & ~0xF0000u) | rest << 16;
      cnt += __popcll(bm);
    }
  };

  // Keep only the survivors at their atom's current best bucket (an atom that lost an entry to a full
  // list is flagged in st_ovf, and pass 2 gives its rows).
  auto compact = [&]() {
    const uint32_t n = min(surv_n[wave], static_cast<uint32_t>(kT2Surv));
    uint32_t w = 0u;
    for (uint32_t base = 0u; base < n; base += 64u) {
      const uint32_t i = base + static_cast<uint32_t>(lane);
      uint32_t e = 0u;
      bool keep = false;
      if (i < n) {
        e = surv[wave][i];
        keep = (e >> 17) + 0x4000u == st_m[wave][e & 0x7Fu];
      }
      const uint64_t msk = __ballot(keep);
      // (in place: every lane read its entry before any writes, and w + rank <= i)
      if (keep)
        surv[wave][w + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(msk >> 32),
                                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(msk), 0u))] = e;
      w += static_cast<uint32_t>(__popcll(msk));
    }
    if (lane == 0) surv_n[wave] = w;
  };

  // The threshold on U: an octad can reach bucket B only if U >= lo(B) - margin; no bucket below the
  // floor (2.0, the best type-1 bucket, the best octad bucket found so far) can win.
  float thr[AT];
  auto set_thr = [&](int at, uint32_t mlow) {
    mlow = max(mlow, 0x4000u);
    thr[at] = __uint_as_float((mlow << 16) - 0x8000u) - mg[at];
  };

  const int a_off = (q < 3 ? q : 0) * 256 + j * 16;
  const uint32_t ebase = static_cast<uint32_t>(j) | static_cast<uint32_t>(q) << 13;  // the lane's entry bits
  stage_copy(0, 0);
  __syncthreads();
  // The floor from two octads per atom, one lane per atom: the octad holding its 5 largest |x| (every 5
  // positions lie in exactly one octad) and the one holding its 4 largest and its 6th largest, usually at
  // or near the atom's best octad, scored exactly and entered like swept candidates (the second octad:
  // 4.1 -> 3.1 octads swept per atom, t12 3.12 -> 2.96 ms on config 4).
  if (lane < NA) {
    const int al = lane;
    const uint16_t *xh = reinterpret_cast<const uint16_t *>(xw[wave][al]);
    // the 6 largest keys |x| bits << 5 | position (bf16 magnitudes order as integers; distinct keys), kept
    // descending by a max / min pair per slot
    uint32_t tk[6] = {0u, 0u, 0u, 0u, 0u, 0u};
    uint32_t ysg = 0u, lk0 = 0xFFFFFFFFu, lk1 = 0xFFFFFFFFu;  // sign bits; the two smallest keys
    T3Setup t3s;  // t3_kernel's set-up record
    for (int i = 0; i < kDim; ++i) {
      const uint32_t h = xh[i];
      t3s.add(__uint_as_float(h << 16), static_cast<uint32_t>(i));
      uint32_t k = (h & 0x7FFFu) << 5 | static_cast<uint32_t>(i);
      ysg |= (h >> 15) << i;
      lk1 = min(lk1, max(lk0, k));
      lk0 = min(lk0, k);
#pragma unroll
      for (int t = 0; t < 6; ++t) {
        const uint32_t hi = max(tk[t], k);
        k = min(tk[t], k);
        tk[t] = hi;
      }
    }
    // The type-3 floor (Chase decoding): the signs of x as a word, and that word with its least reliable
    // position (smallest |x|), its second, or both flipped, each decoded to the nearest Golay word by
    // syndrome (t3_dec); each word's type-3 codes with the -3 at one of the 6 largest |x| scored exactly
    // as t3_kernel scores them (t3_dot, then one fma).  The best bucket is a type-3 code's, so the atom's
    // type-3 best reaches it: octads below it cannot win (same answer, fewer candidates; config-4 atoms
    // simulated: 0.58 -> 0.40 of the atom-tile x octad-tile steps hold a candidate), and t3_kernel
    // starts from it (0.24 -> 0.19 of its steps).
    {
      uint32_t xr[12];
#pragma unroll
      for (int d = 0; d < 12; ++d) xr[d] = xw[wave][al][d];
      uint32_t syn = 0u;
#pragma unroll
      for (int jj = 0; jj < 12; ++jj) syn |= static_cast<uint32_t>(__popc(ysg & t3_dec[4096 + jj]) & 1) << jj;
      const uint32_t l0 = lk0 & 31u, l1 = lk1 & 31u;
      const uint32_t c0 = t3_dec[4108 + l0], c1 = t3_dec[4108 + l1];
      uint32_t tpos[6];
      float xp[6];
#pragma unroll
      for (int c = 0; c < 6; ++c) {
        tpos[c] = tk[c] & 31u;
        xp[c] = __uint_as_float(static_cast<uint32_t>(xh[tpos[c]]) << 16);
      }
      float best = -__builtin_inff();
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t fm = (t & 1 ? 1u << l0 : 0u) | (t & 2 ? 1u << l1 : 0u);
        const uint32_t sy = syn ^ (t & 1 ? c0 : 0u) ^ (t & 2 ? c1 : 0u);
        const uint32_t w = (ysg ^ fm ^ t3_dec[sy]) & 0xFFFFFFu;
        const bool sg = (w >> 23) & 1u;
        const float D = t3_dot(xr, sg ? w ^ 0xFFFFFFu : w);
        const float S = sg ? -D : D;
#pragma unroll
        for (int c = 0; c < 6; ++c) best = fmaxf(best, fmaf(-xp[c], ((w >> tpos[c]) & 1u) ? kT3Beta : kT3Alpha, S));
      }
      const uint32_t f3 = best > 0.f ? t3_bucket(best) : 0u;
      st_f[wave][al] = f3 >= 0x4000u ? f3 : 0u;
    }
    {
      uint2 ra, rb;
      t3s.record(ra, rb);
      const int64_t a = wave_atom0 + al;
      if (a < n_atoms) {
        reinterpret_cast<uint2 *>(&keys[a])[0] = ra;
        rec[a] = rb;
      }
    }
    uint32_t tp[5], tq[5];
#pragma unroll
    for (int t = 0; t < 5; ++t) {
      tp[t] = tk[t] & 31u;
      tq[t] = tk[t < 4 ? t : 5] & 31u;
    }
    // positions ascending (a 5-input sorting network), then the octads of the two subsets
    constexpr int kNet[9][2] = {{0, 1}, {3, 4}, {2, 4}, {2, 3}, {0, 3}, {0, 2}, {1, 4}, {1, 3}, {1, 2}};
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      const uint32_t lo = min(tp[kNet[k][0]], tp[kNet[k][1]]), hi = max(tp[kNet[k][0]], tp[kNet[k][1]]);
      tp[kNet[k][0]] = lo;
      tp[kNet[k][1]] = hi;
      const uint32_t lo2 = min(tq[kNet[k][0]], tq[kNet[k][1]]), hi2 = max(tq[kNet[k][0]], tq[kNet[k][1]]);
      tq[kNet[k][0]] = lo2;
      tq[kNet[k][1]] = hi2;
    }
    // (the keys are distinct, so the positions are; the rank is clamped into the table all the same)
    const uint32_t o1 = t2_steiner[min(subset5_rank(tp), static_cast<uint32_t>(kT2Subsets5 - 1))];
    const uint32_t o2 = t2_steiner[min(subset5_rank(tq), static_cast<uint32_t>(kT2Subsets5 - 1))];
    st_o[wave][al] = o1;
    st_o2[wave][al] = o2;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t o = r ? o2 : o1;
      if (r == 1 && o2 == o1) break;
      float xa[8];
      const uint32_t sg = t2_load(xw[wave][al], t2_pos[o], xa);
      const float S = t2_best(xa, sg);
      const uint32_t bk = S > 0.f ? t3_bucket(S) : 0u;
      if (bk >= 0x4000u && bk >= st_m[wave][al]) {
        st_m[wave][al] = bk;
        const uint32_t slot = atomicAdd(&surv_n[wave], 1u);
        if (slot < static_cast<uint32_t>(kT2Surv))
          surv[wave][slot] = static_cast<uint32_t>(al) | o << 7 | (bk - 0x4000u) << 17;
        else
          atomicOr(&st_ovf[wave][al >> 5], 1u << (al & 31));
      }
    }
  }
#pragma unroll
  for (int at = 0; at < AT; ++at) set_thr(at, max(st_m[wave][at * 16 + j], st_f[wave][at * 16 + j]));
  int g_end = kT2Stages;
  for (int g = 0; g < g_end; ++g) {
    const int pass = 1 + g / kT2Stages, buf = g & 1;
    if (g + 1 < g_end) stage_copy(g + 1, buf ^ 1);
    if (g == kT2Stages) {
      // pass 2 (a survivor list lost entries): thresholds at the final best buckets of the atoms concerned
#pragma unroll
      for (int at = 0; at < AT; ++at) {
        const int al = at * 16 + j;
        const bool redo = rows_by_sweep != 0 || ((st_ovf[wave][al >> 5] >> (al & 31)) & 1u) != 0u;
        const uint32_t M = st_m[wave][al];
        // (an atom below its type-3 floor needs no pair rows)
        thr[at] = redo && M >= 0x4000u && M >= st_f[wave][al] ? __uint_as_float((M << 16) - 0x8000u) - mg[at]
                                                              : __builtin_inff();
      }
    }
    const uint8_t *L = stg[buf] + a_off;
    const int tile0 = (g % kT2Stages) * kT2ST;
    // (unrolled: the A tiles' LDS offsets and the entries' tile bits become constants; 2.71 -> 2.65 ms)
#pragma unroll 8
    for (int k = 0; k < kT2ST; ++k) {
      const bf16x8 a = *reinterpret_cast<const bf16x8 *>(L + k * kTileBytes);
      f32x4 c[AT];
#pragma unroll
      for (int at = 0; at < AT; ++at)
        c[at] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[at], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
      for (int at = 0; at < AT; ++at) {
        // each output against the atom's threshold: the largest of the four against it, one compare and
        // one wave mask; the four compares only on a hit
        // (IEEE maximum, v_maximum3_f32: a NaN output, only a non-finite atom's, makes the step a miss)
        const float mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(c[at][0], c[at][1]),
                                                       __builtin_elementwise_maximum(c[at][2], c[at][3]));
        const bool hit = mx >= thr[at];
        const uint64_t msk = __ballot(hit);
        if (msk == 0ull) continue;
        if (cnt > kT2Cap - 64) flush(pass);
        if (hit) {
          const bool h0 = c[at][0] >= thr[at], h1 = c[at][1] >= thr[at];
          const bool h2 = c[at][2] >= thr[at], h3 = c[at][3] >= thr[at];
          const uint32_t mask = (h0 ? 1u : 0u) | (h1 ? 2u : 0u) | (h2 ? 4u : 0u) | (h3 ? 8u : 0u);
          const uint32_t pos = static_cast<uint32_t>(cnt) +
                               __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(msk >> 32),
                                                         __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(msk), 0u));
          cand[wave][pos] = (ebase + static_cast<uint32_t>(at * 16)) | static_cast<uint32_t>(tile0 + k) << 7 | mask << 16;
        }
        cnt += __popcll(msk);
      }
    }
    // the list is evaluated when it is nearly full (in the tile loop) and at the end of each pass (with the
    // type-3 floor, evaluating at stage ends once 64 entries were listed measured 4% slower); the best
    // buckets change only then, so the survivors are compacted and the thresholds raised only after one
    if (g == kT2Stages - 1 || g == 2 * kT2Stages - 1) flush(pass);
    if (pass == 1 && flushed) {
      compact();
      flushed = false;
#pragma unroll
      for (int at = 0; at < AT; ++at) set_thr(at, max(st_m[wave][at * 16 + j], st_f[wave][at * 16 + j]));
    }
    if (g == kT2Stages - 1) {
      if (__syncthreads_or(rows_by_sweep != 0 || (st_ovf[wave][0] | st_ovf[wave][1]) != 0u)) {
        g_end = 2 * kT2Stages;
        stage_copy(g + 1, buf ^ 1);  // buffer buf ^ 1 was last read in stage g - 1, before the barrier
        __syncthreads();
      }
    } else {
      __syncthreads();
    }
  }
  {
    // the survivors are the octads at their atom's final best bucket (compacted after the last flush; a
    // set-up octad left below it has no code at the final bucket, so it gives no row);
    // pass 2 gave the rows of the atoms whose list lost entries
    const int ns = static_cast<int>(min(surv_n[wave], static_cast<uint32_t>(kT2Surv)));
    for (int i = lane; i < ns; i += 64) {
      const uint32_t se = surv[wave][i];
      const int al = static_cast<int>(se & 0x7Fu);
      if (rows_by_sweep != 0 || ((st_ovf[wave][al >> 5] >> (al & 31)) & 1u) != 0u) continue;
      if (st_m[wave][al] < st_f[wave][al]) continue;  // (below the type-3 floor: no pair rows needed)
      const uint32_t o = (se >> 7) & 0x3FFu;
      float xa[8];
      const uint32_t sg = t2_load(xw[wave][al], t2_pos[o], xa);
      const uint32_t r = t2_rows_at(xa, sg, o, st_m[wave][al], t2_rows);
      if (r != 0xFFFFFFFFu) atomicMin(&st_r[wave][al], r);
    }
  }
  __syncthreads();
  if (q == 0) {
#pragma unroll
    for (int at = 0; at < AT; ++at) {
      const int64_t a = wave_atom0 + at * 16 + j;
      if (a >= n_atoms) continue;
      const uint32_t M = st_m[wave][at * 16 + j], F = st_f[wave][at * 16 + j];
      uint32_t r = st_r[wave][at * 16 + j];
      if (M >= 0x4000u && M >= F && m1b[at] == M) r = min(r, t1_rows_at(xw[wave][at * 16 + j], v1[at], M, t1_rows));
      // (a non-finite atom: the marker kNonFinite, which pick_kernel maps to the origin as the dense sweep
      // does; as a pair bucket it gives t3_kernel a NaN threshold, hence no candidates.  An atom whose
      // type-3 floor is above its best pair bucket: the floor without a row, as t3_kernel's starting best,
      // which its type-3 best reaches, so pick_kernel takes t3_kernel's row)
      reinterpret_cast<uint2 *>(&keys[a])[1] =
          (nonfinite >> at) & 1u ? make_uint2(kNonFinite, 0u)
          : F > M               ? make_uint2(F << 16, 0xFFFFFFFFu)
          : M >= 0x4000u && r != 0xFFFFFFFFu ? make_uint2(M << 16, r)
                                             : make_uint2(0u, 0u);
    }
  }
}

// Resolve: per block 256 atoms.
//   scan     thread per atom: its keys (type-3 region; pair region: NN-B the
//            first and the last group at the best bucket, NN-T / NN-P the
//            first group at the best |score|), the atom's coordinates into LDS
//            (bf16 pairs; NN-P: fp32), and its candidates: (group, lane) of
//            the keys' masks in the regions holding the overall best;
//   rounds   up to kRsPerRound candidates per atom per round, compacted into
//            one LDS list by a block prefix sum and rescanned kRL = 4 lanes
//            per candidate, lane t scoring the 4 codes of its quarter in
//            tiles t, t+4, t+8, t+12 of the group (NN-B/T: value ids from
//            sw_dq expanded to bf16 pairs, v_dot2_f32_bf16 = exact bf16
//            products, fp32 sums; NN-P: the rows' raw int8 coordinates, fp64
//            dot products of the fp32 atom with the fp32 codebook values,
//            exact to 2^-48), combined by DPP quad moves and merged per atom;
//   span     NN-B atoms whose best pair bucket is reached in a group that is
//            neither a first nor a last group of any lane (a lane with three or
//            more such groups, or three or more pair slices at that bucket) and
//            whose earliest such group holds no positive hit: the pair groups
//            after the earliest up to the latest are rescanned by the whole
//            block, in ascending chunks, until one holds a positive hit
//            (~0.04% of atoms).
// Selection (the reference's rule: lowest codebook row among the best):
//   a type-3 code wins with its own row; a representative r with score s wins
//   as r when s is the best (s > 0) and as its antipode when -s is.  Rows of
//   representatives rise with sweep order and their antipodes' rows fall
//   (negation reverses the lexicographic order) and every representative row
//   is below every antipode row, so among pair codes the lowest winning row is
//   the lowest positive hit if one exists -- in the first group that reaches
//   the best bucket when that group has one, else somewhere up to the last --
//   and otherwise the antipode of the highest negative hit, which lies in the
//   last group.  The answer is the lower of that and the type-3 winner.
// NN-T / NN-P compare exact scores, where two codes reach the same maximum
// only on an exact fp32 tie (a near-tie); the first group's winner is taken.
// NN-B falls back to the best rounded score, lowest row on ties, if the fp32
// sums disagree with the sweep's bucket.  Then the int32 index and,
// optionally, the packed 9-byte groups.
constexpr int kRsPerRound = 4;
constexpr int kRsCap = 256 * kRsPerRound;
constexpr int kRL = 4;         // rescan lanes per candidate (one quad)
constexpr int kRT = kG / kRL;  // tiles per rescan lane
constexpr uint32_t kNone = 0xFFFFFFFFu;

template <int MODE>
struct RsScore {  // per-candidate / per-atom running result
  typedef typename std::conditional<MODE == kModeP, double, float>::type T;
};

// Sweep position (global, code granularity) of lane qq's code e in tile t of group g.
__device__ __forceinline__ int sweep_pos(int g, int t, int qq, int e) { return (g * kG + t) * kTileCodes + 4 * qq + e; }

// The 256 indices of a block (ids, in LDS) as packed 9-byte groups of 4 atoms at packed_out (bytes: LDS
// staging of 64 groups); every thread of the block calls it.
__device__ __forceinline__ void store_packed_block(const int32_t *ids, uint8_t *bytes, int64_t a0, int64_t n_atoms,
                                                   uint8_t *__restrict__ packed_out, int tid) {
  const int64_t n_groups = (n_atoms + 3) / 4;
  const int64_t g0 = a0 / 4;
  const int64_t groups_here = min(static_cast<int64_t>(64), n_groups - g0);
  if (tid < groups_here) {
    const int i = tid * 4;
    group_to_bytes(ids[i], ids[i + 1], ids[i + 2], ids[i + 3], bytes + tid * 9);
  }
  __syncthreads();
  uint8_t *dst = packed_out + g0 * 9;
  if (groups_here == 64 && aligned16(packed_out)) {
    if (tid < 36) reinterpret_cast<uint4 *>(dst)[tid] = reinterpret_cast<const uint4 *>(bytes)[tid];
  } else {
    const int nb = static_cast<int>(groups_here * 9);
    for (int i = tid; i < nb; i += 256) dst[i] = bytes[i];
  }
}

template <int MODE, bool FUSED>
__global__ __launch_bounds__(256) void resolve_kernel(const uint4 *__restrict__ keys, int64_t n_atoms,
                                                      const float *__restrict__ src,
                                                      const float *__restrict__ sigma, int64_t atoms_per_row,
                                                      const uint4 *__restrict__ xb,
                                                      const uint32_t *__restrict__ sw_dq,
                                                      const uint32_t *__restrict__ sw_idx,
                                                      const uint32_t *__restrict__ sw_anti,
                                                      const int8_t *__restrict__ cb_raw,
                                                      const uint8_t *__restrict__ sw_tiles,
                                                      const uint64_t *__restrict__ recs, int n_recs,
                                                      int64_t rec_stride,
                                                      int32_t *__restrict__ idx_out, uint8_t *__restrict__ packed_out) {
  typedef typename RsScore<MODE>::T score_t;
  constexpr bool B = MODE == kModeB;
  constexpr int XW = MODE == kModeP ? kDim : 12;  // words of one atom's coordinates in LDS
  constexpr int kP0 = kType3Tiles / kG;           // first global group of the pair region
  __shared__ __align__(16) uint32_t xs[256 * XW];
  __shared__ uint32_t tmp[kRsPerRound * 256];     // per-thread candidates before compaction
  __shared__ uint32_t cand[kRsCap];               // atom | lane << 8 | pair << 10 | global group << 11
  __shared__ score_t res_v[kRsCap];
  __shared__ uint32_t res_c[kRsCap];              // row of the best (rounded) score
  __shared__ uint32_t res_f0[B ? kRsCap : 1];     // NN-B: lowest row at bucket M (pair: positive hits)
  __shared__ uint32_t res_f1[B ? kRsCap : 1];     // NN-B pair: lowest antipode row of negative hits
  __shared__ uint32_t Ms[256];                    // per atom: the best bucket (NN-B)
  __shared__ int wave_sum[4];
  __shared__ int32_t ids[256];
  __shared__ __align__(16) uint8_t bytes[64 * 9];
  __shared__ uint32_t span_list[B ? 256 : 1];      // NN-B: atoms needing the span rescan, their first code,
  __shared__ uint32_t span_lo[B ? 256 : 1];        // code count, running offset and lowest positive-hit row
  __shared__ uint32_t span_cnt[B ? 256 : 1];
  __shared__ uint32_t span_min[B ? 256 : 1];
  __shared__ uint32_t span_n;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t a0 = static_cast<int64_t>(blockIdx.x) * 256;
  const int64_t a = a0 + tid;
  if (tid == 0) span_n = 0;

  // ---- scan: keys, coordinates, origin rules ----
  // candidate groups (global) and lane masks: [0] type-3; [1..4] pair groups:
  // NN-B the first and last group of the pair record with the earliest first
  // group and of the one with the latest last group (the records of the pair
  // slices at the best pair bucket, in slice = group order); NN-T / NN-P the
  // first group at the best |score| in [1]
  uint32_t M = 0, grp[5] = {0u, 0u, 0u, 0u, 0u}, lanes[5] = {0u, 0u, 0u, 0u, 0u};
  uint32_t span_g0 = 0, span_g1 = 0;  // NN-B: pair groups (span_g0, span_g1] to rescan for positive hits
  bool many = false;
  bool active = false;
  if (a < n_atoms) {
    const uint4 k = keys[a];
    if constexpr (B) {
      const uint32_t MT = k.x >> 16;
      uint32_t MP = 0u;
      uint64_t rF = 0ull, rL = 0ull;
      int n_at = 0;
      for (int i = 0; i < n_recs; ++i) {
        const uint64_t r = recs[static_cast<int64_t>(i) * rec_stride + a];
        const uint32_t bb = static_cast<uint32_t>(r >> 48);
        if (bb > MP) {
          MP = bb;
          rF = rL = r;
          n_at = 1;
          many = ((r >> 40) & 1ull) != 0ull;
        } else if (bb == MP && bb != 0u) {
          rL = r;
          ++n_at;
          many |= ((r >> 40) & 1ull) != 0ull;
        }
      }
      many |= n_at > 2;  // a record between the two: its groups are not candidates
      M = max(MT, MP);
      if (M != 0u && MT == M) {
        grp[0] = 0x3FFu - ((k.x >> 6) & 0x3FFu);
        lanes[0] = (k.x >> 2) & 0xFu;
      }
      if (M != 0u && MP == M) {
        const uint64_t rr[2] = {rF, rL};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (h == 1 && n_at < 2) break;
          const uint32_t F = kP0 + static_cast<uint32_t>((rr[h] >> 32) & 0xFFu);
          const uint32_t Lg = kP0 + static_cast<uint32_t>((rr[h] >> 24) & 0xFFu);
          grp[1 + 2 * h] = F;
          lanes[1 + 2 * h] = static_cast<uint32_t>((rr[h] >> 4) & 0xFu);
          if (Lg == F) {
            lanes[1 + 2 * h] |= static_cast<uint32_t>(rr[h] & 0xFu);
          } else {
            grp[2 + 2 * h] = Lg;
            lanes[2 + 2 * h] = static_cast<uint32_t>(rr[h] & 0xFu);
          }
        }
        span_g0 = kP0 + static_cast<uint32_t>((rF >> 32) & 0xFFu);
        span_g1 = kP0 + static_cast<uint32_t>((rL >> 24) & 0xFFu);
      } else {
        many = false;
      }
    } else {
      const uint64_t kt = (static_cast<uint64_t>(k.y) << 32) | k.x, kp = (static_cast<uint64_t>(k.w) << 32) | k.z;
      const uint32_t MT = static_cast<uint32_t>(kt >> 32), MP = static_cast<uint32_t>(kp >> 32);
      M = max(MT, MP);
      if (kt != 0ull && MT == M) {
        grp[0] = 0x3FFu - static_cast<uint32_t>((kt >> 4) & 0x3FFu);
        lanes[0] = static_cast<uint32_t>(kt & 0xFu);
      }
      if (kp != 0ull && MP == M) {
        grp[1] = kP0 + 0x3FFu - static_cast<uint32_t>((kp >> 4) & 0x3FFu);
        lanes[1] = static_cast<uint32_t>(kp & 0xFu);
      }
    }
    double nrm2 = 0.0;
    bool nonfinite = false;  // NN-B / NN-T: a NaN or infinite coordinate (its index is the origin)
#pragma unroll
    for (int qq = 0; qq < 3; ++qq) {
      if constexpr (MODE == kModeP) {
        float v[8];
        load_coords8<FUSED>(src, sigma, atoms_per_row, n_atoms, a, qq, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xs[tid * XW + 8 * qq + e] = __float_as_uint(v[e]);
          nrm2 = fma(static_cast<double>(v[e]), static_cast<double>(v[e]), nrm2);
        }
      } else {
        const uint4 w = xb[a * 3 + qq];  // bf16 pairs from prep_kernel
        *reinterpret_cast<uint4 *>(xs + tid * XW + 4 * qq) = w;
        const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
          nonfinite |= (wv[k] & 0x7F80u) == 0x7F80u || (wv[k] & 0x7F800000u) == 0x7F800000u;
      }
    }
    // NN-P's origin rule (pack.py:174): |x|_2 < fp32(1e-8); no scan needed
    const bool p_snap = MODE == kModeP && sqrt(nrm2) < static_cast<double>(__uint_as_float(kEpsBits));
    active = M != 0u && (lanes[0] | lanes[1] | lanes[2] | lanes[3] | lanes[4]) != 0u && !p_snap && !nonfinite;
  }
  Ms[tid] = M;

  // per-atom merge state
  uint32_t fT = kNone, fPpos = kNone, fPneg = kNone;  // NN-B
  bool pos_first = false;  // NN-B: a positive hit in the earliest pair group (then the lowest pair row is known)
  score_t best_v = -__builtin_inf();
  uint32_t best_code = kNone;
  int next = 0;  // next candidate slot: 4 * kind + lane
  const uint4 bt = bf16_value_table();
  for (;;) {
    // ---- this thread's next candidates ----
    int nm = 0;
    if (active) {
      while (next < 20 && nm < kRsPerRound) {
        const int kind = next >> 2, qq = next & 3;
        ++next;
        if ((lanes[kind] >> qq) & 1u)
          tmp[nm++ * 256 + tid] = static_cast<uint32_t>(tid) | static_cast<uint32_t>(qq) << 8 |
                                  static_cast<uint32_t>(kind != 0) << 10 | grp[kind] << 11;
      }
    }
    bool more = false;
    if (active) {
      for (int s2 = next; s2 < 20; ++s2) more |= ((lanes[s2 >> 2] >> (s2 & 3)) & 1u) != 0u;
    }

    // ---- compact: exclusive prefix sum of nm over the block ----
    int incl = nm;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int t = __shfl_up(incl, d, 64);
      if (lane >= d) incl += t;
    }
    if (lane == 63) wave_sum[wave] = incl;
    __syncthreads();
    int off = incl - nm, total = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int ws = wave_sum[w];
      if (w < wave) off += ws;
      total += ws;
    }
    for (int i = 0; i < nm; ++i) cand[off + i] = tmp[i * 256 + tid];
    __syncthreads();

    // ---- rescan: kRL lanes per candidate ----
    // Lane t of a candidate scores the 4 codes of its quarter in tiles t,
    // t + kRL, ... of the group (16 codes), then the candidate's lanes combine
    // by DPP quad moves.  Rows are monotone in sweep position within a region
    // (rising for type-3 codes and representatives, falling for antipodes,
    // and every representative row is below every antipode row), so a lane
    // tracks positions and the candidate looks its rows up once, after the
    // reduction: NN-B the lowest position at bucket M (type-3: any score;
    // pair: positive) and the highest pair position at bucket M with a
    // negative score; all modes the best value and a preference that orders
    // equal values the way their rows order and encodes the position
    // (type-3: kPrefBase - pos; pair, positive: 2^31 + kPrefBase - pos; pair,
    // negative: pos; 0: nothing compared).
    constexpr uint32_t kPrefBase = 1u << 20;  // above every sweep position
    const int n_tasks = total * kRL;           // a multiple of kRL: quads stay whole
    for (int task = tid; task < n_tasks; task += 256) {
      const int c = task / kRL, t = task % kRL;
      const uint32_t cd = cand[c];
      const int al = static_cast<int>(cd & 0xFFu), qq = static_cast<int>((cd >> 8) & 3u);
      const bool pair = ((cd >> 10) & 1u) != 0u;
      const int g = static_cast<int>(cd >> 11);
      int pos0[kRT];
#pragma unroll
      for (int j = 0; j < kRT; ++j) pos0[j] = sweep_pos(g, t + kRL * j, qq, 0);
      score_t sc[kRT][4];
      if constexpr (MODE == kModeP) {
        uint32_t rows[kRT][4];
#pragma unroll
        for (int j = 0; j < kRT; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) rows[j][e] = sw_idx[pos0[j] + e];
        double xd[kDim];
#pragma unroll
        for (int k = 0; k < kDim; ++k) xd[k] = static_cast<double>(__uint_as_float(xs[al * XW + k]));
#pragma unroll
        for (int j = 0; j < kRT; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint2 *cr = reinterpret_cast<const uint2 *>(cb_raw + static_cast<size_t>(rows[j][e]) * kDim);
            const uint2 r0 = cr[0], r1 = cr[1], r2 = cr[2];
            const uint32_t w6[6] = {r0.x, r0.y, r1.x, r1.y, r2.x, r2.y};
            double sv = 0.0;
#pragma unroll
            for (int k = 0; k < kDim; ++k) {
              const int r = static_cast<int32_t>(w6[k / 4] << (24 - 8 * (k % 4))) >> 24;
              sv = fma(xd[k], static_cast<double>(raw_value_f32(r)), sv);
            }
            sc[j][e] = sv;
          }
      } else {
        uint32_t idw[kRT][12];
#pragma unroll
        for (int j = 0; j < kRT; ++j) {
          const uint4 *q = reinterpret_cast<const uint4 *>(sw_dq + static_cast<size_t>(pos0[j]) * 3);
          const uint4 q0 = q[0], q1 = q[1], q2 = q[2];
          const uint32_t w[12] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w, q2.x, q2.y, q2.z, q2.w};
#pragma unroll
          for (int k = 0; k < 12; ++k) idw[j][k] = w[k];
        }
        const uint4 *xq = reinterpret_cast<const uint4 *>(xs + al * XW);
        const uint4 x0 = xq[0], x1 = xq[1], x2 = xq[2];
        const uint32_t xw[12] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w, x2.x, x2.y, x2.z, x2.w};
#pragma unroll
        for (int j = 0; j < kRT; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            uint32_t cw[12];
#pragma unroll
            for (int p3 = 0; p3 < 3; ++p3) {
              const uint4 o = ids_to_pairs(idw[j][3 * e + p3], bt);
              cw[4 * p3] = o.x;
              cw[4 * p3 + 1] = o.y;
              cw[4 * p3 + 2] = o.z;
              cw[4 * p3 + 3] = o.w;
            }
            float sv = 0.f;
#pragma unroll
            for (int d = 0; d < 12; ++d)
              sv = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, xw[d]), __builtin_bit_cast(bf16x2, cw[d]),
                                                   sv, false);
            sc[j][e] = sv;
          }
      }
      const uint32_t Mk = Ms[al];
      uint32_t p_lo = kNone, bpref = 0u, p_hi = 0u;  // p_hi: highest negative-hit position + 1
      score_t bv = -__builtin_inf();
#pragma unroll
      for (int j = 0; j < kRT; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t pos = static_cast<uint32_t>(pos0[j] + e);
          const bool neg = pair && sc[j][e] < static_cast<score_t>(0);
          score_t v = neg ? -sc[j][e] : sc[j][e];
          const uint32_t pref = !pair ? kPrefBase - pos : neg ? pos : 0x80000000u + kPrefBase - pos;
          if constexpr (B) {
            const uint32_t bk = bf16_rne_bits(static_cast<float>(sc[j][e]));
            if (bk == Mk) p_lo = min(p_lo, pos);
            if (pair && bk == (Mk | 0x8000u)) p_hi = max(p_hi, pos + 1u);
            v = bf16_bits_to_float(bf16_rne_bits(static_cast<float>(v)));
          }
          if (v > bv || (v == bv && pref > bpref)) {
            bv = v;
            bpref = pref;
          }
        }
      // combine the candidate's kRL = 4 lanes (one quad): xor 1, then xor 2
      auto step = [&](auto ctrl) {
        constexpr int C = decltype(ctrl)::value;
        const uint32_t opref = dpp_u32<C>(bpref);
        score_t ov;
        if constexpr (MODE == kModeP) {
          const uint64_t b = static_cast<uint64_t>(__double_as_longlong(bv));
          const uint64_t o = static_cast<uint64_t>(dpp_u32<C>(static_cast<uint32_t>(b))) |
                             static_cast<uint64_t>(dpp_u32<C>(static_cast<uint32_t>(b >> 32))) << 32;
          ov = __longlong_as_double(static_cast<long long>(o));
        } else {
          ov = dpp_f32<C>(bv);
        }
        if (ov > bv || (ov == bv && opref > bpref)) {
          bv = ov;
          bpref = opref;
        }
        if constexpr (B) {
          p_lo = min(p_lo, dpp_u32<C>(p_lo));
          p_hi = max(p_hi, dpp_u32<C>(p_hi));
        }
      };
      step(std::integral_constant<int, 0xB1>{});
      step(std::integral_constant<int, 0x4E>{});
      if (t == 0) {
        const uint32_t bpos = !pair ? kPrefBase - bpref : bpref < 0x80000000u ? bpref : 0x80000000u + kPrefBase - bpref;
        res_v[c] = bv;
        res_c[c] = bpref == 0u ? kNone : pair && bpref < 0x80000000u ? sw_anti[bpos - kType3Codes] : sw_idx[bpos];
        if constexpr (B) {
          res_f0[c] = p_lo == kNone ? kNone : sw_idx[p_lo];
          res_f1[c] = p_hi == 0u ? kNone : sw_anti[p_hi - 1u - kType3Codes];
        }
      }
    }
    __syncthreads();

    // ---- merge this thread's candidates ----
    for (int i = 0; i < nm; ++i) {
      const score_t v = res_v[off + i];
      const uint32_t code = res_c[off + i];
      if (v > best_v || (v == best_v && code < best_code)) {
        best_v = v;
        best_code = code;
      }
      if constexpr (B) {
        if (((cand[off + i] >> 10) & 1u) == 0u) {
          fT = min(fT, res_f0[off + i]);
        } else {
          fPpos = min(fPpos, res_f0[off + i]);
          fPneg = min(fPneg, res_f1[off + i]);
          pos_first |= (cand[off + i] >> 11) == span_g0 && res_f0[off + i] != kNone;
        }
      }
    }
    if (!__syncthreads_or(more)) break;
  }

  uint32_t fS = kNone;  // NN-B: the lowest winning pair-code row
  if constexpr (B) {
    // ---- span rescan for atoms whose first pair group has only negative hits ----
    // (rare: some group at the best pair bucket is not among the candidates)
    // The block steps through the span in ascending chunks of kSpanChunk
    // codes, kSpanChunk / 256 per thread with all their loads (the codes' bf16
    // planes from the sweep tiles) issued first, and stops at the first chunk
    // holding a positive hit: the lowest of that chunk's hits (an LDS atomic
    // min) is the lowest positive row, since every earlier chunk had none.
    const bool span = active && many && !pos_first && span_g1 > span_g0;
    if (span) {
      const uint32_t slot = atomicAdd(&span_n, 1u);
      span_list[slot] = static_cast<uint32_t>(tid);
      span_lo[slot] = (span_g0 + 1u) * kG * kTileCodes;
      span_cnt[slot] = (span_g1 - span_g0) * kG * kTileCodes;
      span_min[slot] = kNone;
    }
    __syncthreads();
    const int n_span = static_cast<int>(span_n);
    constexpr int kSpanPer = 8;  // codes per thread per chunk
    for (int si = 0; si < n_span; ++si) {
      const int al = static_cast<int>(span_list[si]);
      const uint32_t lo = span_lo[si], cnt = span_cnt[si];
      const uint32_t Mk = Ms[al];
      const uint4 *xq = reinterpret_cast<const uint4 *>(xs + al * XW);
      const uint4 x0 = xq[0], x1 = xq[1], x2 = xq[2];
      const uint32_t xw[12] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w, x2.x, x2.y, x2.z, x2.w};
      for (uint32_t base = 0; base < cnt; base += 256u * kSpanPer) {
        uint4 pl[kSpanPer][3];
#pragma unroll
        for (int u = 0; u < kSpanPer; ++u) {
          const uint32_t w = base + static_cast<uint32_t>(u) * 256u + static_cast<uint32_t>(tid);
          const uint32_t pos = lo + (w < cnt ? w : 0u);
          const uint8_t *tb = sw_tiles + static_cast<size_t>(pos / kTileCodes) * kTileBytes + (pos % kTileCodes) * 16;
#pragma unroll
          for (int p3 = 0; p3 < 3; ++p3) pl[u][p3] = *reinterpret_cast<const uint4 *>(tb + p3 * 256);
        }
        uint32_t mine = kNone;
#pragma unroll
        for (int u = 0; u < kSpanPer; ++u) {
          const uint32_t w = base + static_cast<uint32_t>(u) * 256u + static_cast<uint32_t>(tid);
          const uint32_t cw[12] = {pl[u][0].x, pl[u][0].y, pl[u][0].z, pl[u][0].w, pl[u][1].x, pl[u][1].y,
                                   pl[u][1].z, pl[u][1].w, pl[u][2].x, pl[u][2].y, pl[u][2].z, pl[u][2].w};
          float sc2 = 0.f;
#pragma unroll
          for (int d = 0; d < 12; ++d)
            sc2 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, xw[d]), __builtin_bit_cast(bf16x2, cw[d]),
                                                  sc2, false);
          if (w < cnt && bf16_rne_bits(sc2) == Mk) {
            const uint32_t row = sw_idx[lo + w];
            if (row != 0u) mine = min(mine, row);
          }
        }
        if (mine != kNone) atomicMin(&span_min[si], mine);
        if (__syncthreads_or(mine != kNone)) break;
      }
      __syncthreads();
      if (tid == al) fPpos = min(fPpos, span_min[si]);
    }
    fS = fPpos != kNone ? fPpos : fPneg;
  }

  int32_t id = 0;
  if (active) {
    bool snap;
    uint32_t row;
    if (MODE == kModeP) {
      row = best_code;
      snap = best_code == kNone;  // non-finite atom: no score compared
    } else if (B) {
      const uint32_t found = min(fT, fS);
      const uint32_t bucket = found != kNone ? M : (__float_as_uint(static_cast<float>(best_v)) >> 16);
      row = found != kNone ? found : best_code;
      // bf16 max below 2.0
      snap = (found == kNone && !(best_v > 0.f)) || bucket < 0x4000u;
    } else {
      row = best_code;
      snap = !(2.0f * static_cast<float>(best_v) >= __uint_as_float(kCSqNormBits));
    }
    id = snap || row == kNone ? 0 : static_cast<int32_t>(row);
  }
  if (idx_out && a < n_atoms) idx_out[a] = id;
  if (!packed_out) return;
  ids[tid] = id;
  __syncthreads();
  store_packed_block(ids, bytes, a0, n_atoms, packed_out, tid);
}

// NN-B with the structured scorers: the higher of the pair key (t12_kernel)
// and the type-3 key (t3_kernel), the lower row on equal buckets, the origin
// when neither reaches 2.0 or the atom has a NaN or infinite coordinate; then
// the int32 index and, optionally, the packed 9-byte groups.
__global__ __launch_bounds__(256) void pick_kernel(const uint4 *__restrict__ keys, int64_t n_atoms,
                                                   int32_t *__restrict__ idx_out, uint8_t *__restrict__ packed_out) {
  __shared__ int32_t ids[256];
  __shared__ __align__(16) uint8_t bytes[64 * 9];
  const int tid = threadIdx.x;
  const int64_t a0 = static_cast<int64_t>(blockIdx.x) * 256;
  const int64_t a = a0 + tid;
  int32_t id = 0;
  if (a < n_atoms) {
    const uint4 k = keys[a];
    const uint32_t M3 = k.x >> 16, M2 = k.z >> 16, M = max(M2, M3);
    uint32_t row = kNone;
    if (M >= 0x4000u && k.z != kNonFinite) {  // (a non-finite atom: the origin)
      if (M3 == M) row = k.y;
      if (M2 == M) row = min(row, k.w);
    }
    id = row == kNone ? 0 : static_cast<int32_t>(row);
    if (idx_out) idx_out[a] = id;
  }
  if (!packed_out) return;
  ids[tid] = id;
  __syncthreads();
  store_packed_block(ids, bytes, a0, n_atoms, packed_out, tid);
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

// Codebook slices per launch.  One slice when the atom blocks alone give
// every CU slot several waves of work-groups (>= 6144 blocks): each atom's
// planes are read once and the longer sweep per block amortises its set-up
// and flushes (measured on 16.8M atoms: 84.3 ms with 1 slice, 87.2 with 2,
// 89.4 with 4, identical indices).  Smaller launches double the slice count
// until the grid reaches that size, up to 32 (9216 tiles / 32 = 9 whole
// stages per slice).
int choose_slices(int64_t ablocks) {
  int s = 1;
  while (s < 32 && ablocks * s < 6144) s *= 2;
  return s;
}
static_assert(kSweepTiles % (32 * kST) == 0, "every slice count holds whole stages");
static_assert(kType3Tiles % kST == 0, "the pair region starts on a stage boundary");

// per-atom key slots: 16 bytes (NN-B dense sweep: the type-3 key; NN-B
// structured: the type-3 key (t3_kernel), then the pair key (t12_kernel);
// NN-T / NN-P: type-3 and pair keys of 64 bits)
size_t keys_bytes(int64_t n_atoms) { return (static_cast<size_t>(n_atoms) * 16 + 255) & ~static_cast<size_t>(255); }

// First slice holding pair tiles, for a launch of n_slices slices.
int first_pair_slice(int n_slices) { return kType3Tiles / (kSweepTiles / n_slices); }

// NN-B pair records of the dense sweep: 8 bytes per (atom, slice holding pair
// tiles), sized for every slice
size_t recs_bytes(int64_t n_atoms) {
  const int64_t ablocks = (n_atoms + kAtomsPerBlock - 1) / kAtomsPerBlock;
  const int n_slices = choose_slices(ablocks);
  return (static_cast<size_t>(n_atoms) * static_cast<size_t>(n_slices) * 8 + 255) & ~static_cast<size_t>(255);
}

// t3_kernel: atom tiles per wave by launch size, so small launches still fill the chip.
int t3_launch(const uint4 *xb, int64_t n_atoms, const DeviceTables *tab, uint4 *keys, const uint2 *rec,
              hipStream_t s, int rows_by_sweep) {
  // 4 atom tiles per wave from 131,072 atoms, 2 from 98,304, else 1 (measured per launch size: 55,296
  // atoms take 35 + 42 us in t12 + t3 at 1 tile, 39 + 47 at 2; from 165,888 atoms 4 tiles are fastest).
  // At 4 tiles: 40 KB of LDS (16-tile stages) and 128 VGPRs, 4 blocks (16 waves) per CU, which the
  // kernel's stalls need (8 tiles per wave at 2 blocks per CU was 30% slower); the representative words
  // and, when a list is worked, the atoms' coordinates are read from global memory (L1 / L2) to leave
  // the LDS to the stages and lists.
  const int AT = n_atoms >= 131072 ? 4 : n_atoms >= 98304 ? 2 : 1;
  const int64_t per_block = static_cast<int64_t>(kWaves) * AT * 16;
  const int64_t blocks = (n_atoms + per_block - 1) / per_block;
  if (blocks > 0x7FFFFFFFll) return fail(PLX_EINVAL, "quantize: %lld atoms exceed one launch", static_cast<long long>(n_atoms));
  const dim3 g(static_cast<unsigned>(blocks));
  profile_before(s, PLX_PROF_T3);
  if (AT == 4)
    hipLaunchKernelGGL(t3_kernel<4>, g, dim3(kThreads), 0, s, xb, n_atoms, tab->t3_tiles, tab->t3_words, tab->t3_rows,
                       keys, rec, rows_by_sweep);
  else if (AT == 2)
    hipLaunchKernelGGL(t3_kernel<2>, g, dim3(kThreads), 0, s, xb, n_atoms, tab->t3_tiles, tab->t3_words, tab->t3_rows,
                       keys, rec, rows_by_sweep);
  else
    hipLaunchKernelGGL(t3_kernel<1>, g, dim3(kThreads), 0, s, xb, n_atoms, tab->t3_tiles, tab->t3_words, tab->t3_rows,
                       keys, rec, rows_by_sweep);
  profile_after(s, PLX_PROF_T3);
  return check_launch("t3_kernel");
}

// t12_kernel: atom tiles per wave by launch size, as t3_kernel (38 KB of LDS at 4 tiles per wave).
template <int LOAD>
int t12_launch_load(uint4 *xb, const float *src, const float *sigma, int64_t apr, int64_t n_atoms,
                    const DeviceTables *tab, uint4 *keys, uint2 *rec, hipStream_t s, int rows_by_sweep) {
  const int AT = n_atoms >= 131072 ? 4 : n_atoms >= 98304 ? 2 : 1;
  const int64_t per_block = static_cast<int64_t>(kWaves) * AT * 16;
  const int64_t blocks = (n_atoms + per_block - 1) / per_block;
  if (blocks > 0x7FFFFFFFll) return fail(PLX_EINVAL, "quantize: %lld atoms exceed one launch", static_cast<long long>(n_atoms));
  const dim3 g(static_cast<unsigned>(blocks));
  profile_before(s, PLX_PROF_T12);
  if (AT == 4)
    hipLaunchKernelGGL((t12_kernel<4, LOAD>), g, dim3(kThreads), 0, s, xb, src, sigma, apr, n_atoms, tab->t2_tiles,
                       tab->t2_pos, tab->t2_rows, tab->t1_rows, tab->t2_steiner, tab->t3_dec, keys, rec, rows_by_sweep);
  else if (AT == 2)
    hipLaunchKernelGGL((t12_kernel<2, LOAD>), g, dim3(kThreads), 0, s, xb, src, sigma, apr, n_atoms, tab->t2_tiles,
                       tab->t2_pos, tab->t2_rows, tab->t1_rows, tab->t2_steiner, tab->t3_dec, keys, rec, rows_by_sweep);
  else
    hipLaunchKernelGGL((t12_kernel<1, LOAD>), g, dim3(kThreads), 0, s, xb, src, sigma, apr, n_atoms, tab->t2_tiles,
                       tab->t2_pos, tab->t2_rows, tab->t1_rows, tab->t2_steiner, tab->t3_dec, keys, rec, rows_by_sweep);
  profile_after(s, PLX_PROF_T12);
  return check_launch("t12_kernel");
}

// The structured NN-B path: t12_kernel (types 1-2; LOAD 1 / 2: it also rounds the atoms into xb, so no
// prep_kernel runs), t3_kernel (type 3), pick_kernel.  Every atom's key halves are written by the two
// scorers, so the keys need no clearing.
template <int LOAD>
int structured_launch(uint4 *xb, const float *src, const float *sigma, int64_t apr, int64_t n_atoms,
                      const DeviceTables *tab, uint4 *keys, uint2 *rec, int32_t *idx_out, uint8_t *packed_out,
                      hipStream_t s, int rows_by_sweep) {
  int st;
  if ((st = t12_launch_load<LOAD>(xb, src, sigma, apr, n_atoms, tab, keys, rec, s, rows_by_sweep)) != PLX_OK)
    return st;
  if ((st = t3_launch(xb, n_atoms, tab, keys, rec, s, rows_by_sweep)) != PLX_OK) return st;
  hipLaunchKernelGGL(pick_kernel, dim3(static_cast<unsigned>((n_atoms + 255) / 256)), dim3(256), 0, s, keys, n_atoms,
                     idx_out, packed_out);
  return check_launch("pick_kernel");
}

// workspace = per-atom keys, the NN-B pair records, then (NN-B / NN-T) the bf16 planes.
// STRUCT (NN-B): the structured scorers (t12_kernel, t3_kernel, pick_kernel);
// otherwise every sweep code is scored densely (nn_kernel, resolve_kernel).
template <int MODE, bool FUSED, bool STRUCT = false>
int launch_mode(const float *x, const float *sigma, int64_t apr, int64_t n_atoms, const DeviceTables *tab,
                int32_t *idx_out, uint8_t *packed_out, uint8_t *workspace, hipStream_t s, int rows_by_sweep = 0) {
  static_assert(!STRUCT || MODE == kModeB, "the structured scorers have NN-B semantics");
  const int64_t ablocks = (n_atoms + kAtomsPerBlock - 1) / kAtomsPerBlock;
  const int n_slices = choose_slices(ablocks);
  const int tiles_per_slice = kSweepTiles / n_slices;
  const int64_t grid = ablocks * n_slices;
  if (grid > 0x7FFFFFFFll) return fail(PLX_EINVAL, "quantize: %lld atoms exceed one launch", static_cast<long long>(n_atoms));
  uint4 *keys = reinterpret_cast<uint4 *>(workspace);
  uint64_t *recs = reinterpret_cast<uint64_t *>(workspace + keys_bytes(n_atoms));
  uint4 *xb = reinterpret_cast<uint4 *>(workspace + keys_bytes(n_atoms) + recs_bytes(n_atoms));
  const int s0 = first_pair_slice(n_slices);
  if constexpr (STRUCT)
    return structured_launch<FUSED ? 2 : 1>(xb, x, sigma, apr, n_atoms, tab, keys, reinterpret_cast<uint2 *>(recs),
                                            idx_out, packed_out, s, rows_by_sweep);
  int st;
  if (MODE != kModeP) {
    hipLaunchKernelGGL((prep_kernel<FUSED>), dim3(static_cast<unsigned>((n_atoms * 3 + 255) / 256)), dim3(256), 0, s, x,
                       sigma, apr, n_atoms, xb, keys);
    if ((st = check_launch("prep_kernel")) != PLX_OK) return st;
  } else {
    hipLaunchKernelGGL(clear_keys_kernel, dim3(static_cast<unsigned>((n_atoms + 255) / 256)), dim3(256), 0, s, keys,
                       n_atoms);
    if ((st = check_launch("clear_keys_kernel")) != PLX_OK) return st;
  }
  profile_before(s);
  const uint8_t *tiles = MODE == kModeP ? tab->sw_raw_tiles : tab->sw_bf16_tiles;
  const void *operand = MODE == kModeP ? static_cast<const void *>(x) : static_cast<const void *>(xb);
  hipLaunchKernelGGL((nn_kernel<MODE>), dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s, operand, n_atoms, tiles,
                     n_slices, tiles_per_slice, keys, recs, s0);
  if ((st = check_launch("nn_kernel")) != PLX_OK) return st;
  profile_after(s);
  hipLaunchKernelGGL((resolve_kernel<MODE, FUSED>), dim3(static_cast<unsigned>((n_atoms + 255) / 256)), dim3(256), 0, s,
                     keys, n_atoms, x, sigma, apr, xb, tab->sw_dq, tab->sw_idx, tab->sw_anti, tab->cb_raw,
                     tab->sw_bf16_tiles, static_cast<const uint64_t *>(recs), n_slices - s0, n_atoms, idx_out,
                     packed_out);
  return check_launch("resolve_kernel");
}

}  // namespace

size_t quantize_workspace_bytes(int64_t n_atoms) {
  if (n_atoms <= 0) return 0;
  return keys_bytes(n_atoms) + recs_bytes(n_atoms) + static_cast<size_t>(n_atoms) * 48;
}

int check_quantize_args(const float *x, int64_t n_atoms, const void *workspace, size_t workspace_bytes) {
  if (n_atoms <= 0) return PLX_OK;
  if (workspace == nullptr || workspace_bytes < quantize_workspace_bytes(n_atoms))
    return fail(PLX_EINVAL, "quantize: workspace of %zu bytes is smaller than the %zu needed for %lld atoms",
                workspace_bytes, quantize_workspace_bytes(n_atoms), static_cast<long long>(n_atoms));
  if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0 || (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0)
    return fail(PLX_EINVAL, "quantize: input and workspace must be 16-byte aligned");
  const int64_t ablocks = (n_atoms + kAtomsPerBlock - 1) / kAtomsPerBlock;
  if (ablocks * choose_slices(ablocks) > 0x7FFFFFFFll || (n_atoms * 6 + 255) / 256 > 0x7FFFFFFFll)
    return fail(PLX_EINVAL, "quantize: %lld atoms exceed one launch", static_cast<long long>(n_atoms));
  return PLX_OK;
}

int launch_quantize(const float *x, const float *sigma, int64_t rows, int64_t cols, int64_t n_atoms, int mode,
                    int32_t *idx_out, uint8_t *packed_out, float *weight_out, void *workspace,
                    size_t workspace_bytes, hipStream_t s) {
  (void)rows;
  if (n_atoms <= 0) return PLX_OK;
  int st = check_quantize_args(x, n_atoms, workspace, workspace_bytes);
  if (st != PLX_OK) return st;
  const DeviceTables *tab = nullptr;
  st = get_tables(&tab);
  if (st != PLX_OK) return st;
  uint8_t *ws = static_cast<uint8_t *>(workspace);
  const bool fused = sigma != nullptr;
  const int64_t apr = cols / kDim;
  const bool dense = (mode & PLX_NN_DENSE_TYPE3) != 0;
  const int rows_by_sweep = (mode & PLX_NN_T3_ROWS_BY_SWEEP) != 0 ? 1 : 0;
  mode &= ~(PLX_NN_DENSE_TYPE3 | PLX_NN_T3_ROWS_BY_SWEEP);
  if (mode == PLX_NN_PACK_FP32)
    st = launch_mode<PLX_NN_PACK_FP32, false>(x, nullptr, apr, n_atoms, tab, idx_out, packed_out, ws, s);
  else if (mode == PLX_NN_BF16_SCORES && !dense)
    st = fused ? launch_mode<PLX_NN_BF16_SCORES, true, true>(x, sigma, apr, n_atoms, tab, idx_out, packed_out, ws, s,
                                                             rows_by_sweep)
               : launch_mode<PLX_NN_BF16_SCORES, false, true>(x, sigma, apr, n_atoms, tab, idx_out, packed_out, ws, s,
                                                              rows_by_sweep);
  else if (mode == PLX_NN_BF16_SCORES)
    st = fused ? launch_mode<PLX_NN_BF16_SCORES, true>(x, sigma, apr, n_atoms, tab, idx_out, packed_out, ws, s)
               : launch_mode<PLX_NN_BF16_SCORES, false>(x, sigma, apr, n_atoms, tab, idx_out, packed_out, ws, s);
  else
    st = fused ? launch_mode<PLX_NN_FP32_SCORES, true>(x, sigma, apr, n_atoms, tab, idx_out, packed_out, ws, s)
               : launch_mode<PLX_NN_FP32_SCORES, false>(x, sigma, apr, n_atoms, tab, idx_out, packed_out, ws, s);
  if (st != PLX_OK) return st;
  if (weight_out) {
    const dim3 gg(static_cast<unsigned>((n_atoms * 6 + 255) / 256));
    hipLaunchKernelGGL((gather_kernel<0, true>), gg, dim3(256), 0, s, idx_out, n_atoms, tab->cb_raw, sigma, apr,
                       static_cast<void *>(weight_out));
    if ((st = check_launch("gather_kernel")) != PLX_OK) return st;
  }
  return PLX_OK;
}

namespace {

// Several latents in one scoring pass: row scale and operand planes per
// matrix, one launch of the scorers over all their atoms (STRUCT: t12_kernel
// and t3_kernel; otherwise nn_kernel with fewer codebook slices per atom
// block; no per-matrix tail of the grid either way), then per matrix the
// index + pack (pick_kernel / resolve_kernel) and the scaled gather of the
// reconstructed weight.
template <int MODE, bool STRUCT = false>
int launch_batch_mode(const RequantItem *items, int n_items, const DeviceTables *tab, uint8_t *workspace,
                      hipStream_t s) {
  static_assert(!STRUCT || MODE == kModeB, "the structured scorers have NN-B semantics");
  int64_t total = 0;
  for (int i = 0; i < n_items; ++i) total += items[i].rows * (items[i].cols / kDim);
  if (total == 0) return PLX_OK;
  const int64_t ablocks = (total + kAtomsPerBlock - 1) / kAtomsPerBlock;
  const int n_slices = choose_slices(ablocks);
  const int tiles_per_slice = kSweepTiles / n_slices;
  const int64_t grid = ablocks * n_slices;
  if (grid > 0x7FFFFFFFll) return fail(PLX_EINVAL, "requantize_batch: %lld atoms exceed one launch", static_cast<long long>(total));
  uint4 *keys = reinterpret_cast<uint4 *>(workspace);
  uint64_t *recs = reinterpret_cast<uint64_t *>(workspace + keys_bytes(total));
  uint4 *xb = reinterpret_cast<uint4 *>(workspace + keys_bytes(total) + recs_bytes(total));
  const int s0 = first_pair_slice(n_slices);
  int st;
  int64_t off = 0;
  for (int i = 0; i < n_items; ++i) {
    const RequantItem &it = items[i];
    const int64_t apr = it.cols / kDim, n = it.rows * apr;
    if (n == 0) continue;
    if ((st = launch_row_rms(it.latent, it.rows, it.cols, it.sigma, nullptr, s)) != PLX_OK) return st;
    hipLaunchKernelGGL((prep_kernel<true>), dim3(static_cast<unsigned>((n * 3 + 255) / 256)), dim3(256), 0, s, it.latent,
                       it.sigma, apr, n, xb + off * 3, keys + off);
    if ((st = check_launch("prep_kernel")) != PLX_OK) return st;
    off += n;
  }
  if constexpr (STRUCT) {
    if ((st = t12_launch_load<0>(xb, nullptr, nullptr, 1, total, tab, keys, reinterpret_cast<uint2 *>(recs), s, 0)) !=
        PLX_OK)
      return st;
    if ((st = t3_launch(xb, total, tab, keys, reinterpret_cast<const uint2 *>(recs), s, 0)) != PLX_OK) return st;
  } else {
    profile_before(s);
    hipLaunchKernelGGL((nn_kernel<MODE>), dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s,
                       static_cast<const void *>(xb), total, tab->sw_bf16_tiles, n_slices, tiles_per_slice, keys, recs,
                       s0);
    if ((st = check_launch("nn_kernel")) != PLX_OK) return st;
    profile_after(s);
  }
  off = 0;
  for (int i = 0; i < n_items; ++i) {
    const RequantItem &it = items[i];
    const int64_t apr = it.cols / kDim, n = it.rows * apr;
    if (n == 0) continue;
    if constexpr (STRUCT) {
      hipLaunchKernelGGL(pick_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, keys + off, n,
                         it.idx, it.packed);
      if ((st = check_launch("pick_kernel")) != PLX_OK) return st;
    } else {
      hipLaunchKernelGGL((resolve_kernel<MODE, true>), dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
                         keys + off, n, it.latent, it.sigma, apr, xb + off * 3, tab->sw_dq, tab->sw_idx, tab->sw_anti,
                         tab->cb_raw, tab->sw_bf16_tiles, static_cast<const uint64_t *>(recs + off), n_slices - s0,
                         total, it.idx, it.packed);
      if ((st = check_launch("resolve_kernel")) != PLX_OK) return st;
    }
    if (it.weight) {
      hipLaunchKernelGGL((gather_kernel<0, true>), dim3(static_cast<unsigned>((n * 6 + 255) / 256)), dim3(256), 0, s,
                         it.idx, n, tab->cb_raw, it.sigma, apr, static_cast<void *>(it.weight));
      if ((st = check_launch("gather_kernel")) != PLX_OK) return st;
    }
    off += n;
  }
  return PLX_OK;
}

}  // namespace

int launch_requantize_batch(const RequantItem *items, int n_items, int mode, void *workspace, size_t workspace_bytes,
                            hipStream_t s) {
  int64_t total = 0;
  for (int i = 0; i < n_items; ++i) total += items[i].rows * (items[i].cols / kDim);
  if (total == 0) return PLX_OK;
  if (workspace == nullptr || workspace_bytes < quantize_workspace_bytes(total))
    return fail(PLX_EINVAL, "requantize_batch: workspace of %zu bytes is smaller than the %zu needed for %lld atoms",
                workspace_bytes, quantize_workspace_bytes(total), static_cast<long long>(total));
  if ((reinterpret_cast<uintptr_t>(workspace) & 15u) != 0) return fail(PLX_EINVAL, "requantize_batch: workspace must be 16-byte aligned");
  for (int i = 0; i < n_items; ++i)
    if ((reinterpret_cast<uintptr_t>(items[i].latent) & 15u) != 0)
      return fail(PLX_EINVAL, "requantize_batch: latent %d must be 16-byte aligned", i);
  const DeviceTables *tab = nullptr;
  int st = get_tables(&tab);
  if (st != PLX_OK) return st;
  uint8_t *ws = static_cast<uint8_t *>(workspace);
  const bool dense = (mode & PLX_NN_DENSE_TYPE3) != 0;
  mode &= ~(PLX_NN_DENSE_TYPE3 | PLX_NN_T3_ROWS_BY_SWEEP);
  if (mode == PLX_NN_BF16_SCORES)
    return dense ? launch_batch_mode<PLX_NN_BF16_SCORES>(items, n_items, tab, ws, s)
                 : launch_batch_mode<PLX_NN_BF16_SCORES, true>(items, n_items, tab, ws, s);
  return launch_batch_mode<PLX_NN_FP32_SCORES>(items, n_items, tab, ws, s);
}

// ---- allocation-free requantize (plx_requantize_noalloc) ----
// The workspace of up to PLX_NOALLOC_MAX_ATOMS atoms (per-atom keys, then the
// bf16 operand planes) as one file-scope device array, held by every device
// the library runs on until the process ends.  In host code `scratch` names a
// host-side stand-in: its device address comes from hipGetSymbolAddress, once
// per device, and only that address is passed to kernels.  Every call on a
// device shares its array; prep_kernel clears the keys each call, so a call
// needs nothing from the previous one, but calls that overlap on one device
// (different streams at once) race on it.
static_assert(PLX_NOALLOC_MAX_ATOMS > 0, "maximum atoms of the allocation-free entry point");
// (at 2^20 atoms a launch uses 8 slices, with pair-record slots for each: 16 B
// of keys + 8 x 8 B of pair records + 48 B of operand planes per atom, the
// largest workspace of any size up to the maximum, plus the 256-byte rounding
// of its three parts; checked on every call)
constexpr size_t kScratchBytes = static_cast<size_t>(PLX_NOALLOC_MAX_ATOMS) * (16 + 8 * 8 + 48) + 1024;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
void *g_scratch[64] = {};  // per device: the address of `scratch`
}  // namespace

int noalloc_setup() {
  int dev = 0;
  int st = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (st != PLX_OK) return st;
  if (dev < 0 || dev >= 64) return fail(PLX_EINVAL, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] != nullptr) return PLX_OK;
  void *p = nullptr;
  st = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  if (st != PLX_OK) return st;
  if (p == nullptr || (reinterpret_cast<uintptr_t>(p) & 255u) != 0)
    return fail(PLX_EHIP, "the scratch array of device %d has no usable device address", dev);
  g_scratch[dev] = p;
  return PLX_OK;
}

int launch_requantize_noalloc(const float *latent, int64_t rows, int64_t cols, int mode, float *sigma_out,
                              int32_t *idx_out, uint8_t *packed_out, float *weight_out, hipStream_t s) {
  const int64_t n_atoms = rows * (cols / kDim);
  if (n_atoms > PLX_NOALLOC_MAX_ATOMS)
    return fail(PLX_EINVAL, "plx_requantize_noalloc: %lld atoms exceed its maximum of %d (use plx_requantize)",
                static_cast<long long>(n_atoms), PLX_NOALLOC_MAX_ATOMS);
  const DeviceTables *tab = nullptr;
  int st = get_tables_built(&tab);  // never builds (allocates) them here
  if (st != PLX_OK) return st;
  int dev = 0;
  if ((st = check_hip(hipGetDevice(&dev), "hipGetDevice")) != PLX_OK) return st;
  void *ws = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ws = g_scratch[dev];
  }
  if (ws == nullptr)
    return fail(PLX_EINVAL, "plx_requantize_noalloc: call plx_device_init() on device %d first", dev);
  // every argument check before the first launch: a refused call writes nothing
  if ((st = check_quantize_args(latent, n_atoms, ws, kScratchBytes)) != PLX_OK) return st;
  if ((st = launch_row_rms(latent, rows, cols, sigma_out, nullptr, s)) != PLX_OK) return st;
  return launch_quantize(latent, sigma_out, rows, cols, n_atoms, mode, idx_out, packed_out, weight_out, ws,
                         kScratchBytes, s);
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

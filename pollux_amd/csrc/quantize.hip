// Leech nearest-neighbour quantizer on CDNA4 MFMA (replaces castor.py:374-560).
//
// Scores x.c of every atom against all 196,560 kissing points as a dense bf16
// contraction on v_mfma_f32_16x16x32_bf16 (K = 24 coordinates + 8 zero pad),
// keeping only a running maximum per (atom, lane) and the index of the code
// group where it was reached; no score is ever written to memory.
//
// nn_kernel -- the scoring sweep.
//   grid.x = atom_blocks * n_slices; block b works on atom block b / n_slices
//   and codebook slice b % n_slices.  Work-groups are dispatched round-robin
//   over the 8 XCDs, so with 8 slices each XCD only ever streams its own
//   1.18 MB of the 9.4 MB bf16 codebook and serves it from its 4 MB L2.
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
//   mask to find the lowest code, kG lanes per (group, lane) with coalesced
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
// Also clears the atoms' 8-byte key slots (keys8 may hold 32-bit keys in its
// first half: NN-B), before nn_kernel merges its slices into them.
template <bool FUSED>
__global__ __launch_bounds__(256) void prep_kernel(const float *__restrict__ src, const float *__restrict__ sigma,
                                                   int64_t atoms_per_row, int64_t n_atoms, uint4 *__restrict__ xb,
                                                   uint2 *__restrict__ keys8) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // plane i % 3 of atom i / 3
  if (i >= n_atoms * 3) return;
  const int64_t a = i / 3;
  if (i == 3 * a) keys8[a] = make_uint2(0u, 0u);
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
__global__ __launch_bounds__(256) void clear_keys_kernel(uint2 *__restrict__ keys8, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) keys8[i] = make_uint2(0u, 0u);
}

// NN-B tracking key of a group: bucket (round-half-up, see raised_threshold)
// in the high half, 0xFFFF - group in the low half, so one signed max keeps
// the highest bucket and, within it, the earliest group.
// v_perm_b32 takes bytes 2-3 of the rounded score and bytes 0-1 of the
// (uniform) group field in one instruction.
__device__ __forceinline__ int group_key(int gm, int group) {
  return static_cast<int>(__builtin_amdgcn_perm(static_cast<uint32_t>(gm) + 0x8000u,
                                                static_cast<uint32_t>(0xFFFF - group) & 0xFFFFu, 0x07060100u));
}

// src: NN-P: the fp32 atoms; NN-B / NN-T: xb, the bf16 planes of prep_kernel.
template <int MODE>
__global__ __launch_bounds__(kThreads, 2) void nn_kernel(const void *__restrict__ src, int64_t n_atoms,
                                                          const uint8_t *__restrict__ tiles, int n_slices,
                                                          int tiles_per_slice, void *__restrict__ keys) {
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

  int R[kAT], best[kAT];
#pragma unroll
  for (int at = 0; at < kAT; ++at) {
    R[at] = initial_threshold<MODE>();
    best[at] = -1;
  }

  const int t0 = slice * tiles_per_slice;
  const int n_stages = tiles_per_slice / kST;
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
  // Software pipeline: the MFMA result of tile k for atom tile `at` is folded
  // into the group maximum while tile k+1's MFMAs issue, and tile k+1's A
  // operand is read from LDS right after tile k's first MFMA.  A group of kG
  // tiles is compared against the threshold once its last tile has been
  // folded, i.e. during the next group's first tile (NN-B: the next group's
  // tile at % 8); the slice's last tile is folded after the loop.
  int gm[kAT];
  f32x4 acc[kAT], part[kAT];
#pragma unroll
  for (int at = 0; at < kAT; ++at) {
    gm[at] = INT_MIN;
    acc[at] = f32x4{-0.f, -0.f, -0.f, -0.f};  // INT_MIN bit patterns: neutral for the fold
  }
  int group_prev = -1;  // global id of the group whose compare is pending
  for (int st = 0; st < n_stages; ++st) {
    const int buf = st & 1;
    if (st + 1 < n_stages) stage_copy(st + 1, buf ^ 1);
    const uint8_t *L = lds[buf] + a_off;
    bf16x8 a = *reinterpret_cast<const bf16x8 *>(L);
    bool up[kAT];
    int gdone[kAT];
    // One group of kG tiles: tile 0 closes the previous group, tile 1 starts
    // this group's maximum.
    auto group_tiles = [&](int k0) {
      constexpr bool FIRST = true;
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
          if (FIRST && t == 1) {
            m = max(max(__float_as_int(acc[at][0]), __float_as_int(acc[at][1])), __float_as_int(acc[at][2]));
            m = max(m, __float_as_int(acc[at][3]));
          } else {
            m = max(max(gm[at], __float_as_int(acc[at][0])), __float_as_int(acc[at][1]));
            m = max(max(m, __float_as_int(acc[at][2])), __float_as_int(acc[at][3]));
          }
          // The empty asm pins the fold next to this MFMA (IR passes would
          // otherwise sink the chain to the group end) and the sched_barrier
          // stops the machine scheduler from hoisting every MFMA, so the
          // matrix pipe and the VALU work in parallel.
          asm volatile("" : "+v"(m));
          if (FIRST && t == 0) {
            gdone[at] = m;
            if constexpr (MODE != kModeB) up[at] = m > R[at];
          }
          // NN-B: the closed group's key enters R in tile at % 8 of the next
          // group, one atom tile per code tile, so the key's VALU work is
          // spread evenly under the MFMAs instead of piling up in tile 0.
          if (MODE == kModeB && at % 8 == t) R[at] = max(R[at], group_key(gdone[at], group_prev));
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
  // fold the slice's last tile and close its last group
#pragma unroll
  for (int at = 0; at < kAT; ++at) {
    int m = max(max(gm[at], __float_as_int(acc[at][0])), __float_as_int(acc[at][1]));
    m = max(max(m, __float_as_int(acc[at][2])), __float_as_int(acc[at][3]));
    if constexpr (MODE == kModeB) {
      R[at] = max(R[at], group_key(m, group_prev));
    } else if (m > R[at]) {
      R[at] = raised_threshold<MODE>(m);
      best[at] = group_prev;
    }
  }

  // ---- merge this slice into the atom's key ----
  // The four lanes of atom j (j, j+16, j+32, j+48) hold the slice's best
  // per lane; their maximum is the slice's best (score, earliest group) and
  // the mask names the lanes that reached it in that group.
#pragma unroll
  for (int at = 0; at < kAT; ++at) {
    const int64_t a = wave_atom0 + at * 16 + j;
    if constexpr (MODE == kModeB) {
      int Rm = R[at];
      Rm = max(Rm, __shfl_xor(Rm, 16, 64));
      Rm = max(Rm, __shfl_xor(Rm, 32, 64));
      const uint64_t bal = __ballot(R[at] == Rm);  // bit l: lane l holds the maximum
      const uint32_t mask = static_cast<uint32_t>(((bal >> j) & 1u) | ((bal >> (j + 15)) & 2u) |
                                                  ((bal >> (j + 30)) & 4u) | ((bal >> (j + 45)) & 8u));
      const uint32_t g = 0xFFFFu - (static_cast<uint32_t>(Rm) & 0xFFFFu);
      // no hit: key 0, which leaves the atom's key as it is (a select, not a
      // branch: a conditional atomic here costs the main loop ~20 VGPRs)
      const uint32_t key = Rm != initial_threshold<MODE>()
                               ? (static_cast<uint32_t>(Rm) & 0xFFFF0000u) | ((0x3FFu - g) << 6) | (mask << 2)
                               : 0u;
      if (q == 0 && a < n_atoms) atomicMax(static_cast<unsigned int *>(keys) + a, key);
    } else {
      // (score, 1023 - group) as one 64-bit value, lanes that never beat the threshold 0
      const bool hit = best[at] >= 0;
      uint64_t v = hit ? (static_cast<uint64_t>(static_cast<uint32_t>(R[at])) << 32) |
                             (static_cast<uint64_t>(0x3FFu - static_cast<uint32_t>(best[at])) << 4)
                       : 0ull;
      uint64_t vm = v;
      uint64_t o = static_cast<uint64_t>(__shfl_xor(static_cast<long long>(vm), 16, 64));
      vm = o > vm ? o : vm;
      o = static_cast<uint64_t>(__shfl_xor(static_cast<long long>(vm), 32, 64));
      vm = o > vm ? o : vm;
      const uint64_t bal = __ballot(v == vm);
      const uint64_t mask = ((bal >> j) & 1u) | ((bal >> (j + 15)) & 2u) | ((bal >> (j + 30)) & 4u) |
                            ((bal >> (j + 45)) & 8u);
      const uint64_t key = vm != 0ull ? vm | mask : 0ull;
      if (q == 0 && a < n_atoms) atomicMax(static_cast<unsigned long long *>(keys) + a, static_cast<unsigned long long>(key));
    }
  }
}

// Resolve: per block 256 atoms.
//   scan     thread per atom: its key (the bucket or score M, the earliest
//            group G holding it, the lanes of G that reach it), the atom's
//            coordinates into LDS (bf16 pairs; NN-P: fp32), one candidate
//            per lane of the mask, each naming G's kG tiles x 4 codes of that lane;
//   compact  a block-wide prefix sum packs the candidates into one list;
//   rescan   kG lanes per candidate, lane t scoring the 4 codes of tile t of
//            the group (NN-B/T: 3-bit value ids from kp_dq expanded to bf16,
//            v_dot2_f32_bf16 = exact bf16 products, fp32 sums; NN-P: 4
//            consecutive rows of the raw int8 codebook, fp64 dot products of
//            the fp32 atom with the fp32 codebook values, exact to 2^-48),
//            then a 4-step shuffle reduction per candidate;
//   merge    thread per atom folds its candidates' results in list order.
// keys / xb point at this call's first atom (a batched sweep covers several
// matrices; each resolves its own range).
// NN-B picks the lowest code whose bf16 score bucket equals M (falling back to
// the best rounded score, lowest code on ties, if the fp32 sums disagree with
// the sweep's); NN-T the highest fp32 score, lowest code on ties; NN-P the
// highest fp64 score, lowest code on ties.  Then the int32 index and,
// optionally, the packed 9-byte groups.
constexpr int kRsPerRound = 4;  // lanes of one atom: every candidate in one round
constexpr int kRsCap = 256 * kRsPerRound;

template <int MODE>
struct RsScore {  // per-candidate / per-atom running result
  typedef typename std::conditional<MODE == kModeP, double, float>::type T;
};

template <int MODE, bool FUSED>
__global__ __launch_bounds__(256) void resolve_kernel(const void *__restrict__ keys, int64_t n_atoms,
                                                      const float *__restrict__ src,
                                                      const float *__restrict__ sigma, int64_t atoms_per_row,
                                                      const uint4 *__restrict__ xb, const uint8_t *__restrict__ rescan,
                                                      int32_t *__restrict__ idx_out, uint8_t *__restrict__ packed_out) {
  typedef typename RsScore<MODE>::T score_t;
  constexpr int XW = MODE == kModeP ? kDim : 12;  // words of one atom's coordinates in LDS
  __shared__ __align__(16) uint32_t xs[256 * XW];
  __shared__ uint32_t tmp[kRsPerRound * 256];     // per-thread candidates before compaction
  __shared__ uint32_t cand[kRsCap];               // atom | lane << 8 | group << 10
  __shared__ score_t res_v[kRsCap];
  __shared__ uint32_t res_code[kRsCap];
  __shared__ uint32_t res_found[MODE == kModeB ? kRsCap : 1];
  __shared__ uint32_t Ms[256];                    // per atom: the sweep's best bucket (NN-B)
  __shared__ int wave_sum[4];
  __shared__ int32_t ids[256];
  __shared__ __align__(16) uint8_t bytes[64 * 9];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t a0 = static_cast<int64_t>(blockIdx.x) * 256;
  const int64_t a = a0 + tid;

  // ---- scan: the key, coordinates, origin rules ----
  uint32_t M = 0, G = 0, lanes = 0;
  bool active = false;
  if (a < n_atoms) {
    if constexpr (MODE == kModeB) {
      const uint32_t k = static_cast<const uint32_t *>(keys)[a];
      M = k >> 16;
      G = 0x3FFu - ((k >> 6) & 0x3FFu);
      lanes = (k >> 2) & 0xFu;
    } else {
      const uint64_t k = static_cast<const unsigned long long *>(keys)[a];
      M = static_cast<uint32_t>(k >> 32);
      G = 0x3FFu - static_cast<uint32_t>((k >> 4) & 0x3FFu);
      lanes = static_cast<uint32_t>(k & 0xFu);
    }
    double nrm2 = 0.0;
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
        *reinterpret_cast<uint4 *>(xs + tid * XW + 4 * qq) = xb[a * 3 + qq];  // bf16 pairs from prep_kernel
      }
    }
    // NN-P's origin rule (pack.py:174): |x|_2 < fp32(1e-8); no scan needed
    const bool p_snap = MODE == kModeP && sqrt(nrm2) < static_cast<double>(__uint_as_float(kEpsBits));
    active = M != 0 && lanes != 0 && !p_snap;
  }
  Ms[tid] = M;

  uint32_t found = 0xFFFFFFFFu;  // NN-B: lowest code whose bucket equals M
  score_t best_v = -__builtin_inf();
  uint32_t best_code = 0xFFFFFFFFu;
  {
    // ---- this thread's candidates: the lanes of its mask, all in group G ----
    int nm = 0;
    if (active) {
#pragma unroll
      for (int qq = 0; qq < 4; ++qq)
        if ((lanes >> qq) & 1u) tmp[nm++ * 256 + tid] = static_cast<uint32_t>(tid) | static_cast<uint32_t>(qq) << 8 | G << 10;
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

    // ---- rescan: kG lanes per candidate ----
    const uint4 bt = bf16_value_table();
    for (int task = tid; task < total * kG; task += 256) {
      const int c = task / kG, t = task % kG;
      const uint32_t cd = cand[c];
      const int al = static_cast<int>(cd & 0xFFu), qq = static_cast<int>((cd >> 8) & 3u);
      const int tile = static_cast<int>(cd >> 10) * kG + t;
      uint32_t f = 0xFFFFFFFFu, bc = 0xFFFFFFFFu;
      score_t bv = -__builtin_inf();
      if (tile < kRealTiles) {
        if constexpr (MODE == kModeP) {
          double xd[kDim];
#pragma unroll
          for (int k = 0; k < kDim; ++k) xd[k] = static_cast<double>(__uint_as_float(xs[al * XW + k]));
          const uint32_t code0 = static_cast<uint32_t>(tile * kTileCodes + 4 * qq);
          const uint2 *cr = reinterpret_cast<const uint2 *>(rescan + (static_cast<size_t>(code0) + 1) * kDim);
          uint2 rw[12];
#pragma unroll
          for (int k = 0; k < 12; ++k) rw[k] = cr[k];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t w6[6] = {rw[3 * e].x, rw[3 * e].y, rw[3 * e + 1].x, rw[3 * e + 1].y, rw[3 * e + 2].x,
                                    rw[3 * e + 2].y};
            double sc = 0.0;
#pragma unroll
            for (int k = 0; k < kDim; ++k) {
              const int r = static_cast<int32_t>(w6[k / 4] << (24 - 8 * (k % 4))) >> 24;
              sc = fma(xd[k], static_cast<double>(raw_value_f32(r)), sc);
            }
            if (sc > bv) {  // codes ascend with e: the first maximum is kept
              bv = sc;
              bc = code0 + e;
            }
          }
        } else {
          const uint4 *xq = reinterpret_cast<const uint4 *>(xs + al * XW);
          const uint4 x0 = xq[0], x1 = xq[1], x2 = xq[2];
          const uint32_t xw[12] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w, x2.x, x2.y, x2.z, x2.w};
          // 4 consecutive codebook rows (code + 1): 12 words of 3-bit value
          // ids, expanded to bf16 pairs by byte lookups
          const uint32_t code0 = static_cast<uint32_t>(tile * kTileCodes + 4 * qq);
          const uint32_t *cp = reinterpret_cast<const uint32_t *>(rescan) + (static_cast<size_t>(code0) + 1) * 3;
          uint32_t idw[12];
#pragma unroll
          for (int k = 0; k < 12; ++k) idw[k] = cp[k];
          const uint32_t Mk = Ms[al];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            uint32_t cw[12];
#pragma unroll
            for (int p = 0; p < 3; ++p) {
              const uint4 o = ids_to_pairs(idw[3 * e + p], bt);
              cw[4 * p] = o.x;
              cw[4 * p + 1] = o.y;
              cw[4 * p + 2] = o.z;
              cw[4 * p + 3] = o.w;
            }
            float sc = 0.f;
#pragma unroll
            for (int d = 0; d < 12; ++d)
              sc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, xw[d]), __builtin_bit_cast(bf16x2, cw[d]),
                                                   sc, false);
            const uint32_t code = static_cast<uint32_t>(tile * kTileCodes + 4 * qq + e);
            float v = sc;
            if (MODE == kModeB) {
              const uint32_t bk = bf16_rne_bits(sc);
              v = bf16_bits_to_float(bk);
              if (bk == Mk && code < f) f = code;
            }
            if (v > bv) {
              bv = v;
              bc = code;
            }
          }
        }
      }
      // reduce over the candidate's kG lanes: lowest found code; best score, lowest code on ties
#pragma unroll
      for (int d = 1; d < kG; d <<= 1) {
        const uint32_t of = static_cast<uint32_t>(__shfl_xor(static_cast<int>(f), d, 64));
        const uint32_t oc = static_cast<uint32_t>(__shfl_xor(static_cast<int>(bc), d, 64));
        score_t ov;
        if constexpr (MODE == kModeP)
          ov = __longlong_as_double(__shfl_xor(__double_as_longlong(bv), d, 64));
        else
          ov = __shfl_xor(bv, d, 64);
        f = min(f, of);
        if (ov > bv || (ov == bv && oc < bc)) {
          bv = ov;
          bc = oc;
        }
      }
      if (t == 0) {
        res_v[c] = bv;
        res_code[c] = bc;
        if constexpr (MODE == kModeB) res_found[c] = f;
      }
    }
    __syncthreads();

    // ---- merge this thread's candidates ----
    for (int i = 0; i < nm; ++i) {
      const score_t v = res_v[off + i];
      const uint32_t code = res_code[off + i];
      if (v > best_v || (v == best_v && code < best_code)) {
        best_v = v;
        best_code = code;
      }
      if constexpr (MODE == kModeB) found = min(found, res_found[off + i]);
    }
  }

  int32_t id = 0;
  if (active) {
    bool snap;
    uint32_t code;
    if (MODE == kModeP) {
      code = best_code;
      snap = best_code == 0xFFFFFFFFu;  // non-finite atom: no score compared
    } else if (MODE == kModeB) {
      const uint32_t bucket = found != 0xFFFFFFFFu ? M : (__float_as_uint(static_cast<float>(best_v)) >> 16);
      code = found != 0xFFFFFFFFu ? found : best_code;
      snap = !(best_v > 0.f) || bucket < 0x4000u;  // bf16 max below 2.0
    } else {
      code = best_code;
      snap = !(2.0f * static_cast<float>(best_v) >= __uint_as_float(kCSqNormBits));
    }
    id = snap ? 0 : static_cast<int32_t>(code) + 1;
  }
  if (idx_out && a < n_atoms) idx_out[a] = id;
  if (!packed_out) return;
  ids[tid] = id;
  __syncthreads();
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

// Codebook slices per launch.  Blocks are dispatched round-robin over the 8
// XCDs, so with 4 slices each XCD streams one 2.36 MB quarter of the bf16
// codebook (L2-resident in its 4 MB L2) and each atom block's operand planes
// are fetched by 4 XCDs (with 8 slices: 1.18 MB per XCD, planes fetched 8
// times; measured on 16.8M atoms: 4 slices 0.5% faster, half the plane
// traffic).  Small launches use more slices so the grid still has several
// waves of work-groups per CU slot.
int choose_slices(int64_t ablocks) {
  int s = 4;
  while (s < 64 && ablocks * s < 6144) s *= 2;
  return s;
}

// per-atom key slots (8 bytes; NN-B uses the first 4 n bytes as 32-bit keys)
size_t keys_bytes(int64_t n_atoms) { return (static_cast<size_t>(n_atoms) * 8 + 255) & ~static_cast<size_t>(255); }

// workspace = per-atom keys, then (NN-B / NN-T) the bf16 planes
template <int MODE, bool FUSED>
int launch_mode(const float *x, const float *sigma, int64_t apr, int64_t n_atoms, const DeviceTables *tab,
                int32_t *idx_out, uint8_t *packed_out, uint8_t *workspace, hipStream_t s) {
  const int64_t ablocks = (n_atoms + kAtomsPerBlock - 1) / kAtomsPerBlock;
  const int n_slices = choose_slices(ablocks);
  const int tiles_per_slice = kPaddedTiles / n_slices;
  const int64_t grid = ablocks * n_slices;
  if (grid > 0x7FFFFFFFll) return fail(PLX_EINVAL, "quantize: %lld atoms exceed one launch", static_cast<long long>(n_atoms));
  uint2 *keys8 = reinterpret_cast<uint2 *>(workspace);
  uint4 *xb = reinterpret_cast<uint4 *>(workspace + keys_bytes(n_atoms));
  int st;
  if (MODE != kModeP) {
    hipLaunchKernelGGL((prep_kernel<FUSED>), dim3(static_cast<unsigned>((n_atoms * 3 + 255) / 256)), dim3(256), 0, s, x,
                       sigma, apr, n_atoms, xb, keys8);
    if ((st = check_launch("prep_kernel")) != PLX_OK) return st;
  } else {
    hipLaunchKernelGGL(clear_keys_kernel, dim3(static_cast<unsigned>((n_atoms + 255) / 256)), dim3(256), 0, s, keys8,
                       n_atoms);
    if ((st = check_launch("clear_keys_kernel")) != PLX_OK) return st;
  }
  profile_before(s);
  const uint8_t *tiles = MODE == kModeP ? tab->kp_raw_tiles : tab->kp_bf16_tiles;
  const uint8_t *rescan =
      MODE == kModeP ? reinterpret_cast<const uint8_t *>(tab->cb_raw) : reinterpret_cast<const uint8_t *>(tab->kp_dq);
  const void *operand = MODE == kModeP ? static_cast<const void *>(x) : static_cast<const void *>(xb);
  hipLaunchKernelGGL((nn_kernel<MODE>), dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s, operand, n_atoms, tiles,
                     n_slices, tiles_per_slice, static_cast<void *>(keys8));
  if ((st = check_launch("nn_kernel")) != PLX_OK) return st;
  profile_after(s);
  hipLaunchKernelGGL((resolve_kernel<MODE, FUSED>), dim3(static_cast<unsigned>((n_atoms + 255) / 256)), dim3(256), 0, s,
                     static_cast<const void *>(keys8), n_atoms, x, sigma, apr, xb, rescan, idx_out, packed_out);
  return check_launch("resolve_kernel");
}

}  // namespace

size_t quantize_workspace_bytes(int64_t n_atoms) {
  if (n_atoms <= 0) return 0;
  return keys_bytes(n_atoms) + static_cast<size_t>(n_atoms) * 48;
}

int launch_quantize(const float *x, const float *sigma, int64_t rows, int64_t cols, int64_t n_atoms, int mode,
                    int32_t *idx_out, uint8_t *packed_out, float *weight_out, void *workspace,
                    size_t workspace_bytes, hipStream_t s) {
  (void)rows;
  if (n_atoms <= 0) return PLX_OK;
  if (workspace == nullptr || workspace_bytes < quantize_workspace_bytes(n_atoms))
    return fail(PLX_EINVAL, "quantize: workspace of %zu bytes is smaller than the %zu needed for %lld atoms",
                workspace_bytes, quantize_workspace_bytes(n_atoms), static_cast<long long>(n_atoms));
  if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0 || (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0)
    return fail(PLX_EINVAL, "quantize: input and workspace must be 16-byte aligned");
  const DeviceTables *tab = nullptr;
  int st = get_tables(&tab);
  if (st != PLX_OK) return st;
  uint8_t *ws = static_cast<uint8_t *>(workspace);
  const bool fused = sigma != nullptr;
  const int64_t apr = cols / kDim;
  if (mode == PLX_NN_PACK_FP32)
    st = launch_mode<PLX_NN_PACK_FP32, false>(x, nullptr, apr, n_atoms, tab, idx_out, packed_out, ws, s);
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

// Several latents in one scoring sweep: row scale and operand planes per
// matrix, one nn_kernel launch over all their atoms (fewer codebook slices per
// atom block and no per-matrix tail of the grid), then per matrix the resolve
// (index + pack) and the scaled gather of the reconstructed weight.
template <int MODE>
int launch_batch_mode(const RequantItem *items, int n_items, const DeviceTables *tab, uint8_t *workspace,
                      hipStream_t s) {
  int64_t total = 0;
  for (int i = 0; i < n_items; ++i) total += items[i].rows * (items[i].cols / kDim);
  if (total == 0) return PLX_OK;
  const int64_t ablocks = (total + kAtomsPerBlock - 1) / kAtomsPerBlock;
  const int n_slices = choose_slices(ablocks);
  const int tiles_per_slice = kPaddedTiles / n_slices;
  const int64_t grid = ablocks * n_slices;
  if (grid > 0x7FFFFFFFll) return fail(PLX_EINVAL, "requantize_batch: %lld atoms exceed one launch", static_cast<long long>(total));
  uint2 *keys8 = reinterpret_cast<uint2 *>(workspace);
  uint4 *xb = reinterpret_cast<uint4 *>(workspace + keys_bytes(total));
  int st;
  int64_t off = 0;
  for (int i = 0; i < n_items; ++i) {
    const RequantItem &it = items[i];
    const int64_t apr = it.cols / kDim, n = it.rows * apr;
    if (n == 0) continue;
    if ((st = launch_row_rms(it.latent, it.rows, it.cols, it.sigma, nullptr, s)) != PLX_OK) return st;
    hipLaunchKernelGGL((prep_kernel<true>), dim3(static_cast<unsigned>((n * 3 + 255) / 256)), dim3(256), 0, s, it.latent,
                       it.sigma, apr, n, xb + off * 3, keys8 + off);
    if ((st = check_launch("prep_kernel")) != PLX_OK) return st;
    off += n;
  }
  profile_before(s);
  hipLaunchKernelGGL((nn_kernel<MODE>), dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s,
                     static_cast<const void *>(xb), total, tab->kp_bf16_tiles, n_slices, tiles_per_slice,
                     static_cast<void *>(keys8));
  if ((st = check_launch("nn_kernel")) != PLX_OK) return st;
  profile_after(s);
  off = 0;
  for (int i = 0; i < n_items; ++i) {
    const RequantItem &it = items[i];
    const int64_t apr = it.cols / kDim, n = it.rows * apr;
    if (n == 0) continue;
    hipLaunchKernelGGL((resolve_kernel<MODE, true>), dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
                       MODE == kModeB ? static_cast<const void *>(reinterpret_cast<const uint32_t *>(keys8) + off)
                                      : static_cast<const void *>(keys8 + off),
                       n, it.latent, it.sigma, apr, xb + off * 3,
                       reinterpret_cast<const uint8_t *>(tab->kp_dq), it.idx, it.packed);
    if ((st = check_launch("resolve_kernel")) != PLX_OK) return st;
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
  return mode == PLX_NN_BF16_SCORES ? launch_batch_mode<PLX_NN_BF16_SCORES>(items, n_items, tab, ws, s)
                                    : launch_batch_mode<PLX_NN_FP32_SCORES>(items, n_items, tab, ws, s);
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
constexpr size_t kScratchBytes = static_cast<size_t>(PLX_NOALLOC_MAX_ATOMS) * (8 + 48);
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

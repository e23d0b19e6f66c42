// LUT-gather dequantization to fp16 (replaces PackedH24Linear.materialize,
// pollux.py:485-504).
//
//   W[r, 24a + c] = fp16( fp32(fp16(cb16[idx] * sigma16[r])) * fp32(1/sqrt 2) )
//
// cb16 is the RNE fp16 cast of the fp32 codebook (castor.py:193-199); both
// products are computed in fp32 and rounded to fp16, the way torch evaluates
// ``atoms * sigma_rows.view(-1,1,1) * s_lattice`` on fp16 tensors (fp32
// opmath; the Python float scalar enters as fp32).  The raw coordinates take
// the 8 values {0,1,2,4,-4,-3,-2,-1}, so per row the output takes one of 8
// fp16 values; every step of the formula is an odd function of the code
// value, so the negative entries are the positive ones with the sign flipped.
//
// Layout of the work: a block covers 256 atoms = 768 output chunks of 16 B
// (8 coordinates); thread t of the block writes chunks t, t+256, t+512, so each
// store instruction writes 4 KiB contiguous.  Few stores per thread matter on
// MI355X: with 3 chunks per thread the kernel sustains ~82% of HBM peak, with
// 12 (1,024-atom blocks) ~72%.  Per block the packed bytes are staged in LDS
// and decoded once per atom, and each row met by the block gets its 8-entry
// value table (low bytes, high bytes: 4 words) in LDS; a chunk is then one
// 4-byte kp_dq load (3-bit value ids, L2-resident) and 6 v_perm_b32 byte
// lookups.  The output is written with non-temporal stores: as ordinary
// stores its 48 B/atom stream evicts kp_dq from L2 and the gathers then miss
// (measured: 30-40% of HBM peak).
//
// Indices above 196,560 (not produced by the reference packer) decode as the
// origin, so corrupt input can never read outside the table.

#include <hip/hip_fp16.h>

#include <type_traits>

#include "plx_device.h"

namespace plx {
namespace {

constexpr int kThreads = 256;
constexpr int kDqAtoms = 256;                      // atoms per block

constexpr int kDqPackedBytes = kDqAtoms / 4 * 9;   // 576
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void dequant_kernel(const uint8_t *__restrict__ packed, int64_t packed_bytes,
                                                           const uint16_t *__restrict__ sigma16, int64_t n_atoms,
                                                           int64_t atoms_per_row, const uint32_t *__restrict__ kp_dq,
                                                           uint16_t *__restrict__ w16) {
  __shared__ __align__(16) uint8_t pk[kDqPackedBytes];
  __shared__ uint32_t ent[kDqAtoms];        // code | (row - row0) << 18
  __shared__ uint4 tab[kDqAtoms + 1];       // per row: low bytes ids 0-3, 4-7, high bytes ids 0-3, 4-7
  const int64_t a0 = static_cast<int64_t>(blockIdx.x) * kDqAtoms;
  const int atoms_here = static_cast<int>(min(static_cast<int64_t>(kDqAtoms), n_atoms - a0));
  const int tid = threadIdx.x;

  // packed bytes of the block's 256 groups (the last block may hold fewer)
  const uint8_t *src = packed + a0 / 4 * 9;
  const int nb = static_cast<int>(min(static_cast<int64_t>(kDqPackedBytes), packed_bytes - a0 / 4 * 9));
  if (nb == kDqPackedBytes && aligned16(packed)) {
    for (int i = tid; i < kDqPackedBytes / 16; i += kThreads)
      reinterpret_cast<uint4 *>(pk)[i] = reinterpret_cast<const uint4 *>(src)[i];
  } else {
    for (int i = tid; i < nb; i += kThreads) pk[i] = src[i];
  }
  const int64_t row0 = a0 / atoms_per_row;
  const uint32_t base = static_cast<uint32_t>(a0 - row0 * atoms_per_row);  // < atoms_per_row
  const uint32_t apr32 = static_cast<uint32_t>(atoms_per_row);
  const int n_rows = static_cast<int>((base + static_cast<uint32_t>(atoms_here) - 1u) / apr32) + 1;
  const float sl = __uint_as_float(kSLatticeBits);
  for (int r = tid; r < n_rows; r += kThreads) {
    const float sig = __half2float(__ushort_as_half(sigma16[row0 + r]));
    const uint32_t v0 = dq_value(0, sig, sl), v1 = dq_value(1, sig, sl), v2 = dq_value(2, sig, sl);
    const uint32_t v3 = dq_value(3, sig, sl), v4 = dq_value(4, sig, sl);
    // ids 0..7 -> {0, 1, 2, 4, -4, -3, -2, -1}
    const uint32_t e[8] = {v0, v1, v2, v4, v4 ^ 0x8000u, v3 ^ 0x8000u, v2 ^ 0x8000u, v1 ^ 0x8000u};
    uint4 t;
    t.x = (e[0] & 0xFFu) | (e[1] & 0xFFu) << 8 | (e[2] & 0xFFu) << 16 | (e[3] & 0xFFu) << 24;
    t.y = (e[4] & 0xFFu) | (e[5] & 0xFFu) << 8 | (e[6] & 0xFFu) << 16 | (e[7] & 0xFFu) << 24;
    t.z = (e[0] >> 8) | (e[1] >> 8) << 8 | (e[2] >> 8) << 16 | (e[3] >> 8) << 24;
    t.w = (e[4] >> 8) | (e[5] >> 8) << 8 | (e[6] >> 8) << 16 | (e[7] >> 8) << 24;
    tab[r] = t;
  }
  __syncthreads();
  for (int i = tid; i < atoms_here; i += kThreads) {
    int32_t code = packed_index(pk, i);
    if (code > kKissing) code = 0;
    ent[i] = static_cast<uint32_t>(code) | (((base + static_cast<uint32_t>(i)) / apr32) << 18);
  }
  __syncthreads();

  u32x4_t *dst = reinterpret_cast<u32x4_t *>(w16 + a0 * kDim);
  const int n_chunks = atoms_here * 3;
#pragma unroll
  for (int c = tid; c < n_chunks; c += kThreads) {
    const int atom = c / 3, plane = c - 3 * atom;
    const uint32_t en = ent[atom];
    const uint32_t ids = kp_dq[(en & 0x3FFFFu) * 3 + static_cast<uint32_t>(plane)];
    const uint4 t = tab[en >> 18];
    const uint32_t s_lo = ids & 0x0F0F0F0Fu, s_hi = (ids >> 4) & 0x0F0F0F0Fu;
    const uint32_t l_lo = __builtin_amdgcn_perm(t.y, t.x, s_lo), h_lo = __builtin_amdgcn_perm(t.w, t.z, s_lo);
    const uint32_t l_hi = __builtin_amdgcn_perm(t.y, t.x, s_hi), h_hi = __builtin_amdgcn_perm(t.w, t.z, s_hi);
    u32x4_t o;
    o.x = __builtin_amdgcn_perm(h_lo, l_lo, 0x05010400u);  // coordinates 0, 1
    o.y = __builtin_amdgcn_perm(h_lo, l_lo, 0x07030602u);  // 2, 3
    o.z = __builtin_amdgcn_perm(h_hi, l_hi, 0x05010400u);  // 4, 5
    o.w = __builtin_amdgcn_perm(h_hi, l_hi, 0x07030602u);  // 6, 7
    __builtin_nontemporal_store(o, dst + c);
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
  if (n_atoms == 0) return PLX_OK;
  const int64_t pb = (n_atoms + 3) / 4 * 9;
  const dim3 g(static_cast<unsigned>((n_atoms + kDqAtoms - 1) / kDqAtoms));
  profile_before(s, PLX_PROF_DEQUANT);
  hipLaunchKernelGGL(dequant_kernel, g, dim3(kThreads), 0, s, packed, pb, sigma16, n_atoms, apr, tab->kp_dq, w16);
  profile_after(s, PLX_PROF_DEQUANT);
  return check_launch("dequant_kernel");
}

namespace {

// ---------------------------------------------------------------------------
// Fused dequant-linear: y[m, r] = sum_i x[m, i] * W[r, i] without materialising
// W (replaces PackedH24Linear.materialize + F.linear, pollux.py:485-507).
//
// Every weight of row r is +-v_k(r) with v_k the fp16 materialised magnitude
// of |k| = 1..4 (dq_value), so one atom with raw code k and activations x
// contributes, with D = sum_c k_c x_c over the raw integer code:
//   type 1 (+-4 at two coordinates)     v4 * D / 4
//   type 2 (+-2 on an octad)            v2 * D / 2
//   type 3 (+-1, one -3 at coordinate p) v1 * (D + 3 x_p) - v3 * x_p
//   origin                              0
// The row keeps four fp32 partial sums and applies the magnitudes once at the
// end: the same products as F.linear(x.float(), W.float()), regrouped (fp32
// rounding differs at the 1e-7 relative level).  With `round_w` (bf16 x and
// PLX_DQL_W_AS_X) the magnitudes are first rounded to bf16 (RNE, an odd
// function, so the signed weights follow): the products of the reference's
// literal F.linear(x, W.to(x.dtype)) (pollux.py:507).
//
// Per code the kernel reads one 16-byte entry of kp_gemv (24 signed 4-bit
// coordinates + type/position byte; 3.1 MB, L2-resident per XCD).
// L lanes share a row and stride over its atoms; a block is NT threads.
// ---------------------------------------------------------------------------

// Output epilogue of the dequant-linear kernels: GELU in torch's erf form
// (F.gelu: x * 0.5 * (1 + erf(x * sqrt(1/2))), pollux.py:645) and / or a
// residual added after it (x + linear(h), pollux.py:660-661).
__device__ __forceinline__ float dql_epilogue(float v, const float *__restrict__ residual, int64_t i, int gelu) {
  if (gelu) v = (v * 0.5f) * (1.0f + erff(v * __uint_as_float(kSLatticeBits)));  // fp32(1/sqrt 2)
  if (residual) v = residual[i] + v;
  return v;
}

// Up to kDqlMaxTargets weights sharing one x in one GEMV launch: blockIdx.y is
// the target, blockIdx.x the row block (blocks past a shorter target's rows
// return at once).
constexpr int kDqlMaxTargets = 4;
struct DqlTargets {
  const uint8_t *packed[kDqlMaxTargets];
  int64_t packed_bytes[kDqlMaxTargets];
  const uint16_t *sigma16[kDqlMaxTargets];
  int64_t rows[kDqlMaxTargets];
  float *y[kDqlMaxTargets];
  const float *residual[kDqlMaxTargets];
  const float *norm_w;  // fp32 x is RMS-normalised per token row in LDS first (or NULL)
  float norm_eps;
  int n;
};

// One target without epilogue: the plain call (selecting a target and the
// epilogue's checks cost ~0.7 us per launch at M = 1, measured).
struct DqlOne {
  const uint8_t *packed;
  int64_t packed_bytes;
  const uint16_t *sigma16;
  int64_t rows;
  float *y;
};

// element ti of a kernel-argument array by wave-uniform selects (no dynamic indexing of the argument block)
// (the loaded values are made opaque: otherwise the compiler turns the selects
// into a kernel-argument load at a computed offset, a dependent round trip)
template <typename T>
__device__ __forceinline__ T pick(const T (&a)[kDqlMaxTargets], int ti) {
  static_assert(kDqlMaxTargets == 4 && sizeof(T) == 8, "pick: four 64-bit values");
  T v0 = a[0], v1 = a[1], v2 = a[2], v3 = a[3];
  asm volatile("" : "+s"(v0), "+s"(v1), "+s"(v2), "+s"(v3));
  return ti == 1 ? v1 : ti == 2 ? v2 : ti == 3 ? v3 : v0;
}

// Accesses through pointers the compiler cannot trace to a kernel argument
// (those pick() returns) as global memory operations: flat ones would also
// count against the scalar loads' wait counter, so every kernel-argument load
// would wait for them.
template <typename T>
__device__ __forceinline__ T gload(const T *p) {
  return *(const __attribute__((address_space(1))) T *)(p);
}
template <typename T>
__device__ __forceinline__ void gstore(T *p, T v) {
  *(__attribute__((address_space(1))) T *)(p) = v;
}
// 16 bytes as a native vector (a struct copy would be lowered to flat loads)
__device__ __forceinline__ uint4 gload16(const void *p) {
  const u32x4_t v = *(const __attribute__((address_space(1))) u32x4_t *)(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 gload16f(const float *p) {
  const uint4 v = gload16(p);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

template <bool XF32>
__device__ __forceinline__ void load_x8(const void *__restrict__ x, int64_t off, float *v) {
  if (XF32) {
    const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(x) + off);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 w = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(x) + off);
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(d[i] << 16);
      v[2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
    }
  }
}

template <bool XF32>
__device__ __forceinline__ float load_x1(const void *__restrict__ x, int64_t off) {
  if (XF32) return static_cast<const float *>(x)[off];
  return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t *>(x)[off]) << 16);
}

// x for the block in LDS as fp32 (XL == true) or read from global memory.
template <bool XF32>
__device__ __forceinline__ float x_at(const void *__restrict__ x, int64_t off) {
  if (XF32) return static_cast<const float *>(x)[off];
  return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t *>(x)[off]) << 16);
}

// One pass over the packed rows for MB tokens.  Block = NT threads = R = NT/L
// rows; the block's packed bytes (and, when XL, the MB token rows of x as
// fp32) are staged in LDS first; each lane then handles atoms sub, sub+L, ...
// of its row in chunks of kDqlGather, issuing the chunk's table gathers before
// scoring any of them.  At one token the kernel is a chain of memory round
// trips, so everything that does not depend on the staged data is requested
// before the first barrier (which waits for all of it): x and the norm weights
// into registers when each thread holds at most one 8-value piece of the first
// MB token rows, the packed bytes, the row's sigma16 and residual values.
template <bool GEN>
using DqlArgs = typename std::conditional<GEN, DqlTargets, DqlOne>::type;

// table gathers in flight per lane: the Pollux-1920 rows (80 atoms at 16 lanes,
// 320 at 64) give every lane exactly 5 atoms, one round (4 per round: two
// rounds, 2% slower at one token; 8: wasted slots, 11% slower)
constexpr int kDqlGather = 5;
constexpr int kDqlPlVecs = 2;          // PL: record vectors per thread at 512 threads (16 KB per block)
constexpr int kDqlPlTableVecs = 1536;  // PL: plane-table capacity in 16-byte vectors (24 KB; lookups clamped to it)

// GEN: several targets and the epilogue (DqlTargets); else one target, no epilogue (DqlOne).
// XREG (with XL, m_total <= MB and MB token rows of at most 8 * NT values): x
// goes through registers into LDS and the general staging loop is compiled
// out - at one token these kernels are short enough that their code size
// shows in the time (cold instruction fetch).
// PL: `packed` is the plane layout (3 uint16 records per atom); the coordinate
// words come from the plane table (kp_gemv's format) staged in LDS instead of a
// kp_gemv gather; the block's records are staged with kDqlPlVecs raw buffer
// loads per thread, x after them, the table after x.
template <int L, int MB, bool XF32, bool XL, int NT, bool GEN, bool XREG, bool PL = false>
__global__ __launch_bounds__(NT) void dqlinear_kernel(const DqlArgs<GEN> targets, int64_t atoms_per_row,
                                                       const void *__restrict__ x, int64_t m_total,
                                                       const uint4 *__restrict__ kp_gemv, int round_w, int gelu,
                                                       const uint32_t *__restrict__ pl_nib, int pl_vecs) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float norm_red[NT / 64][MB];  // per-wave sums of squares (GEN with norm_w)
  constexpr int R = NT / L;
  const uint8_t *__restrict__ packed;
  const uint16_t *__restrict__ sigma16;
  float *__restrict__ y;
  const float *__restrict__ residual = nullptr;
  const float *__restrict__ norm_w = nullptr;
  int64_t packed_bytes, rows;
  if constexpr (GEN) {
    const int ti = static_cast<int>(blockIdx.y);
    packed = pick(targets.packed, ti);
    packed_bytes = pick(targets.packed_bytes, ti);
    sigma16 = pick(targets.sigma16, ti);
    rows = pick(targets.rows, ti);
    y = pick(targets.y, ti);
    residual = pick(targets.residual, ti);
    norm_w = targets.norm_w;
    if (static_cast<int64_t>(blockIdx.x) * R >= rows) return;  // the whole block: before any barrier
  } else {
    packed = targets.packed;
    packed_bytes = targets.packed_bytes;
    sigma16 = targets.sigma16;
    rows = targets.rows;
    y = targets.y;
  }
  const int64_t cols = atoms_per_row * kDim;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * R;
  const int64_t rows_here = min(static_cast<int64_t>(R), rows - row0);
  const int lane = threadIdx.x & 63;
  const int sub = lane % L;
  const int64_t row = row0 + threadIdx.x / L;
  const bool live = row < rows;
  const bool writer = live && sub == 0;

  // packed bytes of atoms [row0*apr, (row0+rows_here)*apr): whole 9-byte groups
  const int64_t atom0 = row0 * atoms_per_row;
  const int64_t g_lo = atom0 >> 2, g_hi = (atom0 + rows_here * atoms_per_row + 3) >> 2;
  // Copy the bytes [g_lo*9, g_hi*9) as aligned 16-byte vectors: byte b of the
  // stream lands at LDS offset b - base16, so vectors stay aligned on both
  // sides; a last vector that would cross the end of the stream goes bytewise.
  const int64_t start = PL ? 6 * atom0 : g_lo * 9;
  const int64_t end = PL ? 6 * (atom0 + rows_here * atoms_per_row) : g_hi * 9;
  const int64_t base16 = start & ~static_cast<int64_t>(15);
  const int nvec = static_cast<int>((end - base16 + 15) >> 4);
  const uint8_t *pb = smem + (start - base16);
  constexpr int PVT = kDqlPlVecs * 512 / NT;  // PL: staged record vectors per thread
  float *xs = reinterpret_cast<float *>(smem + (PL ? PVT * NT * 16 : static_cast<int64_t>(nvec) * 16));
  constexpr int TPT = (kDqlPlTableVecs + NT - 1) / NT;  // PL: plane-table vectors per thread
  uint32_t *ptab = reinterpret_cast<uint32_t *>(reinterpret_cast<uint8_t *>(xs) +
                                                (XL ? static_cast<int64_t>(MB) * atoms_per_row * kDim * 4 : 0));
  // the thread's first vector is requested before anything else (from a
  // clamped address, so no branch holds the load)
  const int64_t gb0 = base16 + 16 * static_cast<int64_t>(threadIdx.x);
  const bool v0ok = static_cast<int>(threadIdx.x) < nvec && gb0 + 16 <= packed_bytes;
  uint4 pk0 = make_uint4(0u, 0u, 0u, 0u);
  if (!PL && packed_bytes >= 16) pk0 = gload16(packed + (v0ok ? gb0 : 0));
  // PL: the block's records by raw buffer loads (a dword wholly or partly past the layout reads as
  // zero; the range is the layout rounded up to whole dwords, inside the allocation's last page)
  uint32_t pd[PL ? PVT : 1][4];
  if constexpr (PL) {
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(packed), static_cast<short>(0), static_cast<int>((packed_bytes + 3) & ~3ll), 0x00020000);
#pragma unroll
    for (int v = 0; v < PVT; ++v) {
      const int vi = static_cast<int>(threadIdx.x) + v * NT;
      int poff = vi < nvec ? static_cast<int>(base16) + 16 * vi : 0x7FFFFFF0;
      asm("" : "+v"(poff));
#pragma unroll
      for (int k = 0; k < 4; ++k) pd[v][k] = __builtin_amdgcn_raw_buffer_load_b32(prs, poff + 4 * k, 0, 0);
    }
  }
  uint4 tq[PL ? TPT : 1];
  if constexpr (PL) {
#pragma unroll
    for (int v = 0; v < TPT; ++v) {
      const int vi = static_cast<int>(threadIdx.x) + v * NT;
      tq[v] = reinterpret_cast<const uint4 *>(pl_nib)[vi < pl_vecs ? vi : 0];
    }
  }

  // requests that need nothing staged: sigma16, residuals and (first MB tokens) x and norm weights;
  // every lane loads its (clamped) row: a load under a divergent branch would be
  // waited for at once (the other path writes the same register)
  const int64_t rrow = live ? row : rows - 1;
  const uint16_t sig_bits = gload(sigma16 + rrow);
  const int mb0 = static_cast<int>(min(static_cast<int64_t>(MB), m_total));
  float res0[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) res0[mb] = 0.f;
  if constexpr (GEN) {
    if (residual) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        if (mb < mb0) res0[mb] = gload(residual + static_cast<int64_t>(mb) * rows + rrow);
    }
  }
  const int64_t items0 = mb0 * cols / 8;  // 8-value pieces of the first MB token rows
  constexpr bool xreg = XL && XREG;
  float xv0[8], nv0[8];
  if (xreg && threadIdx.x < items0) {
    load_x8<XF32>(x, 8 * static_cast<int64_t>(threadIdx.x), xv0);
    if constexpr (GEN) {
      if (norm_w) {
        const int64_t c8 = 8 * static_cast<int64_t>(threadIdx.x) % cols;
        const float4 g0 = gload16f(norm_w + c8);
        const float4 g1 = gload16f(norm_w + c8 + 4);
        nv0[0] = g0.x; nv0[1] = g0.y; nv0[2] = g0.z; nv0[3] = g0.w;
        nv0[4] = g1.x; nv0[5] = g1.y; nv0[6] = g1.z; nv0[7] = g1.w;
      }
    }
  }

  if constexpr (PL) {
#pragma unroll
    for (int v = 0; v < PVT; ++v)
      reinterpret_cast<uint4 *>(smem)[threadIdx.x + v * NT] = make_uint4(pd[v][0], pd[v][1], pd[v][2], pd[v][3]);
#pragma unroll
    for (int v = 0; v < TPT; ++v) reinterpret_cast<uint4 *>(ptab)[threadIdx.x + v * NT] = tq[v];
  }
  for (int i = threadIdx.x; !PL && i < nvec; i += NT) {
    const int64_t gb = base16 + 16 * static_cast<int64_t>(i);
    if (i == static_cast<int>(threadIdx.x) && v0ok) {
      reinterpret_cast<uint4 *>(smem)[i] = pk0;
    } else if (gb + 16 <= packed_bytes) {
      reinterpret_cast<uint4 *>(smem)[i] = gload16(packed + gb);
    } else {
      for (int k = 0; k < 16 && gb + k < packed_bytes; ++k) smem[16 * i + k] = gload(packed + gb + k);
    }
  }

  for (int64_t m0 = 0; m0 < m_total; m0 += MB) {
    const int mb_here = static_cast<int>(min(static_cast<int64_t>(MB), m_total - m0));
    if (XL) {
      if (m0 > 0) __syncthreads();  // the previous tokens' reads of xs are done
      if constexpr (xreg) {
        const bool mine = threadIdx.x < items0;
        if constexpr (GEN) {
          // RMSNorm of each token row (pollux.py:580-582) from the registers:
          // every block sums the squares in the same order, so all blocks scale alike
          if (norm_w) {
            const int tr = mine ? static_cast<int>(8 * static_cast<int64_t>(threadIdx.x) / cols) : MB;
            float s = 0.f;
            if (mine) {
#pragma unroll
              for (int c = 0; c < 8; ++c) s = fmaf(xv0[c], xv0[c], s);
            }
            float ss[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) ss[mb] = tr == mb ? s : 0.f;
            group_reduce<64>(ss);
            if (lane == 0)
#pragma unroll
              for (int mb = 0; mb < MB; ++mb) norm_red[threadIdx.x >> 6][mb] = ss[mb];
            __syncthreads();
            float r = 0.f;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
              float t = 0.f;
#pragma unroll
              for (int w = 0; w < NT / 64; ++w) t += norm_red[w][mb];
              const float rm = 1.0f / sqrtf(t / static_cast<float>(cols) + targets.norm_eps);
              r = tr == mb ? rm : r;
            }
            if (mine) {
#pragma unroll
              for (int c = 0; c < 8; ++c) xv0[c] = xv0[c] * r * nv0[c];
            }
          }
        }
        if (mine) {
          float4 *d = reinterpret_cast<float4 *>(xs + 8 * static_cast<int64_t>(threadIdx.x));
          d[0] = make_float4(xv0[0], xv0[1], xv0[2], xv0[3]);
          d[1] = make_float4(xv0[4], xv0[5], xv0[6], xv0[7]);
        }
      } else {
        float ss[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) ss[mb] = 0.f;
        // token rows are whole multiples of 8 elements (cols = 24 * apr): 8 per thread-step
        for (int64_t i = threadIdx.x; i < mb_here * cols / 8; i += NT) {
          float v[8];
          load_x8<XF32>(x, m0 * cols + 8 * i, v);
          float4 *d = reinterpret_cast<float4 *>(xs + 8 * i);
          d[0] = make_float4(v[0], v[1], v[2], v[3]);
          d[1] = make_float4(v[4], v[5], v[6], v[7]);
          if constexpr (GEN) {
            if (norm_w) {
              float s = 0.f;
#pragma unroll
              for (int c = 0; c < 8; ++c) s = fmaf(v[c], v[c], s);
              const int tr = static_cast<int>(8 * i / cols);
#pragma unroll
              for (int mb = 0; mb < MB; ++mb) ss[mb] += tr == mb ? s : 0.f;
            }
          }
        }
        if constexpr (GEN) {
          if (norm_w) {
            group_reduce<64>(ss);
            if (lane == 0)
#pragma unroll
              for (int mb = 0; mb < MB; ++mb) norm_red[threadIdx.x >> 6][mb] = ss[mb];
            __syncthreads();
            float rs[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
              float t = 0.f;
#pragma unroll
              for (int w = 0; w < NT / 64; ++w) t += norm_red[w][mb];
              rs[mb] = 1.0f / sqrtf(t / static_cast<float>(cols) + targets.norm_eps);
            }
            for (int64_t i = threadIdx.x; i < mb_here * cols / 8; i += NT) {
              const int tr = static_cast<int>(8 * i / cols);
              const int64_t c8 = 8 * i - static_cast<int64_t>(tr) * cols;
              float r = rs[0];
#pragma unroll
              for (int mb = 1; mb < MB; ++mb) r = tr == mb ? rs[mb] : r;
              float4 *d = reinterpret_cast<float4 *>(xs + 8 * i);
              const float4 g0 = gload16f(norm_w + c8), g1 = gload16f(norm_w + c8 + 4);
              const float4 a = d[0], b = d[1];
              d[0] = make_float4(a.x * r * g0.x, a.y * r * g0.y, a.z * r * g0.z, a.w * r * g0.w);
              d[1] = make_float4(b.x * r * g1.x, b.y * r * g1.y, b.z * r * g1.z, b.w * r * g1.w);
            }
          }
        }
      }
    }
    __syncthreads();
    float acc[MB][4];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[mb][t] = 0.f;
    if (live) {
      // block-local 32-bit atom indices (the staged groups hold < 2^31 atoms)
      const int apr32 = static_cast<int>(atoms_per_row);
      const int nbase = static_cast<int>(row * atoms_per_row - (PL ? atom0 : g_lo * 4));  // atom index in the stage
      for (int a0 = sub; a0 < apr32; a0 += kDqlGather * L) {
        uint4 e[kDqlGather];
#pragma unroll
        for (int i = 0; i < kDqlGather; ++i) {
          const int a = a0 + i * L;
          if constexpr (PL) {
            const uint16_t *rp = reinterpret_cast<const uint16_t *>(pb + 6 * (nbase + min(a, apr32 - 1)));
            const uint32_t r0 = rp[0], r1 = rp[1], r2 = rp[2];
            const uint32_t pos = ((r1 >> 13) & 7u) | ((r2 >> 13) & 3u) << 3;
            constexpr uint32_t kLast = TPT * NT * 4 - 1;  // clamped to the staged table (any layout stays inside)
            e[i] = make_uint4(ptab[min(r0 & 0x1FFFu, kLast)], ptab[min(r1 & 0x1FFFu, kLast)],
                              ptab[min(r2 & 0x1FFFu, kLast)], ((r0 >> 13) & 3u) | pos << 8);
            continue;
          }
          int32_t code = 0;
          if (a < apr32) {
            const int n = nbase + a;
            const uint8_t *bp = pb + (n >> 2) * 9 + 2 * (n & 3);
            const uint32_t v = (static_cast<uint32_t>(bp[0]) << 16) | (static_cast<uint32_t>(bp[1]) << 8) | bp[2];
            code = static_cast<int32_t>((v >> (6 - 2 * (n & 3))) & 0x3FFFFu);
            if (code > kKissing) code = 0;
          }
          e[i] = kp_gemv[code];
        }
#pragma unroll
        for (int i = 0; i < kDqlGather; ++i) {
          const int a = a0 + i * L;
          if (a >= apr32) break;
          const uint32_t type = e[i].w & 3u;
          const int pos = static_cast<int>((e[i].w >> 8) & 31u);
          const uint32_t cw[3] = {e[i].x, e[i].y, e[i].z};
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            if (mb >= mb_here) break;
            const int64_t xoff = (XL ? mb * cols : (m0 + mb) * cols) + a * kDim;
            float D = 0.f;
#pragma unroll
            for (int p = 0; p < 3; ++p) {
              float xv[8];
              if (XL) {
                const float4 *q4 = reinterpret_cast<const float4 *>(xs + xoff + 8 * p);
                const float4 u = q4[0], w = q4[1];
                xv[0] = u.x; xv[1] = u.y; xv[2] = u.z; xv[3] = u.w; xv[4] = w.x; xv[5] = w.y; xv[6] = w.z; xv[7] = w.w;
              } else {
                load_x8<XF32>(x, xoff + 8 * p, xv);
              }
#pragma unroll
              for (int c = 0; c < 8; ++c) {
                const int k = static_cast<int>(static_cast<int32_t>(cw[p] << (28 - 4 * c)) >> 28);  // signed nibble
                D = fmaf(static_cast<float>(k), xv[c], D);
              }
            }
            const float xp = XL ? xs[xoff + pos] : x_at<XF32>(x, xoff + pos);
            acc[mb][0] += type == 1u ? D : 0.f;
            acc[mb][1] += type == 2u ? D : 0.f;
            acc[mb][2] += type == 3u ? fmaf(3.f, xp, D) : 0.f;
            acc[mb][3] += type == 3u ? xp : 0.f;
          }
        }
      }
    }
    // reduce the L lanes of each row
    {
      float flat[MB * 4];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int t = 0; t < 4; ++t) flat[4 * mb + t] = acc[mb][t];
      group_reduce<L>(flat);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[mb][t] = flat[4 * mb + t];
    }
    if (writer) {
      const float sig = __half2float(__ushort_as_half(sig_bits));
      const float sl = __uint_as_float(kSLatticeBits);
      const float v1 = __half2float(__ushort_as_half(static_cast<uint16_t>(dq_value(1, sig, sl))));
      const float v2 = __half2float(__ushort_as_half(static_cast<uint16_t>(dq_value(2, sig, sl))));
      const float v3 = __half2float(__ushort_as_half(static_cast<uint16_t>(dq_value(3, sig, sl))));
      const float v4 = __half2float(__ushort_as_half(static_cast<uint16_t>(dq_value(4, sig, sl))));
      const float m1 = round_w ? bf16_bits_to_float(bf16_rne_bits(v1)) : v1;
      const float m2 = round_w ? bf16_bits_to_float(bf16_rne_bits(v2)) : v2;
      const float m3 = round_w ? bf16_bits_to_float(bf16_rne_bits(v3)) : v3;
      const float m4 = round_w ? bf16_bits_to_float(bf16_rne_bits(v4)) : v4;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        if (mb < mb_here) {
          const int64_t i = (m0 + mb) * rows + row;
          float v = m4 * (acc[mb][0] * 0.25f) + m2 * (acc[mb][1] * 0.5f) + m1 * acc[mb][2] - m3 * acc[mb][3];
          if constexpr (GEN) {
            // GELU (torch's erf form), then the residual (prefetched for the first tokens)
            if (gelu) v = (v * 0.5f) * (1.0f + erff(v * __uint_as_float(kSLatticeBits)));
            if (residual) v = (m0 == 0 ? res0[mb] : gload(residual + i)) + v;
          }
          gstore(y + i, v);
        }
    }
  }
}

// One token of bf16 activations, one target, no epilogue (the plain GEMV
// call): the arithmetic of dqlinear_kernel<L, 1> with three changes.
// - Codes as bf16 pairs from a table of halves: the codebook rows' 8-coordinate
//   planes take only 161 distinct 4-coordinate halves, so gv_tab holds each
//   half as two bf16 pairs (raw integers, exact) and each plane as two half
//   symbols; the block stages it in LDS (11.3 KB with the plane entries, 1.3
//   KB without) and v_dot2_f32_bf16 multiplies the looked-up pairs by the bf16
//   x pairs (exact products, fp32 sums in the fixed order pairs 0,1 | 2,3 |
//   4,5 | 6,7 per plane).  Nothing is decoded per atom: a code (packed stream)
//   gathers its 8-byte kp_half entry (6 half symbols, type, position of -3), a
//   plane-layout record its plane's two symbols from LDS.  (The half table
//   replaced v_perm_b32 expansion of 3-bit value ids, 11 VALU instructions per
//   plane, and the 19.8 KB table of plane value ids.)
// - It is written so that the compiler issues one round of loads (packed
//   bytes as raw buffer loads, sigma16, x, the table), one barrier, then the
//   rounds of LDS reads and gathers: every thread stores to LDS (no load sits
//   under a branch) and atoms past the row decode as the origin (no branch
//   per atom).
// - The epilogue's four dequantized values of the row scale are computed by
//   four lanes of the row (one each) and broadcast within the quad by DPP.
// Measured in a graph of 200 calls on distinct copies: value-id expansion
// 5.40 / 5.43 us (7680 x 1920 / 1920 x 7680), and probe copies attributed
// 0.44 us to the expansion and 0.23 us to staging the plane value ids.  fp32
// activations keep dqlinear_kernel (this layout measured the same there).
constexpr int kG1Atoms = 5;  // atoms per lane
// PL: `packed` is the plane layout (3 uint16 records per atom: plane index |
// extra bits << 13): the plane's two half symbols come from the staged table.
template <int L, bool PL>
__global__ __launch_bounds__(512) void dqgemv1_kernel(const uint8_t *__restrict__ packed, int packed_bytes,
                                                      const uint16_t *__restrict__ sigma16, int rows, int apr,
                                                      const uint16_t *__restrict__ x, const uint2 *__restrict__ kp_half,
                                                      const uint4 *__restrict__ gv_tab, int round_w,
                                                      float *__restrict__ y) {
  constexpr int NT = 512, R = NT / L, G = kG1Atoms;
  constexpr int VPT = PL ? 2 : 1;   // staged 16-byte vectors of the block's atom bytes per thread
  constexpr int TV = PL ? kGvVecs : kGvHalfVecs;  // table vectors staged (PL: halves and plane entries)
  constexpr int TPT = (TV + NT - 1) / NT;         // per thread
  static_assert(L >= 8, "the epilogue takes its four values from the row's first quad");
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  const int sub = tid % L;
  const int row0 = static_cast<int>(blockIdx.x) * R;
  const int row = row0 + tid / L;
  const int rows_here = min(R, rows - row0);
  const int cols = apr * kDim;
  // the block's atom bytes as aligned 16-byte vectors (the host checks nvec <= VPT * NT):
  // whole 9-byte groups [g_lo, g_hi) of the packed stream, or 6 bytes per atom of the plane layout
  const int atom0 = row0 * apr;
  const int g_lo = atom0 >> 2, g_hi = (atom0 + rows_here * apr + 3) >> 2;
  const int start = PL ? 6 * atom0 : g_lo * 9, end = PL ? 6 * (atom0 + rows_here * apr) : g_hi * 9;
  const int base16 = start & ~15;
  const int nvec = (end - base16 + 15) >> 4;
  const int pb_off = start - base16;
  // LDS: VPT NT atom-byte vectors, 2 NT pieces of 8 bf16 x values, TPT NT table vectors;
  // every thread stores all its slots, so no load sits under a branch
  uint16_t *xh = reinterpret_cast<uint16_t *>(smem + VPT * NT * 16);
  uint4 *tabs = reinterpret_cast<uint4 *>(smem + VPT * NT * 16 + 2 * NT * 16);
  const uint2 *hp = reinterpret_cast<const uint2 *>(tabs);                    // [kGvHalves] half pairs
  const uint16_t *php = reinterpret_cast<const uint16_t *>(tabs + kGvHalfVecs);  // [kGvPlanes] (PL)
  // round of loads: atom bytes, table, sigma16, x pieces.  The buffer range covers the
  // stream rounded up to whole dwords (a dword reaching past the range reads as zero; the last
  // dword lies in the same page as the stream's last byte, the base being 16-byte aligned);
  // dwords wholly past it read as zero.
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(packed), static_cast<short>(0), (packed_bytes + 3) & ~3, 0x00020000);
  uint32_t d[VPT][4];
#pragma unroll
  for (int v = 0; v < VPT; ++v) {
    const int vi = tid + v * NT;
    int poff = vi < nvec ? base16 + 16 * vi : 0x7FFFFFF0;
    asm("" : "+v"(poff));
#pragma unroll
    for (int k = 0; k < 4; ++k) d[v][k] = __builtin_amdgcn_raw_buffer_load_b32(prs, poff + 4 * k, 0, 0);
  }
  uint4 tq[TPT];
#pragma unroll
  for (int v = 0; v < TPT; ++v) {
    const int vi = tid + v * NT;
    tq[v] = gv_tab[vi < TV ? vi : 0];
  }
  const uint16_t sig_bits = sigma16[row < rows ? row : rows - 1];
  const int items = cols / 8;  // pieces of x (the host checks items <= 2 * NT)
  uint4 xq[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int it = tid + h * NT;
    xq[h] = reinterpret_cast<const uint4 *>(x)[it < items ? it : 0];
  }
#pragma unroll
  for (int v = 0; v < VPT; ++v) reinterpret_cast<uint4 *>(smem)[tid + v * NT] = make_uint4(d[v][0], d[v][1], d[v][2], d[v][3]);
#pragma unroll
  for (int h = 0; h < 2; ++h) reinterpret_cast<uint4 *>(xh)[tid + h * NT] = xq[h];  // pieces past x: unused slots
#pragma unroll
  for (int v = 0; v < TPT; ++v) tabs[tid + v * NT] = tq[v];
  __syncthreads();
  float sig = __half2float(__ushort_as_half(sig_bits));
  asm volatile("" : "+v"(sig));  // keeps the sigma16 load in the first round (else it sinks into the epilogue)
  const int lrow = min(tid / L, rows_here - 1);
  uint32_t hs[G][3];  // per atom and plane: its two half symbols (lo | hi << 8)
  uint32_t meta[G];   // per atom: type | position of -3 << 8
  if constexpr (PL) {
    // round of LDS reads: the lane's atoms' 3 records, then their planes' half symbols
    uint32_t r[G][3];
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int off = pb_off + 6 * (lrow * apr + min(sub + i * L, apr - 1));
      const uint16_t *rp = reinterpret_cast<const uint16_t *>(smem + off);
      r[i][0] = rp[0];
      r[i][1] = rp[1];
      r[i][2] = rp[2];
    }
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const bool in = sub + i * L < apr;
      const uint32_t type = in ? (r[i][0] >> 13) & 3u : 0u;
      const uint32_t pos = ((r[i][1] >> 13) & 7u) | ((r[i][2] >> 13) & 3u) << 3;
      // (clamped to the staged entries: a layout not made by plane_layout_kernel cannot index past them)
#pragma unroll
      for (int k = 0; k < 3; ++k) hs[i][k] = php[min(r[i][k] & 0x1FFFu, static_cast<uint32_t>(kGvPlanes - 1))];
      meta[i] = type | pos << 8;
    }
  } else {
    // round of LDS reads: the lane's atoms sub, sub + L, ... (clamped to the block's atoms), 3 bytes
    // each from two aligned words; then the round of kp_half gathers
    const int nbase = lrow * apr + (atom0 - g_lo * 4);
    uint32_t w0[G], w1[G];
    int nn[G];
#pragma unroll
    for (int i = 0; i < G; ++i) {
      nn[i] = nbase + min(sub + i * L, apr - 1);
      const int off = pb_off + (nn[i] >> 2) * 9 + 2 * (nn[i] & 3);
      const uint32_t *wp = reinterpret_cast<const uint32_t *>(smem + (off & ~3));
      w0[i] = wp[0];
      w1[i] = wp[1];
    }
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int n = nn[i];
      const uint32_t o = static_cast<uint32_t>((pb_off + (n >> 2) * 9 + 2 * (n & 3)) & 3);
      const uint32_t v = __builtin_amdgcn_perm(w1[i], w0[i], (o + 2) | ((o + 1) << 8) | (o << 16) | 0x0C000000u);
      int32_t code = static_cast<int32_t>((v >> (6 - 2 * (n & 3))) & 0x3FFFFu);
      if (code > kKissing || sub + i * L >= apr) code = 0;
      const uint2 kh = kp_half[code];
      hs[i][0] = kh.x & 0xFFFFu;
      hs[i][1] = kh.x >> 16;
      hs[i][2] = kh.y & 0xFFFFu;
      meta[i] = kh.y >> 16;
    }
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int a = min(sub + i * L, apr - 1);
    const uint32_t type = meta[i] & 3u;
    const int pos = static_cast<int>((meta[i] >> 8) & 31u);
    float D = 0.f;
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const uint2 lo = hp[hs[i][p] & 0xFFu], hi = hp[(hs[i][p] >> 8) & 0xFFu];
      const uint4 xv = *reinterpret_cast<const uint4 *>(xh + a * kDim + 8 * p);
      D = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, lo.x), __builtin_bit_cast(bf16x2_t, xv.x), D, false);
      D = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, lo.y), __builtin_bit_cast(bf16x2_t, xv.y), D, false);
      D = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, hi.x), __builtin_bit_cast(bf16x2_t, xv.z), D, false);
      D = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, hi.y), __builtin_bit_cast(bf16x2_t, xv.w), D, false);
    }
    const float xp = __uint_as_float(static_cast<uint32_t>(xh[a * kDim + pos]) << 16);
    acc[0] += type == 1u ? D : 0.f;
    acc[1] += type == 2u ? D : 0.f;
    acc[2] += type == 3u ? fmaf(3.f, xp, D) : 0.f;
    acc[3] += type == 3u ? xp : 0.f;
  }
  group_reduce<L>(acc);
  // lane sub & 3 of the row's first quad computes the dequantized value of raw coordinate 1 + (sub & 3)
  const float vk = __half2float(__ushort_as_half(static_cast<uint16_t>(
      dq_value(1 + (sub & 3), sig, __uint_as_float(kSLatticeBits)))));
  const float mk = round_w ? bf16_bits_to_float(bf16_rne_bits(vk)) : vk;
  const float m1 = dpp_f32<0x00>(mk), m2 = dpp_f32<0x55>(mk), m3 = dpp_f32<0xAA>(mk), m4 = dpp_f32<0xFF>(mk);
  if (sub == 0 && row < rows) y[row] = m4 * (acc[0] * 0.25f) + m2 * (acc[1] * 0.5f) + m1 * acc[2] - m3 * acc[3];
}

// packed 18-bit indices -> the plane layout: per atom the 3 records of its code
__global__ __launch_bounds__(256) void plane_layout_kernel(const uint8_t *__restrict__ packed, int64_t n_atoms,
                                                           const uint16_t *__restrict__ code_planes,
                                                           uint16_t *__restrict__ planes) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (n >= n_atoms) return;
  int32_t code = packed_index(packed, n);
  if (code > kKissing) code = 0;
  const uint2 r = *reinterpret_cast<const uint2 *>(code_planes + static_cast<int64_t>(code) * 4);
  planes[3 * n] = static_cast<uint16_t>(r.x & 0xFFFFu);
  planes[3 * n + 1] = static_cast<uint16_t>(r.x >> 16);
  planes[3 * n + 2] = static_cast<uint16_t>(r.y & 0xFFFFu);
}

// One token of bf16 x from the plane layout (dqgemv1_kernel<L, true>): L lanes per row by row
// length as in launch_dql; rows of more than 320 atoms are refused (the packed stream takes them).
template <int L>
int launch_gemv1_planes_l(const uint8_t *planes, const uint16_t *sigma16, int64_t rows, int64_t apr, const void *x,
                          const DeviceTables *tab, int round_w, float *y, hipStream_t s) {
  constexpr int NT = 512, R = NT / L;
  const int64_t blocks = (rows + R - 1) / R;
  const int64_t nvec_max = (6 * R * apr + 31) / 16;
  static_assert(kGvVecs <= 2 * NT, "the GEMV table fits its two LDS slots per thread");
  if (apr > static_cast<int64_t>(kG1Atoms) * L || nvec_max > 2 * NT || apr * kDim / 8 > 2 * NT ||
      6 * rows * apr >= (static_cast<int64_t>(1) << 30))
    return fail(PLX_EINVAL, "dequant_linear: the plane layout takes rows of at most %d atoms at one token (got %lld)",
                kG1Atoms * 64, static_cast<long long>(apr));
  hipLaunchKernelGGL((dqgemv1_kernel<L, true>), dim3(static_cast<unsigned>(blocks)), dim3(NT),
                     static_cast<size_t>(NT) * (32 + 32 + 32), s, planes, static_cast<int>(6 * rows * apr), sigma16,
                     static_cast<int>(rows), static_cast<int>(apr), static_cast<const uint16_t *>(x),
                     static_cast<const uint2 *>(nullptr), tab->gv_tab, round_w, y);
  return check_launch("dqgemv1_kernel");
}

int launch_gemv1_planes(const uint8_t *planes, const uint16_t *sigma16, int64_t rows, int64_t apr, const void *x,
                        const DeviceTables *tab, int round_w, float *y, hipStream_t s) {
  if (apr >= 160) return launch_gemv1_planes_l<64>(planes, sigma16, rows, apr, x, tab, round_w, y, s);
  // 16 lanes (32 rows per block) only while a lane's share is at most kG1Atoms atoms and the
  // block's records fit its 2 vectors per thread
  if (apr >= 16)
    return (rows + 31) / 32 < 192 || apr > static_cast<int64_t>(kG1Atoms) * 16 || 6 * 32 * apr + 31 > 16 * 2 * 512
               ? launch_gemv1_planes_l<32>(planes, sigma16, rows, apr, x, tab, round_w, y, s)
               : launch_gemv1_planes_l<16>(planes, sigma16, rows, apr, x, tab, round_w, y, s);
  return launch_gemv1_planes_l<8>(planes, sigma16, rows, apr, x, tab, round_w, y, s);
}

// t.norm_w (fp32 x only): x is normalised in the kernel when its rows fit in
// LDS, else by rmsnorm into xnorm ([m, cols] fp32) first.
// PL: the targets' `packed` are plane layouts (one token; always the general kernel).
template <int L, bool XF32, int NT, bool PL = false>
int launch_dql(DqlTargets t, int64_t apr, const void *x, int64_t m, const uint4 *tab, const DeviceTables *dtab, int round_w,
               int gelu, float *xnorm, hipStream_t s, const uint32_t *pl_nib = nullptr, int pl_vecs = 0) {
  constexpr int R = NT / L;
  int64_t blocks = 0;
  for (int i = 0; i < t.n; ++i) blocks = max(blocks, (t.rows[i] + R - 1) / R);
  if (blocks == 0) return PLX_OK;
  if (blocks > 0x7FFFFFFFll) return fail(PLX_EINVAL, "dequant_linear: too many rows");
  const dim3 g(static_cast<unsigned>(blocks), static_cast<unsigned>(t.n));
  const DqlOne one{t.packed[0], t.packed_bytes[0], t.sigma16[0], t.rows[0], t.y[0]};
  const size_t pbytes = static_cast<size_t>((R * apr + 8) / 4 + 2) * 9;
  const size_t p16 = ((pbytes + 15) & ~static_cast<size_t>(15)) + 16;  // + one vector of alignment slack
  const int64_t cols = apr * kDim;
  const int mb = m >= 4 ? 4 : m >= 2 ? 2 : 1;
  const size_t xbytes = static_cast<size_t>(mb) * cols * 4;
  // PL: records (kDqlPlVecs * 512 vectors, all stored), x when it fits, the plane table
  const size_t prec = static_cast<size_t>(kDqlPlVecs) * 512 * 16;
  const bool xl = PL ? xbytes <= 48 * 1024 : p16 + xbytes <= 48 * 1024;
  const size_t shm = PL ? prec + (xl ? xbytes : 0) + static_cast<size_t>(kDqlPlTableVecs) * 16 : xl ? p16 + xbytes : p16;
  if (PL && (m != 1 || (6 * R * apr + 31) / 16 > kDqlPlVecs * 512 || pl_vecs > kDqlPlTableVecs))
    return fail(PLX_EINVAL, "dequant_linear: the plane layout takes one token and rows of at most %d atoms here",
                kDqlPlVecs * 512 * 16 / (6 * R) - 1);
  for (int i = 0; PL && i < t.n; ++i)  // 32-bit buffer offsets
    if (t.packed_bytes[i] >= (static_cast<int64_t>(1) << 30))
      return fail(PLX_EINVAL, "dequant_linear: plane layouts of 2^30 bytes or more are not read at one token");
  if (shm > (PL ? 96 : 64) * 1024)
    return fail(PLX_EINVAL, "dequant_linear: rows of %lld atoms are too long", static_cast<long long>(apr));
  // x through registers: one pass over all tokens, at most one 8-value piece per thread
  const bool xreg = xl && m <= mb && m * cols <= 8 * NT;
  if (t.norm_w && !xl) {
    const int st = launch_rms_norm(static_cast<const float *>(x), t.norm_w, xnorm, m, cols, t.norm_eps, s);
    if (st != PLX_OK) return st;
    x = xnorm;
    t.norm_w = nullptr;
  }
  const bool gen = PL || t.n > 1 || t.residual[0] != nullptr || gelu || t.norm_w != nullptr;
  if constexpr (NT == 512 && !XF32 && !PL) {
    // one token of bf16 x, one target: dqgemv1_kernel (at most kG1Atoms atoms per lane, int offsets)
    const int64_t nvec_max = (R * apr / 4 + 2) * 9 / 16 + 2;
    if (!gen && m == 1 && apr >= 1 && apr <= static_cast<int64_t>(kG1Atoms) * L && nvec_max <= NT &&
        cols / 8 <= 2 * NT && t.packed_bytes[0] < (static_cast<int64_t>(1) << 30) &&
        t.rows[0] < (static_cast<int64_t>(1) << 30)) {
      hipLaunchKernelGGL((dqgemv1_kernel<L, false>), g, dim3(NT), static_cast<size_t>(NT) * (16 + 32 + 16), s,
                         t.packed[0], static_cast<int>(t.packed_bytes[0]), t.sigma16[0], static_cast<int>(t.rows[0]),
                         static_cast<int>(apr), static_cast<const uint16_t *>(x), dtab->kp_half, dtab->gv_tab, round_w,
                         t.y[0]);
      return check_launch("dqgemv1_kernel");
    }
  }
#define PLX_DQL(MB, XL, XR) \
  do {                                                                                                          \
    if (gen)                                                                                                    \
      hipLaunchKernelGGL((dqlinear_kernel<L, MB, XF32, XL, NT, true, XR>), g, dim3(NT), shm, s, t, apr, x, m, tab, \
                         round_w, gelu, nullptr, 0);                                                             \
    else                                                                                                        \
      hipLaunchKernelGGL((dqlinear_kernel<L, MB, XF32, XL, NT, false, XR>), g, dim3(NT), shm, s, one, apr, x, m,  \
                         tab, round_w, 0, nullptr, 0);                                                           \
  } while (0)
  if constexpr (PL) {
    if (xreg)
      hipLaunchKernelGGL((dqlinear_kernel<L, 1, XF32, true, NT, true, true, true>), g, dim3(NT), shm, s, t, apr, x, m,
                         tab, round_w, gelu, pl_nib, pl_vecs);
    else if (xl)
      hipLaunchKernelGGL((dqlinear_kernel<L, 1, XF32, true, NT, true, false, true>), g, dim3(NT), shm, s, t, apr, x,
                         m, tab, round_w, gelu, pl_nib, pl_vecs);
    else
      hipLaunchKernelGGL((dqlinear_kernel<L, 1, XF32, false, NT, true, false, true>), g, dim3(NT), shm, s, t, apr, x,
                         m, tab, round_w, gelu, pl_nib, pl_vecs);
    return check_launch("dqlinear_kernel");
  }
  if (mb == 4) {
    if (xreg) PLX_DQL(4, true, true); else if (xl) PLX_DQL(4, true, false); else PLX_DQL(4, false, false);
  } else if (mb == 2) {
    if (xreg) PLX_DQL(2, true, true); else if (xl) PLX_DQL(2, true, false); else PLX_DQL(2, false, false);
  } else {
    if (xreg) PLX_DQL(1, true, true); else if (xl) PLX_DQL(1, true, false); else PLX_DQL(1, false, false);
  }
#undef PLX_DQL
  return check_launch("dqlinear_kernel");
}

// ---------------------------------------------------------------------------
// dequant-GEMM: y[m, r] = sum_i x[m, i] W[r, i] on MFMA for bf16 activations.
//
// EXACT (the default): W[r, i] = +-v_|k| (fp16, 11 significant bits) is split
// exactly into two bf16 values, W = hi + lo (hi = bf16_rne(W); lo = W - hi has
// <= 3 significant bits), so two v_mfma_f32_16x16x32_bf16 per tile give exact
// products of the bf16 activations with the fp16 weights, accumulated in fp32:
// the numerics of F.linear(x.float(), W.float()).  Without EXACT only hi is
// used: the products of the reference's literal F.linear(x, W.to(x.dtype))
// (pollux.py:507), which rounds the fp16 weight to bf16 first (RNE is odd, so
// the row's 8-entry table of signed values holds bf16(+-v_|k|)).
//
// Block: WV waves, 32 output rows (two MFMA B tiles of 16) x 16*MT tokens
// (MFMA A tiles), over `apb` atoms of every row (the whole row when that
// fills the chip; otherwise the grid splits K into `splits` ranges and
// dqmm_reduce_kernel sums the split partial tiles in split order).
//   prologue: decode the block's 32 x apb codes from the packed stream and
//             fetch their kp_dq words (3 per code) into LDS; 32 lanes build
//             the 8-entry bf16 byte tables (hi, and lo when EXACT) of the
//             block's rows;
//   k loop:   each wave takes a contiguous share of the block's atoms in
//             quads of 4 (= 3 K steps of 32) and reads its activation
//             fragments (up to 32 bf16 tokens: from x in place; otherwise
//             from a fragment-order copy that a small kernel writes first,
//             fp32 x as three bf16 parts; L2-resident either way: every block
//             reads all of it), PD quads ahead in registers; per K step a
//             lane decodes its B fragments (8 weights of one row = one plane
//             of one atom) from one LDS word with v_perm_b32 byte lookups and
//             issues 2*MT MFMAs (4*MT when EXACT).  No block barrier inside
//             the loop.
//   epilogue: the waves' fp32 tiles are summed through LDS in wave order.
// When the copy is used, xfrag_kernel runs first and writes it into the
// caller's workspace.
// Summing the splits inside this kernel instead (the last split block of a row
// block adds the others' tiles) measured slower both ways it can be made
// coherent across XCDs: with a device fence (which writes back and
// invalidates the XCD's whole L2) 3x, with device-scope atomic stores and
// loads of the tiles 1.35x.
// One block per 32 rows keeps the decode of every weight in one lane and
// fills the chip without a K split for wide layers (7680 rows: 240 blocks);
// the cost is that each block reads all of x from L2.
// Tokens >= m and columns >= cols are zero-filled (so no NaN from outside the
// operands can reach a valid output); atoms >= atoms_per_row and rows >= rows
// decode as the origin (weight 0).
// ---------------------------------------------------------------------------

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMmRows = 32;             // output rows per block
constexpr int kMmMaxApb = 128;          // atoms of a row per block (kp_dq tile: 32 x 388 words = 49.7 KB)
constexpr int kMmTargetBlocks = 192;    // K is split until the grid holds about this many blocks,
constexpr int kMmNoSplitBlocks = 176;   // unless the rows alone give this many (the 5,760-row stacked q/k/v:
                                        // 180 blocks unsplit beat 360 + the split sum at 16 and 64 tokens)
constexpr int kMmRedStride = 36;        // floats per token in the cross-wave sum (conflict-free writes)
constexpr int kXfQuadBytes = 3 * 4 * 1024;       // fragment-order x: 3 K steps x 4 token tiles x 64 lanes x 16 B
constexpr int64_t kMmMaxCols = 1 << 22;           // a slab of fragment-order x (3 parts) stays below 2^31 bytes

// Words per row of the block's kp_dq tile: 3 per atom, padded to 4 mod 8 so the
// 16 rows of a B tile read by one instruction fall into distinct banks.
__host__ __device__ constexpr int mm_row_words(int apb) { return ((3 * apb + 7) & ~7) + 4; }

// 24-bit big-endian window of atom n read as two aligned dwords (bounds-checked
// at the stream's tail), then the 18-bit index.
__device__ __forceinline__ int32_t packed_index_dw(const uint8_t *__restrict__ packed, int64_t packed_bytes,
                                                   int64_t n) {
  const int64_t b = (n >> 2) * 9 + 2 * (n & 3);
  const int64_t b4 = b & ~static_cast<int64_t>(3);
  uint32_t v;
  if (b4 + 8 <= packed_bytes) {
    const uint32_t w0 = *reinterpret_cast<const uint32_t *>(packed + b4);
    const uint32_t w1 = *reinterpret_cast<const uint32_t *>(packed + b4 + 4);
    const uint32_t o = static_cast<uint32_t>(b & 3);
    v = __builtin_amdgcn_perm(w1, w0, (o + 2) | ((o + 1) << 8) | (o << 16) | 0x0C000000u);
  } else {
    v = 0;
    for (int k = 0; k < 3; ++k) v = (v << 8) | (b + k < packed_bytes ? packed[b + k] : 0u);
  }
  return static_cast<int32_t>((v >> (6 - 2 * (n & 3))) & 0x3FFFFu);
}

// 8 bf16 of one plane from a kp_dq word and a row's 4-word byte table.
__device__ __forceinline__ bf16x8_t perm_decode(uint32_t w, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  const uint32_t s_lo = w & 0x0F0F0F0Fu, s_hi = (w >> 4) & 0x0F0F0F0Fu;
  const uint32_t l_lo = __builtin_amdgcn_perm(t1, t0, s_lo), h_lo = __builtin_amdgcn_perm(t3, t2, s_lo);
  const uint32_t l_hi = __builtin_amdgcn_perm(t1, t0, s_hi), h_hi = __builtin_amdgcn_perm(t3, t2, s_hi);
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  const u4 r = {__builtin_amdgcn_perm(h_lo, l_lo, 0x05010400u), __builtin_amdgcn_perm(h_lo, l_lo, 0x07030602u),
                __builtin_amdgcn_perm(h_hi, l_hi, 0x05010400u), __builtin_amdgcn_perm(h_hi, l_hi, 0x07030602u)};
  return __builtin_bit_cast(bf16x8_t, r);
}

// Four codes of one 9-byte packed group from the three dwords covering it
// (o = byte offset of the group in the first dword).
__device__ __forceinline__ void group_codes(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t o, int32_t *c) {
  const uint32_t sel = (o + 3) | ((o + 2) << 8) | ((o + 1) << 16) | (o << 24);
  const uint32_t hi = __builtin_amdgcn_perm(d1, d0, sel);  // B0 B1 B2 B3, big-endian
  const uint32_t lo = __builtin_amdgcn_perm(d2, d1, sel);  // B4 B5 B6 B7
  const uint32_t b8 = (d2 >> (8 * o)) & 0xFFu;
  c[0] = static_cast<int32_t>(hi >> 14);
  c[1] = static_cast<int32_t>(((hi & 0x3FFFu) << 4) | (lo >> 28));
  c[2] = static_cast<int32_t>((lo >> 10) & 0x3FFFFu);
  c[3] = static_cast<int32_t>(((lo & 0x3FFu) << 8) | b8);
}

// Fragment-order copy of the activations for dqmm_kernel (fp32 x, and bf16 x
// above 32 tokens).  One thread per 16-byte fragment position (slab, quad Q,
// K step s, token tile t, lane): x[64 slab + 16t + (lane & 15)][96Q + 32s +
// 8(lane >> 4) .. +8), zero for tokens >= m and columns >= cols (token tiles
// t >= `tiles`, which the GEMM does not read, are not written), stored at
// xf[slab][Q][part][s][t][lane].  bf16 x is one part.  fp32 x is split
// exactly into three bf16 parts, x = h + m + l (h = bf16(x), m = bf16(x - h),
// l = x - h - m, exact while the parts stay normal, |x| >= ~2^-110; inf / nan
// go to h alone), so that bf16 MFMAs form the products of the fp32
// activations.
template <bool XF32>
__global__ __launch_bounds__(256) void xfrag_kernel(const void *__restrict__ x, int64_t m_total, int64_t cols,
                                                    int64_t n_quads_row, int tiles, uint4 *__restrict__ xf) {
  constexpr int XP = XF32 ? 3 : 1;
  constexpr int kQuadFrags = kXfQuadBytes / 16;  // 768 per part
  const int64_t per_slab = n_quads_row * kQuadFrags;
  const int64_t f = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // fragment position within the slab
  if (f >= per_slab) return;
  const int lane = static_cast<int>(f & 63);
  const int64_t rest = f >> 6;  // (3Q + s) * 4 + t
  const int t = static_cast<int>(rest & 3);
  if (t >= tiles) return;  // a token tile the GEMM does not read (it reads `tiles` per slab)
  const int64_t qs = rest >> 2;  // 3Q + s
  const int64_t quad = qs / 3, within = f - quad * kQuadFrags;
  const int64_t tok = static_cast<int64_t>(blockIdx.y) * 64 + 16 * t + (lane & 15);
  const int64_t col = 32 * qs + 8 * (lane >> 4);
  uint4 *dst = xf + static_cast<int64_t>(blockIdx.y) * per_slab * XP + quad * XP * kQuadFrags + within;
  const bool live = tok < m_total && col < cols;
  if constexpr (!XF32) {
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (live) v = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(x) + tok * cols + col);
    dst[0] = v;
  } else {
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (live) {
      const float4 *src = reinterpret_cast<const float4 *>(static_cast<const float *>(x) + tok * cols + col);
      const float4 a = src[0], b = src[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    uint32_t part[3][4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      uint32_t hb[2], mb[2], lb[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const float xv = v[e + u];
        hb[u] = bf16_rne_bits(xv);
        mb[u] = lb[u] = 0u;
        if (fabsf(xv) <= 3.0e38f) {
          const float r1 = xv - __uint_as_float(hb[u] << 16);
          mb[u] = bf16_rne_bits(r1);
          lb[u] = bf16_rne_bits(r1 - __uint_as_float(mb[u] << 16));
        }
      }
      part[0][e / 2] = hb[0] | (hb[1] << 16);
      part[1][e / 2] = mb[0] | (mb[1] << 16);
      part[2][e / 2] = lb[0] | (lb[1] << 16);
    }
#pragma unroll
    for (int pp = 0; pp < 3; ++pp) dst[pp * kQuadFrags] = make_uint4(part[pp][0], part[pp][1], part[pp][2], part[pp][3]);
  }
}

// RMS norm of fp32 token rows written straight into the fragment-order copy:
// rmsnorm_kernel (decode.hip) and xfrag_kernel<true> in one launch, with the
// same values (the sum of squares in rmsnorm_kernel's order: lane l holds
// float4 l + 64k of the row, fmaf over k and the four components, then the
// wave sum).  One wave per token row of each 64-token slab; rows >= m write
// zeros, rows of token tiles the GEMM does not read (t >= tiles) nothing.  Fragment 32k + j holds the row's columns 8(32k + j) .. +8, i.e.
// float4s 64k + 2j and 64k + 2j + 1: lanes 2j and 2j + 1 each write their
// 8-byte half of the fragment in every part.  Rows of up to 32 * kNfVec
// fragments (kNfVec * 256 columns, padding of the last quad included).
constexpr int kNfVec = 8;
__global__ __launch_bounds__(256) void normfrag_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                       int64_t m_total, int cols, int64_t n_quads_row, int tiles,
                                                       float eps, uint2 *__restrict__ xf) {
  constexpr int kQuadFrags = kXfQuadBytes / 16;
  const int lane = threadIdx.x & 63;
  const int64_t tok = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t slab = tok >> 6;
  const int t = static_cast<int>((tok >> 4) & 3), tl = static_cast<int>(tok & 15);
  if (t >= tiles) return;  // a token tile the GEMM does not read (the whole wave: one row)
  const int n4 = cols >> 2;
  const bool live = tok < m_total;
  const float4 *xr = reinterpret_cast<const float4 *>(x + (live ? tok : 0) * static_cast<int64_t>(cols));
  const float4 *wr = reinterpret_cast<const float4 *>(w);
  float4 v[kNfVec], g[kNfVec];
#pragma unroll
  for (int k = 0; k < kNfVec; ++k) {
    const int i = lane + 64 * k;
    v[k] = live && i < n4 ? xr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    g[k] = i < n4 ? wr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNfVec; ++k) {
    ss = fmaf(v[k].x, v[k].x, ss);
    ss = fmaf(v[k].y, v[k].y, ss);
    ss = fmaf(v[k].z, v[k].z, ss);
    ss = fmaf(v[k].w, v[k].w, ss);
  }
  ss = wave_reduce_sum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
  const int64_t n_frag = n_quads_row * 12;
  const int64_t per_slab = n_quads_row * kQuadFrags;
  uint2 *dst = xf + 2 * slab * per_slab * 3 + (lane & 1);
#pragma unroll
  for (int k = 0; k < kNfVec; ++k) {
    const int fg = 32 * k + (lane >> 1);
    if (fg >= n_frag) continue;
    const int qs = fg >> 2, c8 = fg & 3, quad = qs / 3;
    const int64_t within = static_cast<int64_t>(qs * 4 + t) * 64 + tl + 16 * c8 - static_cast<int64_t>(quad) * kQuadFrags;
    const float y[4] = {v[k].x * r * g[k].x, v[k].y * r * g[k].y, v[k].z * r * g[k].z, v[k].w * r * g[k].w};
    uint32_t hb[4], mb[4], lb[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float xv = live ? y[e] : 0.f;
      hb[e] = bf16_rne_bits(xv);
      mb[e] = lb[e] = 0u;
      if (fabsf(xv) <= 3.0e38f) {
        const float r1 = xv - __uint_as_float(hb[e] << 16);
        mb[e] = bf16_rne_bits(r1);
        lb[e] = bf16_rne_bits(r1 - __uint_as_float(mb[e] << 16));
      }
    }
    uint2 *d = dst + 2 * (static_cast<int64_t>(quad) * 3 * kQuadFrags + within);
    d[0] = make_uint2(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16));
    d[2 * kQuadFrags] = make_uint2(mb[0] | (mb[1] << 16), mb[2] | (mb[3] << 16));
    d[4 * kQuadFrags] = make_uint2(lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16));
  }
}

// (hi | lo << 16) with hi + lo == v exactly for an fp16 value v (lo = 0 for inf / nan)
__device__ __forceinline__ uint32_t hi_lo_pack(float v) {
  const uint32_t hb = bf16_rne_bits(v);
  if (!(fabsf(v) <= 3.0e38f)) return hb;
  return hb | (bf16_rne_bits(v - __uint_as_float(hb << 16)) << 16);
}

// token tiles of 16; waves per block; quads of x in flight per wave; exact fp16 weights (hi + lo);
// bf16 parts per activation (1: bf16 x; 3: fp32 x, see xfrag_kernel)
// PLN: `packed` is the plane layout (3 uint16 records per atom); the value-id
// words come from the plane table, staged in LDS, instead of kp_dq gathers.
template <int MT, int WV, int PD, bool EXACT, int XP, bool XD, bool PLN>
__global__ __launch_bounds__(64 * WV, WV <= 4 ? 2 : 1) void dqmm_kernel(
    const uint8_t *__restrict__ packed, int64_t packed_bytes, const uint16_t *__restrict__ sigma16, int64_t rows,
    int64_t atoms_per_row, const uint4 *__restrict__ xf, int64_t n_quads_row, int64_t m_total, int splits, int apb,
    const uint32_t *__restrict__ kp_dq, const uint32_t *__restrict__ pl_ids, int pl_vecs, float *__restrict__ y,
    float *__restrict__ partial, const float *__restrict__ residual, int gelu) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int NT = 64 * WV;
  constexpr int TOK = 16 * MT;
  const int ws = mm_row_words(apb);
  constexpr int TPT = 3;  // PLN: plane-table vectors per thread (the host checks pl_vecs <= TPT * NT)
  const int region = max(kMmRows * ws + (PLN ? TPT * NT * 4 : 0), WV * TOK * kMmRedStride) * 4;
  uint32_t *wt = reinterpret_cast<uint32_t *>(smem);          // [32][ws] kp_dq words
  float *red = reinterpret_cast<float *>(smem);               // after the k loop: [WV][TOK][kMmRedStride]
  uint4 *rtab = reinterpret_cast<uint4 *>(smem + region);     // [EXACT ? 2 : 1][32] row byte tables
  // PLN: the plane table, after the kp_dq words (read in the prologue only; the cross-wave sum may reuse it)
  uint32_t *ptab = wt + kMmRows * ws;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, q = lane >> 4;
  const int64_t row_block = blockIdx.x / static_cast<unsigned>(splits);
  const int split = static_cast<int>(blockIdx.x % static_cast<unsigned>(splits));
  const int64_t row0 = row_block * kMmRows;
  const int64_t tok0 = static_cast<int64_t>(blockIdx.y) * 64;
  const int64_t a_begin = static_cast<int64_t>(split) * apb;
  const int n_atoms = static_cast<int>(min(static_cast<int64_t>(apb), atoms_per_row - a_begin));  // >= 1
  const int n_quads = (n_atoms + 3) >> 2;
  // this wave's quads: a contiguous share of the block's
  const int qbase = n_quads / WV, qextra = n_quads % WV;
  const int wq0 = wave * qbase + min(wave, qextra);
  const int wqn = qbase + (wave < qextra ? 1 : 0);

  // ---- activation fragments ----
  // Quad Q of the row, K step s, token tile t: lane (j, q) holds token 16t + j,
  // columns 96Q + 32s + 8q .. +8.  XD (bf16 x, up to 32 tokens): read
  // straight from x, 16 token rows x 64 B per wave load (half lines).
  // Otherwise from the fragment-order copy xfrag_kernel writes (1 KB
  // contiguous per wave load).  Measured per 7680x1920 call: at 17 tokens in
  // place 8.6 us against 10.4 with the copy kernel; at 64 tokens 13.9 against
  // 12.1 (16 half lines per load twice as many tokens outweigh the launch).
  // Raw buffer loads: a quad past this wave's share, a column past the row and
  // (XD) a token past m take an out-of-range offset, which returns zeros
  // without touching memory, so the loads need no branches (the compiler can
  // then wait for one quad's loads while the next quads' stay in flight).
  const int64_t cols = atoms_per_row * kDim;
  const int slab_bytes =
      XD ? static_cast<int>(min(static_cast<int64_t>(64), m_total - tok0) * cols * 2)
         : static_cast<int>(n_quads_row * XP * kXfQuadBytes);
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      XD ? const_cast<uint8_t *>(reinterpret_cast<const uint8_t *>(xf) + tok0 * cols * 2)
         : reinterpret_cast<uint8_t *>(const_cast<uint4 *>(xf + static_cast<int64_t>(blockIdx.y) * (slab_bytes / 16))),
      static_cast<short>(0), slab_bytes, kBufferFlags);
  const int xbase = XD ? static_cast<int>(j * cols * 2 + 16 * q)
                       : static_cast<int>(a_begin / 4 + wq0) * XP * kXfQuadBytes + 16 * lane;
  const int xcol0 = static_cast<int>(96 * (a_begin / 4 + wq0)) + 8 * q;  // XD: this lane's first column
  auto load_quad = [&](uint4 (&xa)[3][XP][MT], int qd) {
#pragma unroll
    for (int s = 0; s < 3; ++s) {
#pragma unroll
      for (int pp = 0; pp < XP; ++pp) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          int off;
          if constexpr (XD) {
            const int col = xcol0 + 96 * qd + 32 * s;
            off = qd < wqn && col < cols ? xbase + t * static_cast<int>(16 * cols * 2) + 2 * (col - 8 * q)
                                         : kBufferOutOfRange;
          } else {
            off = qd < wqn ? xbase + (qd * XP + pp) * kXfQuadBytes + (4 * s + t) * 1024 : kBufferOutOfRange;
          }
          asm("" : "+v"(off));  // one unconditional load (not one per select outcome under branches)
          xa[s][pp][t] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
        }
      }
    }
  };
  uint4 xa[PD][3][XP][MT];
#pragma unroll
  for (int u = 0; u < PD; ++u) load_quad(xa[u], u);  // in flight during the prologue

  // ---- per-row byte tables (threads 0..31, one row each): low / high bytes of hi (and lo) ----
  auto build_row_tables = [&]() {
    if (tid >= kMmRows) return;
    const int64_t row = row0 + tid;
    const float sl = __uint_as_float(kSLatticeBits);
    const float sig = row < rows ? __half2float(__ushort_as_half(sigma16[row])) : 0.f;
    const uint32_t v0 = dq_value(0, sig, sl), v1 = dq_value(1, sig, sl), v2 = dq_value(2, sig, sl);
    const uint32_t v3 = dq_value(3, sig, sl), v4 = dq_value(4, sig, sl);
    const uint32_t h[8] = {v0, v1, v2, v4, v4 ^ 0x8000u, v3 ^ 0x8000u, v2 ^ 0x8000u, v1 ^ 0x8000u};
    uint32_t hl[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) hl[e] = hi_lo_pack(__half2float(__ushort_as_half(static_cast<uint16_t>(h[e]))));
#pragma unroll
    for (int half = 0; half < (EXACT ? 2 : 1); ++half) {
      uint32_t lb0 = 0, lb1 = 0, hb0 = 0, hb1 = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t b0 = hl[e] >> (16 * half), b1 = hl[e + 4] >> (16 * half);
        lb0 |= (b0 & 0xFFu) << (8 * e);
        lb1 |= (b1 & 0xFFu) << (8 * e);
        hb0 |= ((b0 >> 8) & 0xFFu) << (8 * e);
        hb1 |= ((b1 >> 8) & 0xFFu) << (8 * e);
      }
      rtab[half * kMmRows + tid] = make_uint4(lb0, lb1, hb0, hb1);
    }
  };

  // ---- codes -> kp_dq words in LDS ----
  // Rows holding a multiple of 4 atoms: a thread decodes whole 9-byte groups
  // (4 codes from 3 dwords); the row tables are built while those loads are
  // in flight, then all table loads are issued before any LDS store.
  if constexpr (PLN) {
    // the block's (row, atom) records (atoms up to the end of the last quad), requested before the
    // plane table is staged; then one barrier and the table lookups
    constexpr int NA = (kMmRows * kMmMaxApb + NT - 1) / NT;  // (row, atom) pairs per thread at most
    const int na = 4 * n_quads;
    uint32_t rec[NA][3];
#pragma unroll
    for (int u = 0; u < NA; ++u) {
      const int c = u * NT + tid;
      const int r = c / na, a = c - r * na;
      const int64_t row = row0 + r, atom = a_begin + a;
      const bool live = c < kMmRows * na && row < rows && atom < atoms_per_row;
      const uint16_t *rp = reinterpret_cast<const uint16_t *>(packed) + 3 * (live ? row * atoms_per_row + atom : 0);
      const uint32_t lm = live ? 0xFFFFu : 0u;  // records past the weight read as plane 0 (the origin's)
      rec[u][0] = rp[0] & lm;
      rec[u][1] = rp[1] & lm;
      rec[u][2] = rp[2] & lm;
    }
    // the plane table: TPT vectors per thread, stored unconditionally
    uint4 tq[TPT];
#pragma unroll
    for (int v = 0; v < TPT; ++v) {
      const int vi = tid + v * NT;
      tq[v] = reinterpret_cast<const uint4 *>(pl_ids)[vi < pl_vecs ? vi : 0];
    }
#pragma unroll
    for (int v = 0; v < TPT; ++v) reinterpret_cast<uint4 *>(ptab)[tid + v * NT] = tq[v];
    build_row_tables();
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NA; ++u) {
      const int c = u * NT + tid;
      if (c < kMmRows * na) {
        const int r = c / na, a = c - r * na;
        uint32_t *d = wt + r * ws + 3 * a;
        // the origin's plane (all ids 0) for rows and atoms past the weight: index 0 of the table
        // (clamped to the staged table: a layout not made by plane_layout_kernel cannot index past it)
        d[0] = ptab[min(rec[u][0] & 0x1FFFu, static_cast<uint32_t>(TPT * NT * 4 - 1))];
        d[1] = ptab[min(rec[u][1] & 0x1FFFu, static_cast<uint32_t>(TPT * NT * 4 - 1))];
        d[2] = ptab[min(rec[u][2] & 0x1FFFu, static_cast<uint32_t>(TPT * NT * 4 - 1))];
      }
    }
  } else if ((atoms_per_row & 3) == 0) {
    constexpr int NG = (kMmRows * kMmMaxApb / 4 + NT - 1) / NT;  // groups per thread at most
    const int gpr = n_quads;                                     // groups per row in this block
    uint32_t dw[NG][3], off[NG];
    bool live[NG];
#pragma unroll
    for (int u = 0; u < NG; ++u) {
      const int g = u * NT + tid;
      const int r = g / gpr, k = g - r * gpr;
      const int64_t row = row0 + r;
      live[u] = g < kMmRows * gpr && row < rows;
      dw[u][0] = dw[u][1] = dw[u][2] = 0u;
      off[u] = 0;
      if (live[u]) {
        const int64_t b = (row * atoms_per_row + a_begin + 4 * k) / 4 * 9;
        const int64_t b4 = b & ~static_cast<int64_t>(3);
        off[u] = static_cast<uint32_t>(b & 3);
        const uint32_t *pw = reinterpret_cast<const uint32_t *>(packed + b4);
        if (b4 + 12 <= packed_bytes) {
          dw[u][0] = pw[0];
          dw[u][1] = pw[1];
          dw[u][2] = pw[2];
        } else {  // the stream's last group: byte loads inside the stream
          uint32_t t[3] = {0u, 0u, 0u};
          for (int e = 0; e < 12 && b4 + e < packed_bytes; ++e) t[e / 4] |= static_cast<uint32_t>(packed[b4 + e]) << (8 * (e % 4));
          dw[u][0] = t[0];
          dw[u][1] = t[1];
          dw[u][2] = t[2];
        }
      }
    }
    build_row_tables();
    uint3 e[NG][4];
#pragma unroll
    for (int u = 0; u < NG; ++u) {
      int32_t c[4] = {0, 0, 0, 0};
      if (live[u]) group_codes(dw[u][0], dw[u][1], dw[u][2], off[u], c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int32_t code = c[i] > kKissing ? 0 : c[i];
        e[u][i] = *reinterpret_cast<const uint3 *>(kp_dq + static_cast<int64_t>(code) * 3);
      }
    }
#pragma unroll
    for (int u = 0; u < NG; ++u) {
      const int g = u * NT + tid;
      if (g < kMmRows * gpr) {
        const int r = g / gpr, k = g - r * gpr;
        uint32_t *d = wt + r * ws + 12 * k;   // 48 B at a 16-byte multiple (ws % 4 == 0)
        reinterpret_cast<uint4 *>(d)[0] = make_uint4(e[u][0].x, e[u][0].y, e[u][0].z, e[u][1].x);
        reinterpret_cast<uint4 *>(d)[1] = make_uint4(e[u][1].y, e[u][1].z, e[u][2].x, e[u][2].y);
        reinterpret_cast<uint4 *>(d)[2] = make_uint4(e[u][2].z, e[u][3].x, e[u][3].y, e[u][3].z);
      }
    }
  } else {
    // general rows: one code per (row, atom), atoms up to the end of the last quad
    build_row_tables();
    const int na = 4 * n_quads;
    for (int c = tid; c < kMmRows * na; c += NT) {
      const int r = c / na, a = c - r * na;
      const int64_t row = row0 + r, atom = a_begin + a;
      int32_t code = 0;
      if (row < rows && atom < atoms_per_row) {
        code = packed_index_dw(packed, packed_bytes, row * atoms_per_row + atom);
        if (code > kKissing) code = 0;
      }
      const uint3 e = *reinterpret_cast<const uint3 *>(kp_dq + static_cast<int64_t>(code) * 3);
      uint32_t *d = wt + r * ws + 3 * a;
      d[0] = e.x;
      d[1] = e.y;
      d[2] = e.z;
    }
  }
  __syncthreads();

  f32x4_t acc[MT][2];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) acc[t][rt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const uint4 ta0 = rtab[j], ta1 = rtab[16 + j];
  const uint4 tb0 = rtab[EXACT ? kMmRows + j : j], tb1 = rtab[EXACT ? kMmRows + 16 + j : 16 + j];
  // word of (row, block atom a, plane p) = 3a + p; K step s of quad Q, lane group q: 12Q + 4s + q
  const uint32_t *wrow0 = wt + j * ws + 12 * wq0 + q;
  const uint32_t *wrow1 = wt + (16 + j) * ws + 12 * wq0 + q;
  auto compute_quad = [&](const uint4 (&xa_q)[3][XP][MT], int qd) {
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      const uint32_t w0 = wrow0[12 * qd + 4 * s], w1 = wrow1[12 * qd + 4 * s];
      const bf16x8_t b0 = perm_decode(w0, ta0.x, ta0.y, ta0.z, ta0.w);
      const bf16x8_t b1 = perm_decode(w1, ta1.x, ta1.y, ta1.z, ta1.w);
#pragma unroll
      for (int pp = 0; pp < XP; ++pp)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const bf16x8_t av = __builtin_bit_cast(bf16x8_t, xa_q[s][pp][t]);
          acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b0, acc[t][0], 0, 0, 0);
          acc[t][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b1, acc[t][1], 0, 0, 0);
        }
      if constexpr (EXACT) {
        const bf16x8_t l0 = perm_decode(w0, tb0.x, tb0.y, tb0.z, tb0.w);
        const bf16x8_t l1 = perm_decode(w1, tb1.x, tb1.y, tb1.z, tb1.w);
        // every activation part times the weights' low part: the products stay exact
#pragma unroll
        for (int pp = 0; pp < XP; ++pp)
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            const bf16x8_t av = __builtin_bit_cast(bf16x8_t, xa_q[s][pp][t]);
            acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, l0, acc[t][0], 0, 0, 0);
            acc[t][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, l1, acc[t][1], 0, 0, 0);
          }
      }
    }
    // keep the fragments in their registers until the slot is refilled, so no
    // MFMA result is allocated there (that made the loop wait for every load)
#pragma unroll
    for (int s = 0; s < 3; ++s)
#pragma unroll
      for (int pp = 0; pp < XP; ++pp)
#pragma unroll
        for (int t = 0; t < MT; ++t) asm volatile("" : : "v"(__builtin_bit_cast(u32x4_t, xa_q[s][pp][t])));
  };
  // Whole rounds of PD quads without branches, then the last < PD quads.  The
  // first round is peeled: the loop header then sees the same loads in flight
  // (PD slots, oldest first) from both of its predecessors, so the compiler
  // waits for one slot at a time instead of for every load.
  auto round = [&](int q0) {
#pragma unroll
    for (int u = 0; u < PD; ++u) {
      compute_quad(xa[u], q0 + u);
      __builtin_amdgcn_sched_barrier(0);  // slot u is refilled right after its MFMAs, not at the round's end
      load_quad(xa[u], q0 + u + PD);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  int qd = 0;
  if (PD <= wqn) {
    round(0);
    for (qd = PD; qd + PD <= wqn; qd += PD) round(qd);
  }
#pragma unroll
  for (int u = 0; u < PD - 1; ++u)
    if (qd + u < wqn) compute_quad(xa[u], qd + u);

  // ---- epilogue: the waves' tiles summed in wave order; C[token 16t + 4q + e][row 16rt + j] ----
  __syncthreads();  // every wave is done with the kp_dq tile
  float *rw = red + wave * (TOK * kMmRedStride);
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int e = 0; e < 4; ++e) rw[(16 * t + 4 * q + e) * kMmRedStride + 16 * rt + j] = acc[t][rt][e];
  __syncthreads();
  float *dst = splits == 1 ? y : partial + (static_cast<int64_t>(blockIdx.y) * splits + split) * 64 * rows;
  const int64_t tok_base = splits == 1 ? tok0 : 0;  // partial tiles are indexed per slab
  const bool vec = (rows & 3) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0;
  for (int i = tid; i < TOK * (kMmRows / 4); i += NT) {
    const int tl = i / (kMmRows / 4), g = i - tl * (kMmRows / 4);
    f32x4_t sum = *reinterpret_cast<const f32x4_t *>(red + tl * kMmRedStride + 4 * g);
#pragma unroll
    for (int w = 1; w < WV; ++w) sum += *reinterpret_cast<const f32x4_t *>(red + (w * TOK + tl) * kMmRedStride + 4 * g);
    const int64_t row = row0 + 4 * g;
    if (tok0 + tl >= m_total || row >= rows) continue;
    float *d = dst + (tok_base + tl) * rows + row;
    if (splits == 1) {  // the final output: epilogue here (with a K split, in dqmm_reduce_kernel)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (row + c < rows) sum[c] = dql_epilogue(sum[c], residual, (tok0 + tl) * rows + row + c, gelu);
    }
    if (vec) {
      *reinterpret_cast<f32x4_t *>(d) = sum;
    } else {
      for (int c = 0; c < 4 && row + c < rows; ++c) d[c] = sum[c];
    }
  }
}

// y[tok, r] = sum over splits (ascending) of the partial tiles; 4 outputs per
// thread (rows % 4 == 0) or 1, loads of 4 splits issued together.
template <bool VEC>
__global__ __launch_bounds__(256) void dqmm_reduce_kernel(const float *__restrict__ partial, int splits, int64_t rows,
                                                          int64_t m_total, float *__restrict__ y,
                                                          const float *__restrict__ residual, int gelu) {
  constexpr int W = VEC ? 4 : 1;
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * W;
  if (i >= m_total * rows) return;
  const int64_t tok = i / rows, row = i - tok * rows;
  const int64_t slab = tok / 64, tl = tok - slab * 64;
  const int64_t stride = 64 * rows;
  const float *p = partial + (slab * splits) * stride + tl * rows + row;
  typedef float f4 __attribute__((ext_vector_type(4)));
  typedef float fw __attribute__((ext_vector_type(W)));
  fw s = {};
  int k = 0;
  for (; k + 4 <= splits; k += 4) {
    fw v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const fw *>(p + static_cast<int64_t>(k + u) * stride);
#pragma unroll
    for (int u = 0; u < 4; ++u) s += v[u];
  }
  for (; k < splits; ++k) s += *reinterpret_cast<const fw *>(p + static_cast<int64_t>(k) * stride);
#pragma unroll
  for (int c = 0; c < W; ++c) s[c] = dql_epilogue(s[c], residual, i + c, gelu);
  *reinterpret_cast<fw *>(y + i) = s;
  (void)sizeof(f4);
}

struct MmPlan {
  int apb = 4, splits = 1;
};

// Atoms per block (a multiple of 4, at most kMmMaxApb) and K splits: the fewest
// splits that keep the block's atoms within kMmMaxApb and give the grid about
// kMmTargetBlocks blocks.
MmPlan mm_plan(int64_t rows, int64_t apr) {
  MmPlan p;
  const int64_t row_blocks = (rows + kMmRows - 1) / kMmRows;
  const int64_t fill = row_blocks >= kMmNoSplitBlocks ? 1 : (kMmTargetBlocks + row_blocks - 1) / row_blocks;
  int64_t s = max((apr + kMmMaxApb - 1) / kMmMaxApb, fill);
  s = max(static_cast<int64_t>(1), min(s, (apr + 3) / 4));
  const int64_t apb = (((apr + s - 1) / s) + 3) & ~static_cast<int64_t>(3);
  p.apb = static_cast<int>(apb);
  p.splits = static_cast<int>((apr + apb - 1) / apb);
  return p;
}

template <int MT, int WV, int PD, bool EXACT, int XP, bool XD>
int launch_dqmm_t(const uint8_t *packed, int64_t pb, const uint16_t *sigma16, int64_t rows, int64_t apr,
                  const uint4 *xf, int64_t m, float *y, float *partial, const MmPlan &pl, const uint32_t *kp_dq,
                  const uint32_t *pl_ids, int pl_vecs, const float *residual, int gelu, hipStream_t s) {
  const int64_t row_blocks = (rows + kMmRows - 1) / kMmRows;
  const int64_t slabs = (m + 63) / 64;
  const int64_t nq = (apr + 3) / 4;
  // PLN: 3 plane-table vectors per thread after the kp_dq words (the region the cross-wave sum reuses)
  const size_t region = static_cast<size_t>(max(kMmRows * mm_row_words(pl.apb) + (pl_ids ? 3 * 64 * WV * 4 : 0),
                                                WV * 16 * MT * kMmRedStride)) * 4;
  const size_t shm = region + static_cast<size_t>(kMmRows) * 16 * (EXACT ? 2 : 1);
  if (pl_ids && (pl_vecs > 3 * 64 * WV || shm > 80 * 1024))  // two blocks per CU
    return fail(PLX_EINVAL, "dequant_linear: the plane table does not fit this GEMM block");
  const dim3 g(static_cast<unsigned>(row_blocks * pl.splits), static_cast<unsigned>(slabs));
  if (pl_ids)
    hipLaunchKernelGGL((dqmm_kernel<MT, WV, PD, EXACT, XP, XD, true>), g, dim3(64 * WV), shm, s, packed, pb, sigma16,
                       rows, apr, xf, nq, m, pl.splits, pl.apb, kp_dq, pl_ids, pl_vecs, y, partial, residual, gelu);
  else
    hipLaunchKernelGGL((dqmm_kernel<MT, WV, PD, EXACT, XP, XD, false>), g, dim3(64 * WV), shm, s, packed, pb, sigma16,
                       rows, apr, xf, nq, m, pl.splits, pl.apb, kp_dq, pl_ids, pl_vecs, y, partial, residual, gelu);
  return check_launch("dqmm_kernel");
}

template <int MT>
int launch_dqmm(const uint8_t *packed, int64_t pb, const uint16_t *sigma16, int64_t rows, int64_t apr,
                const uint4 *xf, int64_t m, float *y, float *partial, const MmPlan &pl, const uint32_t *kp_dq,
                const uint32_t *pl_ids, int pl_vecs, bool exact, bool x_f32, bool direct, const float *residual,
                int gelu, hipStream_t s) {
  // 8 waves (two per SIMD cover each other's load latency), one quad of x in
  // flight per wave; 4 waves with 2 quads in flight measured within 3%.
  // `direct`: bf16 x read in place (xf = x), else the fragment-order copy.
  if (x_f32)
    return launch_dqmm_t<MT, 8, 1, true, 3, false>(packed, pb, sigma16, rows, apr, xf, m, y, partial, pl, kp_dq, pl_ids, pl_vecs,
                                                   residual, gelu, s);
  if constexpr (MT <= 2)  // direct is only chosen up to 32 tokens
    if (direct)
      return exact ? launch_dqmm_t<MT, 8, 1, true, 1, true>(packed, pb, sigma16, rows, apr, xf, m, y, partial, pl, kp_dq, pl_ids, pl_vecs,
                                                            residual, gelu, s)
                   : launch_dqmm_t<MT, 8, 1, false, 1, true>(packed, pb, sigma16, rows, apr, xf, m, y, partial, pl,
                                                             kp_dq, pl_ids, pl_vecs, residual, gelu, s);
  return exact ? launch_dqmm_t<MT, 8, 1, true, 1, false>(packed, pb, sigma16, rows, apr, xf, m, y, partial, pl, kp_dq, pl_ids, pl_vecs,
                                                         residual, gelu, s)
               : launch_dqmm_t<MT, 8, 1, false, 1, false>(packed, pb, sigma16, rows, apr, xf, m, y, partial, pl,
                                                          kp_dq, pl_ids, pl_vecs, residual, gelu, s);
}

// Workspace of the batched path: the fragment-order x copy (a multiple of 256
// bytes), then, with a K split, the split partial tiles [slab][split][64][rows] fp32.
struct MmWorkspace {
  size_t xf = 0, partial = 0;
  size_t total() const { return xf + partial; }
};

// bf16 x of up to 32 tokens is read in place by dqmm_kernel; larger batches
// and fp32 x go through the fragment-order copy.
bool mm_x_copy(bool x_f32, int64_t m) { return x_f32 || m > 32; }

MmWorkspace mm_workspace(int64_t rows, int64_t cols, int64_t m, const MmPlan &pl, bool x_f32) {
  MmWorkspace w;
  const size_t slabs = static_cast<size_t>((m + 63) / 64);
  if (mm_x_copy(x_f32, m)) w.xf = slabs * static_cast<size_t>((cols / kDim + 3) / 4) * kXfQuadBytes * (x_f32 ? 3 : 1);
  if (pl.splits > 1) w.partial = slabs * pl.splits * 64 * static_cast<size_t>(rows) * sizeof(float);
  return w;
}

// GEMV up to 4 tokens of fp32 x and 2 of bf16 x, MFMA GEMM above: the GEMV
// streams the packed rows and repeats its codebook gathers once per 4 tokens,
// the GEMM's cost barely changes with the batch (measured per call, fp32 x:
// 7680x1920 GEMV 9.6 us at 4 tokens, 13.9 at 6; GEMM 11.1 at 5 with one token
// tile; bf16 x, 7680x1920 / 1920x7680: GEMV 6.3 / 8.3 at 2 tokens, 10.1 / 13.2
// at 3, 9.0 / 11.5 at 4; GEMM 6.9 / 8.9 at each of 2-4)
bool uses_mfma(int flags, int64_t m) { return m > ((flags & PLX_DQL_X_F32) ? 4 : 2); }

}  // namespace

// MFMA part (fragment-order x + split partials) of the workspace
size_t mm_workspace_bytes_multi(const int64_t *rows, int n, int64_t cols, int64_t m, int flags) {
  if (!uses_mfma(flags, m)) return 0;
  // one fragment-order copy of x for every target, one partial buffer reused by them in stream order
  size_t xf = 0, partial = 0;
  for (int i = 0; i < n; ++i) {
    if (rows[i] <= 0) continue;
    const MmWorkspace w = mm_workspace(rows[i], cols, m, mm_plan(rows[i], cols / kDim), (flags & PLX_DQL_X_F32) != 0);
    xf = w.xf;
    partial = partial > w.partial ? partial : w.partial;
  }
  return xf + partial;
}

// Layout: [MFMA part | normalised x (PLX_DQL_RMS_NORM), 256-byte aligned]
size_t dequant_linear_workspace_bytes_multi(const int64_t *rows, int n, int64_t cols, int64_t m, int flags) {
  if (cols <= 0 || n <= 0 || m <= 0) return 0;
  size_t total = mm_workspace_bytes_multi(rows, n, cols, m, flags);
  if (flags & PLX_DQL_RMS_NORM) total = ((total + 255) & ~static_cast<size_t>(255)) + static_cast<size_t>(m * cols) * 4;
  return total;
}

size_t dequant_linear_workspace_bytes(int64_t rows, int64_t cols, int64_t m, int flags) {
  return dequant_linear_workspace_bytes_multi(&rows, 1, cols, m, flags);
}

int launch_dequant_linear_multi(const DqlTarget *targets, int n, int64_t cols, const void *x, int flags, int64_t m,
                                const float *norm_w, float norm_eps, void *workspace, size_t workspace_bytes,
                                hipStream_t s) {
  if (n < 1 || n > 16) return fail(PLX_EINVAL, "dequant_linear: %d targets (1..16)", n);
  if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0) return fail(PLX_EINVAL, "dequant_linear: x must be 16-byte aligned");
  for (int i = 0; i < n; ++i)
    if ((reinterpret_cast<uintptr_t>(targets[i].packed) & 15u) != 0)
      return fail(PLX_EINVAL, "dequant_linear: packed weights must be 16-byte aligned");
  const int x_is_f32 = flags & PLX_DQL_X_F32;
  const int round_w = !x_is_f32 && (flags & PLX_DQL_W_AS_X) ? 1 : 0;  // W.to(fp32) is exact
  const int gelu = (flags & PLX_DQL_GELU) ? 1 : 0;
  const bool norm = (flags & PLX_DQL_RMS_NORM) != 0;
  if (norm != (norm_w != nullptr))
    return fail(PLX_EINVAL, "dequant_linear: PLX_DQL_RMS_NORM and a norm weight go together");
  if (norm && (!x_is_f32 || (reinterpret_cast<uintptr_t>(norm_w) & 15u) != 0))
    return fail(PLX_EINVAL, "dequant_linear: the RMS norm takes fp32 x and a 16-byte aligned weight");
  int64_t rows_list[16];
  for (int i = 0; i < n; ++i) rows_list[i] = targets[i].rows;
  const size_t need = dequant_linear_workspace_bytes_multi(rows_list, n, cols, m, flags);
  if (workspace_bytes < need || (need && workspace == nullptr))
    return fail(PLX_EINVAL, "dequant_linear: workspace of %zu bytes is smaller than the %zu needed", workspace_bytes, need);
  if (need && (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0)
    return fail(PLX_EINVAL, "dequant_linear: workspace must be 16-byte aligned");
  const DeviceTables *tab = nullptr;
  int st = get_tables(&tab);
  if (st != PLX_OK) return st;
  const int64_t apr = cols / kDim;
  const bool planes = (flags & PLX_DQL_PLANES) != 0;  // `packed` holds plane-layout records
  const int pl_vecs = static_cast<int>((plane_tables_host()->ids.size() + 3) / 4);
  float *xnorm = norm ? reinterpret_cast<float *>(static_cast<uint8_t *>(workspace) +
                                                  ((mm_workspace_bytes_multi(rows_list, n, cols, m, flags) + 255) &
                                                   ~static_cast<size_t>(255)))
                      : nullptr;
  if (uses_mfma(flags, m)) {
    // batches above 4 tokens: MFMA dequant-GEMM in slabs of 64 tokens, one launch (+ split sum) per target
    if (cols > kMmMaxCols)
      return fail(PLX_EINVAL, "dequant_linear: %lld columns exceed the batched path's %lld", static_cast<long long>(cols),
                  static_cast<long long>(kMmMaxCols));
    uint8_t *wsb = static_cast<uint8_t *>(workspace);
    const uint4 *xf = reinterpret_cast<const uint4 *>(wsb);
    const int64_t slabs = (m + 63) / 64, nq = (apr + 3) / 4;
    const dim3 gx(static_cast<unsigned>(nq * 3), static_cast<unsigned>(slabs));
    const bool copy = mm_x_copy(x_is_f32 != 0, m);
    // token tiles per slab the GEMM reads (its MT below): the copies write only these
    const int tiles = m > 32 ? 4 : m > 16 ? 2 : 1;
    if (norm && copy && nq * 12 <= 32 * kNfVec) {
      // the norm writes the fragment-order copy itself (rows that fit normfrag_kernel's registers)
      hipLaunchKernelGGL(normfrag_kernel, dim3(static_cast<unsigned>(slabs * 16)), dim3(256), 0, s,
                         static_cast<const float *>(x), norm_w, m, static_cast<int>(cols), nq, tiles, norm_eps,
                         reinterpret_cast<uint2 *>(wsb));
      st = check_launch("normfrag_kernel");
    } else {
      if (norm) {
        st = launch_rms_norm(static_cast<const float *>(x), norm_w, xnorm, m, cols, norm_eps, s);
        if (st != PLX_OK) return st;
        x = xnorm;
      }
      if (copy) {
        if (x_is_f32)
          hipLaunchKernelGGL((xfrag_kernel<true>), gx, dim3(256), 0, s, x, m, cols, nq, tiles,
                             reinterpret_cast<uint4 *>(wsb));
        else
          hipLaunchKernelGGL((xfrag_kernel<false>), gx, dim3(256), 0, s, x, m, cols, nq, tiles,
                             reinterpret_cast<uint4 *>(wsb));
        st = check_launch("xfrag_kernel");
      } else {
        xf = static_cast<const uint4 *>(x);  // read in place by dqmm_kernel
      }
    }
    for (int i = 0; i < n && st == PLX_OK; ++i) {
      const DqlTarget &t = targets[i];
      if (t.rows <= 0) continue;
      const MmPlan pl = mm_plan(t.rows, apr);
      float *part = reinterpret_cast<float *>(wsb + mm_workspace(t.rows, cols, m, pl, x_is_f32 != 0).xf);
      const int64_t pb = ((t.rows * apr + 3) / 4) * 9;  // packed stream length
      st = m > 32 ? launch_dqmm<4>(t.packed, planes ? 6 * t.rows * apr : pb, t.sigma16, t.rows, apr, xf, m, t.y,
                                   part, pl, tab->kp_dq, planes ? tab->pl_ids : nullptr, pl_vecs, !round_w, x_is_f32,
                                   !copy, t.residual, gelu, s)
                  : m > 16 ? launch_dqmm<2>(t.packed, planes ? 6 * t.rows * apr : pb, t.sigma16, t.rows, apr, xf, m,
                                            t.y, part, pl, tab->kp_dq, planes ? tab->pl_ids : nullptr, pl_vecs,
                                            !round_w, x_is_f32, !copy, t.residual, gelu, s)
                           : launch_dqmm<1>(t.packed, planes ? 6 * t.rows * apr : pb, t.sigma16, t.rows, apr, xf, m,
                                            t.y, part, pl, tab->kp_dq, planes ? tab->pl_ids : nullptr, pl_vecs,
                                            !round_w, x_is_f32, !copy, t.residual, gelu, s);
      if (st != PLX_OK || pl.splits == 1) continue;
      const int64_t cnt = m * t.rows;
      if (t.rows % 4 == 0 && (reinterpret_cast<uintptr_t>(t.y) & 15u) == 0)
        hipLaunchKernelGGL((dqmm_reduce_kernel<true>), dim3(static_cast<unsigned>((cnt / 4 + 255) / 256)), dim3(256), 0,
                           s, part, pl.splits, t.rows, m, t.y, t.residual, gelu);
      else
        hipLaunchKernelGGL((dqmm_reduce_kernel<false>), dim3(static_cast<unsigned>((cnt + 255) / 256)), dim3(256), 0, s,
                           part, pl.splits, t.rows, m, t.y, t.residual, gelu);
      st = check_launch("dqmm_reduce_kernel");
    }
    return st;
  }
  if (planes) {
    // the plane layout below the MFMA path: one token only
    if (m != 1) return fail(PLX_EINVAL, "dequant_linear: the plane layout takes one token or more than 4 (got %lld)",
                            static_cast<long long>(m));
    if (n == 1 && !x_is_f32 && !norm && !gelu && !targets[0].residual) {  // the plain bf16 call
      if (targets[0].rows <= 0) return PLX_OK;
      return launch_gemv1_planes(targets[0].packed, targets[0].sigma16, targets[0].rows, apr, x, tab, round_w,
                                 targets[0].y, s);
    }
    if (apr > 320)
      return fail(PLX_EINVAL, "dequant_linear: the plane layout takes rows of at most 320 atoms at one token (got %lld)",
                  static_cast<long long>(apr));
  }
  const uint4 *kp = reinterpret_cast<const uint4 *>(tab->kp_gemv);
  const DeviceTables *kd = tab;
  // up to kDqlMaxTargets targets per GEMV launch
  for (int i0 = 0; i0 < n && st == PLX_OK; i0 += kDqlMaxTargets) {
    DqlTargets t{};
    t.n = n - i0 < kDqlMaxTargets ? n - i0 : kDqlMaxTargets;
    for (int i = 0; i < kDqlMaxTargets; ++i) {
      const DqlTarget &src = targets[i0 + (i < t.n ? i : 0)];
      t.packed[i] = src.packed;
      t.packed_bytes[i] = planes ? 6 * src.rows * apr : ((src.rows * apr + 3) / 4) * 9;
      t.sigma16[i] = src.sigma16;
      t.rows[i] = i < t.n ? src.rows : 0;
      t.y[i] = src.y;
      t.residual[i] = src.residual;
    }
    t.norm_w = norm_w;
    t.norm_eps = norm_eps;
    // lanes per row: about 3-5 atoms per lane (7680 x 1920 at M = 1: 16 lanes as fast as 32, 8 slower; the
    // 1920-row q/k/v and o_proj launches of the decode step 3% faster with 32, from the doubled grid);
    // 512-thread blocks (4% faster than 256 at M = 1, 1,024 slower), 256 for rows too long to stage 8 in LDS
#define PLX_DQL_SEL(L_)                                                                                   \
  (planes ? (x_is_f32 ? launch_dql<L_, true, 512, true>(t, apr, x, m, kp, kd, round_w, gelu, xnorm, s, tab->pl_nib, \
                                                        pl_vecs)                                                    \
                      : launch_dql<L_, false, 512, true>(t, apr, x, m, kp, kd, round_w, gelu, xnorm, s,             \
                                                         tab->pl_nib, pl_vecs))                                     \
          : (x_is_f32 ? launch_dql<L_, true, 512>(t, apr, x, m, kp, kd, round_w, gelu, xnorm, s)                    \
                      : launch_dql<L_, false, 512>(t, apr, x, m, kp, kd, round_w, gelu, xnorm, s)))
    if (apr >= 3072)  // (the plane layout stops at 320 atoms per row)
      st = x_is_f32 ? launch_dql<64, true, 256>(t, apr, x, m, kp, kd, round_w, gelu, xnorm, s)
                    : launch_dql<64, false, 256>(t, apr, x, m, kp, kd, round_w, gelu, xnorm, s);
    else if (apr >= 160)
      st = PLX_DQL_SEL(64);
    else if (apr >= 16) {
      // 32 lanes per row (16 rows per block) when 16 would leave the grid under 192 blocks
      int64_t mrows = 0;
      for (int i = 0; i < t.n; ++i) mrows = t.rows[i] > mrows ? t.rows[i] : mrows;
      // (the plane layout: 16 lanes only while a block's records fit its stage)
      if ((mrows + 31) / 32 * t.n < 192 || (planes && 6 * 32 * apr + 31 > 16 * kDqlPlVecs * 512))
        st = PLX_DQL_SEL(32);
      else
        st = PLX_DQL_SEL(16);
    }
    else
      st = PLX_DQL_SEL(8);
#undef PLX_DQL_SEL
  }
  return st;
}

int launch_plane_layout(const uint8_t *packed, int64_t n_atoms, uint16_t *planes, hipStream_t s) {
  const DeviceTables *tab = nullptr;
  int st = get_tables(&tab);
  if (st != PLX_OK) return st;
  const int64_t blocks = (n_atoms + 255) / 256;
  if (blocks > 0x7FFFFFFFll) return fail(PLX_EINVAL, "plane_layout: %lld atoms exceed one launch", static_cast<long long>(n_atoms));
  hipLaunchKernelGGL(plane_layout_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, packed, n_atoms,
                     tab->code_planes, planes);
  return check_launch("plane_layout_kernel");
}

int launch_dequant_linear(const uint8_t *packed, const uint16_t *sigma16, int64_t rows, int64_t cols, const void *x,
                          int flags, int64_t m, float *y, void *workspace, size_t workspace_bytes, hipStream_t s) {
  const DqlTarget t{packed, sigma16, rows, y, nullptr};
  return launch_dequant_linear_multi(&t, 1, cols, x, flags, m, nullptr, 0.f, workspace, workspace_bytes, s);
}

}  // namespace plx

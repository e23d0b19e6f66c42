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
// Layout of the work: a block covers 1,024 atoms = 3,072 output chunks of 16 B
// (8 coordinates); thread t of the block writes chunks t, t+256, ... so each
// store instruction writes 1 KiB contiguous.  Per block the packed bytes are
// staged in LDS and decoded once per atom, and each row met by the block gets
// its 8-entry value table (low bytes, high bytes: 4 words) in LDS; a chunk is
// then one 4-byte kp_dq load (3-bit value ids, L2-resident) and 6 v_perm_b32
// byte lookups.  The output is written with non-temporal stores: as
// ordinary stores its 48 B/atom stream evicts kp_dq from L2 and the gathers
// then miss (measured: 41% of HBM peak instead of 70%).
//
// Indices above 196,560 (not produced by the reference packer) decode as the
// origin, so corrupt input can never read outside the table.

#include <hip/hip_fp16.h>

#include "plx_device.h"

namespace plx {
namespace {

constexpr int kThreads = 256;
constexpr int kDqAtoms = 1024;                     // atoms per block
constexpr int kDqChunks = kDqAtoms * 3;            // 16-byte output chunks per block
constexpr int kDqPackedBytes = kDqAtoms / 4 * 9;   // 2,304
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
#pragma unroll 2
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
  hipLaunchKernelGGL(dequant_kernel, g, dim3(kThreads), 0, s, packed, pb, sigma16, n_atoms, apr, tab->kp_dq, w16);
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
// end: the same products as the reference's fp32 F.linear on the fp16 W,
// regrouped (fp32 rounding differs at the 1e-7 relative level).
//
// Per code the kernel reads one 16-byte entry of kp_gemv (24 signed 4-bit
// coordinates + type/position byte; 3.1 MB, L2-resident per XCD).
// L lanes share a row and stride over its atoms; a block is 256 threads.
// ---------------------------------------------------------------------------

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

// One pass over the packed rows for MB tokens.  Block = 256 threads = R = 256/L
// rows; the block's packed bytes (and, when XL, the MB token rows of x as
// fp32) are staged in LDS first; each lane then handles atoms sub, sub+L, ...
// of its row in chunks of 4, issuing the chunk's four table gathers before
// scoring any of them.
template <int L, int MB, bool XF32, bool XL>
__global__ __launch_bounds__(256) void dqlinear_kernel(const uint8_t *__restrict__ packed, int64_t packed_bytes,
                                                       const uint16_t *__restrict__ sigma16, int64_t rows,
                                                       int64_t atoms_per_row, const void *__restrict__ x,
                                                       int64_t m_total, float *__restrict__ y,
                                                       const uint4 *__restrict__ kp_gemv) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int R = 256 / L;
  const int64_t cols = atoms_per_row * kDim;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * R;
  const int64_t rows_here = min(static_cast<int64_t>(R), rows - row0);
  // packed bytes of atoms [row0*apr, (row0+rows_here)*apr): whole 9-byte groups
  const int64_t atom0 = row0 * atoms_per_row;
  const int64_t g_lo = atom0 >> 2, g_hi = (atom0 + rows_here * atoms_per_row + 3) >> 2;
  // Copy the bytes [g_lo*9, g_hi*9) as aligned 16-byte vectors: byte b of the
  // stream lands at LDS offset b - base16, so vectors stay aligned on both
  // sides; a last vector that would cross the end of the stream goes bytewise.
  const int64_t start = g_lo * 9, end = g_hi * 9, base16 = start & ~static_cast<int64_t>(15);
  const int nvec = static_cast<int>((end - base16 + 15) >> 4);
  const uint8_t *pb = smem + (start - base16);
  float *xs = reinterpret_cast<float *>(smem + static_cast<int64_t>(nvec) * 16);
  for (int i = threadIdx.x; i < nvec; i += 256) {
    const int64_t gb = base16 + 16 * static_cast<int64_t>(i);
    if (gb + 16 <= packed_bytes) {
      reinterpret_cast<uint4 *>(smem)[i] = *reinterpret_cast<const uint4 *>(packed + gb);
    } else {
      for (int k = 0; k < 16 && gb + k < packed_bytes; ++k) smem[16 * i + k] = packed[gb + k];
    }
  }

  const int lane = threadIdx.x & 63;
  const int sub = lane % L;
  const int64_t row = row0 + threadIdx.x / L;
  const bool live = row < rows;
  for (int64_t m0 = 0; m0 < m_total; m0 += MB) {
    const int mb_here = static_cast<int>(min(static_cast<int64_t>(MB), m_total - m0));
    if (XL) {
      __syncthreads();
      // token rows are whole multiples of 8 elements (cols = 24 * apr): 8 per thread-step
      for (int64_t i = threadIdx.x; i < mb_here * cols / 8; i += 256) {
        float v[8];
        load_x8<XF32>(x, m0 * cols + 8 * i, v);
        float4 *d = reinterpret_cast<float4 *>(xs + 8 * i);
        d[0] = make_float4(v[0], v[1], v[2], v[3]);
        d[1] = make_float4(v[4], v[5], v[6], v[7]);
      }
    }
    __syncthreads();
    float acc[MB][4];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[mb][t] = 0.f;
    if (live) {
      for (int64_t a0 = sub; a0 < atoms_per_row; a0 += 4 * L) {
        uint4 e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t a = a0 + i * L;
          int32_t code = 0;
          if (a < atoms_per_row) {
            const int64_t n = row * atoms_per_row + a - g_lo * 4;  // atom index relative to the staged groups
            const uint8_t *bp = pb + (n >> 2) * 9 + 2 * (n & 3);
            const uint32_t v = (static_cast<uint32_t>(bp[0]) << 16) | (static_cast<uint32_t>(bp[1]) << 8) | bp[2];
            code = static_cast<int32_t>((v >> (6 - 2 * (n & 3))) & 0x3FFFFu);
            if (code > kKissing) code = 0;
          }
          e[i] = kp_gemv[code];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t a = a0 + i * L;
          if (a >= atoms_per_row) break;
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
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int off = L / 2; off > 0; off >>= 1) acc[mb][t] += __shfl_xor(acc[mb][t], off, 64);
    if (live && sub == 0) {
      const float sig = __half2float(__ushort_as_half(sigma16[row]));
      const float sl = __uint_as_float(kSLatticeBits);
      const float v1 = __half2float(__ushort_as_half(static_cast<uint16_t>(dq_value(1, sig, sl))));
      const float v2 = __half2float(__ushort_as_half(static_cast<uint16_t>(dq_value(2, sig, sl))));
      const float v3 = __half2float(__ushort_as_half(static_cast<uint16_t>(dq_value(3, sig, sl))));
      const float v4 = __half2float(__ushort_as_half(static_cast<uint16_t>(dq_value(4, sig, sl))));
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        if (mb < mb_here)
          y[(m0 + mb) * rows + row] =
              v4 * (acc[mb][0] * 0.25f) + v2 * (acc[mb][1] * 0.5f) + v1 * acc[mb][2] - v3 * acc[mb][3];
    }
  }
}

template <int L, bool XF32>
int launch_dql(const uint8_t *packed, int64_t packed_bytes, const uint16_t *sigma16, int64_t rows, int64_t apr,
               const void *x, int64_t m, float *y, const uint4 *tab, hipStream_t s) {
  constexpr int R = 256 / L;
  const dim3 g(static_cast<unsigned>((rows + R - 1) / R));
  const size_t pbytes = static_cast<size_t>((R * apr + 8) / 4 + 2) * 9;
  const size_t p16 = ((pbytes + 15) & ~static_cast<size_t>(15)) + 16;  // + one vector of alignment slack
  const int64_t cols = apr * kDim;
  const int mb = m >= 4 ? 4 : m >= 2 ? 2 : 1;
  const size_t xbytes = static_cast<size_t>(mb) * cols * 4;
  const bool xl = p16 + xbytes <= 48 * 1024;
  const size_t shm = xl ? p16 + xbytes : p16;
  if (shm > 64 * 1024) return fail(PLX_EINVAL, "dequant_linear: rows of %lld atoms are too long", static_cast<long long>(apr));
#define PLX_DQL(MB, XL) \
  hipLaunchKernelGGL((dqlinear_kernel<L, MB, XF32, XL>), g, dim3(256), shm, s, packed, packed_bytes, sigma16, rows, apr, \
                     x, m, y, tab)
  if (mb == 4) {
    if (xl) PLX_DQL(4, true); else PLX_DQL(4, false);
  } else if (mb == 2) {
    if (xl) PLX_DQL(2, true); else PLX_DQL(2, false);
  } else {
    if (xl) PLX_DQL(1, true); else PLX_DQL(1, false);
  }
#undef PLX_DQL
  return check_launch("dqlinear_kernel");
}

// ---------------------------------------------------------------------------
// dequant-GEMM for larger batches: y[m, r] = sum_i x[m, i] W[r, i] on MFMA.
//
// W[r, i] = +-v_|k| (fp16, 11 significant bits) is split exactly into two bf16
// values, W = hi + lo (hi = bf16_rne(W), lo = W - hi has <= 4 significant
// bits), so two v_mfma_f32_16x16x32_bf16 per tile give exact products of the
// bf16 activations with the fp16 weights, accumulated in fp32.
// Block = KW waves x 64 lanes, 16 output rows (MFMA B columns) x all tokens in
// tiles of 16 (MFMA A rows); the waves split the row's atoms (K) and reduce
// their partial tiles through LDS.  The block's packed bytes are staged in
// LDS; each lane decodes its B operand (row l%16, 8 consecutive K = one plane
// of one atom) from the 16-byte code entry.
// ---------------------------------------------------------------------------

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t hi_lo_pack(uint32_t h16, float v) {
  // returns (hi bf16 | lo bf16 << 16) for the fp16 value with bits h16 (as float v)
  (void)h16;
  if (!(fabsf(v) <= 3.0e38f)) return bf16_rne_bits(v);  // inf / nan: carried by hi alone
  const uint32_t hb = bf16_rne_bits(v);
  const float lo = v - __uint_as_float(hb << 16);
  return hb | (bf16_rne_bits(lo) << 16);
}

template <int KW, int MT>  // KW waves split K; MT token tiles of 16
__global__ __launch_bounds__(KW * 64) void dqgemm_kernel(const uint8_t *__restrict__ packed, int64_t packed_bytes,
                                                         const uint16_t *__restrict__ sigma16, int64_t rows,
                                                         int64_t atoms_per_row, const uint16_t *__restrict__ x,
                                                         int64_t m_total, float *__restrict__ y,
                                                         const uint4 *__restrict__ kp_gemv) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int NT = KW * 64;
  const int64_t cols = atoms_per_row * kDim;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * 16;
  const int64_t rows_here = min(static_cast<int64_t>(16), rows - row0);
  const int64_t atom0 = row0 * atoms_per_row;
  const int64_t g_lo = atom0 >> 2, g_hi = (atom0 + rows_here * atoms_per_row + 3) >> 2;
  const int64_t start = g_lo * 9, end = g_hi * 9, base16 = start & ~static_cast<int64_t>(15);
  const int nvec = static_cast<int>((end - base16 + 15) >> 4);
  const uint8_t *pb = smem + (start - base16);
  float *red = reinterpret_cast<float *>(smem + static_cast<int64_t>(nvec) * 16);  // [KW][MT][256] partial tiles
  for (int i = threadIdx.x; i < nvec; i += NT) {
    const int64_t gb = base16 + 16 * static_cast<int64_t>(i);
    if (gb + 16 <= packed_bytes)
      reinterpret_cast<uint4 *>(smem)[i] = *reinterpret_cast<const uint4 *>(packed + gb);
    else
      for (int k = 0; k < 16 && gb + k < packed_bytes; ++k) smem[16 * i + k] = packed[gb + k];
  }
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int j = lane & 15, q = lane >> 4;
  const int64_t row = row0 + j;
  const bool row_live = j < rows_here;
  // per-row hi/lo bf16 pairs of the magnitudes |k| = 1..4
  uint32_t mag[5];
  mag[0] = 0u;
  {
    const float sig = row_live ? __half2float(__ushort_as_half(sigma16[row])) : 0.f;
    const float sl = __uint_as_float(kSLatticeBits);
#pragma unroll
    for (int k = 1; k <= 4; ++k) {
      const uint32_t h = dq_value(k, sig, sl);
      mag[k] = hi_lo_pack(h, __half2float(__ushort_as_half(static_cast<uint16_t>(h))));
    }
  }
  f32x4_t acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // K = 24 * atoms_per_row; this wave's share of 96-wide chunks (4 atoms).
  // Two-deep pipeline: chunk ch+KW's code words and activation tiles are
  // loaded while chunk ch is decoded and multiplied.
  const int64_t n_chunks = (atoms_per_row + 3) / 4;
  auto load_chunk = [&](int64_t ch, uint32_t (&w)[3], bf16x8_t (&av)[3][MT]) {
#pragma unroll
    for (int ks = 0; ks < 3; ++ks) {
      const int kk = 32 * ks + 8 * q;
      const int64_t a = ch * 4 + kk / 24;
      const int plane = (kk % 24) / 8;
      w[ks] = 0u;
      if (ch < n_chunks && row_live && a < atoms_per_row) {
        const int64_t n = row * atoms_per_row + a - g_lo * 4;
        const uint8_t *bp = pb + (n >> 2) * 9 + 2 * (n & 3);
        const uint32_t v = (static_cast<uint32_t>(bp[0]) << 16) | (static_cast<uint32_t>(bp[1]) << 8) | bp[2];
        int32_t code = static_cast<int32_t>((v >> (6 - 2 * (n & 3))) & 0x3FFFFu);
        if (code > kKissing) code = 0;
        const uint32_t *ep = reinterpret_cast<const uint32_t *>(kp_gemv + code);
        w[ks] = ep[plane];
      }
      const int64_t kcol = ch * 96 + kk;
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int64_t tok = t * 16 + j;
        if (ch < n_chunks && tok < m_total && kcol < cols) {
          av[ks][t] = *reinterpret_cast<const bf16x8_t *>(x + tok * cols + kcol);
        } else {
#pragma unroll
          for (int c = 0; c < 8; ++c) av[ks][t][c] = __builtin_bit_cast(__bf16, static_cast<uint16_t>(0));
        }
      }
    }
  };
  uint32_t w_cur[3], w_nxt[3];
  bf16x8_t a_cur[3][MT], a_nxt[3][MT];
  load_chunk(wave, w_cur, a_cur);
  for (int64_t ch = wave; ch < n_chunks; ch += KW) {
    load_chunk(ch + KW, w_nxt, a_nxt);
#pragma unroll
    for (int ks = 0; ks < 3; ++ks) {
      bf16x8_t bh, bl;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int k = static_cast<int>(static_cast<int32_t>(w_cur[ks] << (28 - 4 * c)) >> 28);
        const int m = k < 0 ? -k : k;
        uint32_t hl = m == 0 ? mag[0] : m == 1 ? mag[1] : m == 2 ? mag[2] : m == 3 ? mag[3] : mag[4];
        if (k < 0) hl ^= 0x80008000u;  // W = hi + lo, both negated
        bh[c] = __builtin_bit_cast(__bf16, static_cast<uint16_t>(hl & 0xFFFFu));
        bl[c] = __builtin_bit_cast(__bf16, static_cast<uint16_t>(hl >> 16));
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_cur[ks][t], bh, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_cur[ks][t], bl, acc[t], 0, 0, 0);
      }
    }
#pragma unroll
    for (int ks = 0; ks < 3; ++ks) {
      w_cur[ks] = w_nxt[ks];
#pragma unroll
      for (int t = 0; t < MT; ++t) a_cur[ks][t] = a_nxt[ks][t];
    }
  }
  // reduce the KW partial tiles: C[token 4q'+e][row j] lives in lane j + 16 q', element e
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[(wave * MT + t) * 256 + e * 64 + lane] = acc[t][e];
  __syncthreads();
  for (int i = threadIdx.x; i < MT * 256; i += NT) {
    const int t = i / 256, e = (i % 256) / 64, l = i % 64;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < KW; ++w) sum += red[(w * MT + t) * 256 + e * 64 + l];
    const int64_t tok = t * 16 + 4 * (l >> 4) + e;
    const int64_t r = row0 + (l & 15);
    if (tok < m_total && r < rows) y[tok * rows + r] = sum;
  }
}

template <int KW>
int launch_dqg(const uint8_t *packed, int64_t packed_bytes, const uint16_t *sigma16, int64_t rows, int64_t apr,
               const uint16_t *x, int64_t m, float *y, const uint4 *tab, hipStream_t s) {
  const int64_t pbytes = (16 * apr + 8) / 4 * 9 + 32;
  const size_t p16 = ((static_cast<size_t>(pbytes) + 15) & ~static_cast<size_t>(15)) + 16;
  const dim3 g(static_cast<unsigned>((rows + 15) / 16));
  const int mt = static_cast<int>((m + 15) / 16);
  const size_t shm = p16 + static_cast<size_t>(KW) * (mt <= 2 ? 2 : 4) * 256 * 4;
  if (shm > 64 * 1024) return fail(PLX_EINVAL, "dequant_linear: rows of %lld atoms are too long", static_cast<long long>(apr));
  if (mt <= 2)
    hipLaunchKernelGGL((dqgemm_kernel<KW, 2>), g, dim3(KW * 64), shm, s, packed, packed_bytes, sigma16, rows, apr, x, m,
                       y, tab);
  else
    hipLaunchKernelGGL((dqgemm_kernel<KW, 4>), g, dim3(KW * 64), shm, s, packed, packed_bytes, sigma16, rows, apr, x, m,
                       y, tab);
  return check_launch("dqgemm_kernel");
}

}  // namespace

int launch_dequant_linear(const uint8_t *packed, const uint16_t *sigma16, int64_t rows, int64_t cols, const void *x,
                          int x_is_f32, int64_t m, float *y, hipStream_t s) {
  if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0 || (reinterpret_cast<uintptr_t>(packed) & 15u) != 0)
    return fail(PLX_EINVAL, "dequant_linear: x and packed must be 16-byte aligned");
  const DeviceTables *tab = nullptr;
  int st = get_tables(&tab);
  if (st != PLX_OK) return st;
  const int64_t apr = cols / kDim;
  const int64_t pb = ((rows * apr + 3) / 4) * 9;  // packed stream length
  const uint4 *kp = reinterpret_cast<const uint4 *>(tab->kp_gemv);
  // bf16 batches of 17..64 tokens: MFMA dequant-GEMM (larger batches loop over 64-token slabs)
  if (!x_is_f32 && m > 16) {
    const uint16_t *xb = static_cast<const uint16_t *>(x);
    for (int64_t m0 = 0; m0 < m; m0 += 64) {
      const int64_t mm = m - m0 < 64 ? m - m0 : 64;
      const int st2 = rows >= 4096 ? launch_dqg<4>(packed, pb, sigma16, rows, apr, xb + m0 * cols, mm, y + m0 * rows, kp, s)
                                   : launch_dqg<8>(packed, pb, sigma16, rows, apr, xb + m0 * cols, mm, y + m0 * rows, kp, s);
      if (st2 != PLX_OK) return st2;
    }
    return PLX_OK;
  }
  // lanes per row: about 2-5 atoms per lane
  if (apr >= 160)
    return x_is_f32 ? launch_dql<64, true>(packed, pb, sigma16, rows, apr, x, m, y, kp, s)
                    : launch_dql<64, false>(packed, pb, sigma16, rows, apr, x, m, y, kp, s);
  if (apr >= 40)
    return x_is_f32 ? launch_dql<32, true>(packed, pb, sigma16, rows, apr, x, m, y, kp, s)
                    : launch_dql<32, false>(packed, pb, sigma16, rows, apr, x, m, y, kp, s);
  return x_is_f32 ? launch_dql<8, true>(packed, pb, sigma16, rows, apr, x, m, y, kp, s)
                  : launch_dql<8, false>(packed, pb, sigma16, rows, apr, x, m, y, kp, s);
}

}  // namespace plx

// Internal declarations shared by the library's translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "../../include/pollux_amd.h"

namespace plx {

constexpr int kDim = 24;
constexpr int kKissing = 196560;
constexpr int kCodebook = 196561;

// MFMA codebook tiles: 16 codes per tile, stored as three K-planes
// (coordinates 8p..8p+7) of 16 rows x 8 bf16, i.e. 768 bytes per tile.
constexpr int kTileCodes = 16;
constexpr int kTileBytes = 768;

// Sweep order of the scoring kernels.  The 98,256 codes of types 1 and 2
// (+-4 pairs, +-2 octads) are closed under negation and negation reverses the
// lexicographic order, so sorted they pair up as s_k and s_{2P-1-k} = -s_k.
// The sweep scores the 98,304 type-3 codes (one -3; no antipodes in this
// codebook) in index order, then one representative per antipodal pair (the
// lower index s_k, k < P = 49,128) in index order: the score of -s_k is
// exactly -score(s_k) (bf16 operands negate exactly, fp32 sums round
// symmetrically), so a max of |score| over the representatives covers both
// members -- 147,432 codes scored instead of 196,560.  Padded with all-zero
// codes (score 0, never above the origin threshold) to whole tiles.
constexpr int kType3Codes = 98304;
constexpr int kPairCodes = 49128;
constexpr int kType3Tiles = kType3Codes / kTileCodes;                        // 6144
constexpr int kPairTiles = (kPairCodes + kTileCodes - 1) / kTileCodes;      // 3071
constexpr int kSweepTiles = 9216;  // 6144 + 3071 + 1 zero tile = 2^10 * 9
static_assert(kType3Tiles + kPairTiles <= kSweepTiles, "sweep tiles");

// Structured type-3 scoring (quantize.hip, NN-B): a type-3 code is a Golay
// sign pattern P(w) (-1 where the codeword w has a 1) times s with one
// coordinate replaced by -3s, so its score is S(w) - x_p (3s + s P_p(w)) with
// S(w) = s P(w).x.  The Golay code holds the complement of every word
// (P(~w) = -P(w)), so the 2,048 words with bit 23 clear represent all 4,096:
// pattern id r < 2048 is representative r, id r + 2048 its complement.
constexpr int kT3Reps = 2048;
constexpr int kT3Tiles = kT3Reps / kTileCodes;  // 128
constexpr int kT3Words = 2 * kT3Reps;

// Structured pair scoring (quantize.hip, NN-B): a type-2 code is +-2s on the
// 8 positions of an octad (759 weight-8 Golay words) with an even number of
// minus signs, a type-1 code +-4s on two positions.
constexpr int kT2Octads = 759;
constexpr int kT2Tiles = 48;  // 768 octad slots
constexpr int kT2Subsets5 = 42504;  // C(24, 5): each in exactly one octad
constexpr int kT3DecWords = 4096 + 12 + 24;  // Golay decoder: leaders by syndrome, basis, position syndromes

// fp32 constants of the reference (castor.py:47,50,68; castor.py:522; pack.py:164)
constexpr uint32_t kLeechScaleBits = 0x3EB504F3u;  // fp32(1/sqrt 8)
constexpr uint32_t kSLatticeBits = 0x3F3504F3u;    // fp32(1/sqrt 2)
constexpr uint32_t kCSqNormBits = 0x407FFFFFu;     // fp32 |codebook[1]|^2
constexpr uint32_t kEpsBits = 0x322BCC77u;         // fp32(1e-8)
constexpr uint32_t kSqrt12Bits = 0x405DB3D7u;      // fp32(sqrt 12)

struct DeviceTables {
  int device = -1;
  uint8_t *sw_bf16_tiles = nullptr;  // [kSweepTiles][3][16][8] bf16 bits of the sweep codes (MFMA A operands)
  uint8_t *sw_raw_tiles = nullptr;   // the same layout, bf16 bits of the raw integers (NN-P)
  uint32_t *sw_dq = nullptr;         // [kSweepTiles*16][3] value-id words of the sweep codes (rescans)
  uint32_t *sw_idx = nullptr;        // [kSweepTiles*16] codebook row of each sweep code, 0 for padding
  uint32_t *sw_anti = nullptr;       // [(kSweepTiles-kType3Tiles)*16] antipode rows, from the pair region's start
  int8_t *cb_raw = nullptr;          // [kCodebook][24] raw integer coordinates
  uint8_t *kp_gemv = nullptr;        // [kCodebook] x 16 B: 24 signed nibbles + (type | pos << 8)
  uint32_t *kp_dq = nullptr;         // [kCodebook][3] words: 3-bit value ids of 8 coordinates per word
  uint2 *kp_half = nullptr;          // [kCodebook] 6 half symbols, type, position of -3 (one byte each)
  uint4 *gv_tab = nullptr;           // [kGvVecs] half bf16 pairs [kGvHalves][2], then plane -> 2 half symbols
  uint32_t *pl_ids = nullptr;        // [n_planes] value-id word (kp_dq's format) of each distinct plane
  uint16_t *code_planes = nullptr;   // [kCodebook][4] the plane-layout record of each code (3 used)
  uint32_t *pl_nib = nullptr;        // [n_planes] the same planes as kp_gemv words: 8 signed 4-bit coordinates
  uint8_t *t3_tiles = nullptr;       // [kT3Tiles][3][16][8] bf16 sign patterns +-s of the representative words
  uint32_t *t3_words = nullptr;      // [4096] word of pattern id (representatives, then their complements)
  uint32_t *t3_rows = nullptr;       // [4096][24] codebook row of the type-3 code (word of id, -3 at position p)
  uint8_t *t2_tiles = nullptr;       // [kT2Tiles][3][16][8] bf16 octad indicators times 2s
  uint2 *t2_pos = nullptr;           // [kT2Tiles*16] the 8 positions of each octad, one byte each
  uint32_t *t2_rows = nullptr;       // [759][128] codebook row of the octad code with sign pattern p
  uint32_t *t1_rows = nullptr;       // [24][24][4] codebook row of the type-1 code at i < j, minus bits
  uint16_t *t2_steiner = nullptr;    // [kT2Subsets5] the octad holding each 5-subset (colex rank)
  uint32_t *t3_dec = nullptr;        // [kT3DecWords] Golay coset leaders by syndrome, basis words, position syndromes
};

// Plane tables (tables.cpp; host, built once): the codebook rows take only a
// few thousand distinct 8-coordinate planes.  ids = their value-id words
// (kp_dq's format), ascending; code_planes[4 code + p] = the record of code's
// plane p in the plane layout: plane index (13 bits) | extra << 13, the extra
// bits being the code's type (record 0), bits 0-2 of its -3 position (record
// 1) and bits 3-4 (record 2).
constexpr int kMaxPlanes = 8192;
// The one-token dequant-GEMV's table (gv_tab): kGvHalves halves of 2 bf16
// pairs (8 B), then kGvPlanes uint16 plane entries, as whole 16-byte vectors.
constexpr int kGvHalves = 168;
constexpr int kGvPlanes = 4992;
constexpr int kGvHalfVecs = kGvHalves * 8 / 16;
constexpr int kGvVecs = kGvHalfVecs + kGvPlanes * 2 / 16;
struct PlaneTables {
  std::vector<uint32_t> ids;
  std::vector<uint16_t> code_planes;
};
const PlaneTables *plane_tables_host();

// Host generator (codebook.cpp): raw coordinates, origin first, sorted.
const int8_t *codebook_raw_host();
// The 4,096 extended Golay codewords (bit b = coordinate b), message order (codebook.cpp).
const uint32_t *golay_words_host();
// fp32 value of raw coordinate k (k in -4..4): k * fp32(1/sqrt 8), rounded to fp32.
float raw_to_f32(int k);

// Lazily built per-device tables for the current device (tables.cpp).
int get_tables(const DeviceTables **out);
// The current device's tables if plx_device_init (or any earlier call) built
// them; PLX_EINVAL without allocating anything otherwise (tables.cpp).
int get_tables_built(const DeviceTables **out);

// Error reporting (capi.cpp).
int fail(int code, const char *fmt, ...);
int check_hip(hipError_t e, const char *what);
int check_launch(const char *what);

// Event bracketing of the scoring kernel (profile.cpp); no-ops unless enabled.
// `kernel`: the PLX_PROF_* id of the bracketed kernel; only the selected one is recorded.
void profile_before(hipStream_t s, int kernel = PLX_PROF_NN);
void profile_after(hipStream_t s, int kernel = PLX_PROF_NN);

// Kernel launchers (one per .hip file); return PLX_* status.
int launch_pack(const void *idx, int idx_is_i64, int64_t n, uint8_t *out, hipStream_t s);
int launch_unpack(const uint8_t *packed, int64_t num_indices, int64_t *out, hipStream_t s);
int launch_row_rms(const float *w, int64_t rows, int64_t cols, float *sigma, uint16_t *sigma16,
                   hipStream_t s);
int launch_quantize(const float *x, const float *sigma, int64_t rows, int64_t cols, int64_t n_atoms,
                    int mode, int32_t *idx_out, uint8_t *packed_out, float *weight_out,
                    void *workspace, size_t workspace_bytes, hipStream_t s);
size_t quantize_workspace_bytes(int64_t n_atoms);
// The checks launch_quantize makes before its first launch (workspace size, 16-byte alignment of the
// input and the workspace, grid limits); composite entry points run them before launching anything.
int check_quantize_args(const float *x, int64_t n_atoms, const void *workspace, size_t workspace_bytes);
// The allocation-free requantize (quantize.hip): its workspace is the file-scope
// device array `scratch`, whose per-device address noalloc_setup() resolves
// once per device (current device) and caches.
int noalloc_setup();
int launch_requantize_noalloc(const float *latent, int64_t rows, int64_t cols, int mode, float *sigma_out,
                              int32_t *idx_out, uint8_t *packed_out, float *weight_out, hipStream_t s);
// One matrix of a batched requantize (the latent's row scale, indices, packed
// bytes and reconstructed weight; packed and weight may be null).
struct RequantItem {
  const float *latent;
  int64_t rows, cols;
  float *sigma;
  int32_t *idx;
  uint8_t *packed;
  float *weight;
};
int launch_requantize_batch(const RequantItem *items, int n_items, int mode, void *workspace, size_t workspace_bytes,
                            hipStream_t s);
int launch_gather(const int32_t *idx, int64_t n, int out_dtype, void *out, hipStream_t s);
int launch_dequant_f16(const uint8_t *packed, const uint16_t *sigma16, int64_t rows, int64_t cols,
                       uint16_t *w16, hipStream_t s);
int launch_int8_linear(const int8_t *q, const uint16_t *mu16, int64_t rows, int64_t cols, const float *x, int64_t m,
                       const float *norm_w, float eps, float *y, uint64_t *keys, hipStream_t s);
int launch_int8_linear_argmax(const int8_t *q, const uint16_t *mu16, int64_t rows, int64_t cols, const float *x,
                              int64_t m, const float *norm_w, float eps, float *y, int64_t *ids, int64_t *history,
                              int64_t hist_len, int64_t *pos, void *workspace, size_t workspace_bytes, hipStream_t s);
size_t int8_linear_argmax_workspace_bytes(int64_t rows, int64_t m);
int launch_int8_embed(const int8_t *q, const uint16_t *mu16, int64_t vocab, int64_t cols, const int64_t *idx,
                      int64_t n, int64_t t, const float *pos_w, int64_t pos_rows, const int64_t *pos0, float *out,
                      hipStream_t s);
int launch_argmax_rows(const float *x, int64_t rows, int64_t cols, int64_t *out, hipStream_t s);
int launch_rms_norm(const float *x, const float *w, float *y, int64_t rows, int64_t d, float eps, hipStream_t s);
int launch_decode_attention(const float *q, const float *k, const float *v, int64_t qkv_stride, int64_t heads,
                            const float *q_w, const float *k_w, float eps, float *k_cache, float *v_cache,
                            const int64_t *pos, int64_t seqs_heads, int64_t max_len, float *out, hipStream_t s);
int launch_prefill_attention(const float *q, const float *k, const float *v, int64_t qkv_stride, const float *q_w,
                             const float *k_w, float eps, float *k_cache, float *v_cache, int64_t b, int64_t heads,
                             int64_t t, int64_t p0, int64_t max_len, float *out, hipStream_t s);
// One weight of a multi-target dequant-linear call (all share x and cols).
struct DqlTarget {
  const uint8_t *packed;
  const uint16_t *sigma16;
  int64_t rows;
  float *y;
  const float *residual;  // y = residual + (x W^T) when not null
};
size_t dequant_linear_workspace_bytes_multi(const int64_t *rows, int n, int64_t cols, int64_t m, int flags);
int launch_dequant_linear_multi(const DqlTarget *targets, int n, int64_t cols, const void *x, int flags, int64_t m,
                                const float *norm_w, float norm_eps, void *workspace, size_t workspace_bytes,
                                hipStream_t s);
size_t dequant_linear_workspace_bytes(int64_t rows, int64_t cols, int64_t m, int flags);
// packed 18-bit indices -> plane layout (3 uint16 records per atom)
int launch_plane_layout(const uint8_t *packed, int64_t n_atoms, uint16_t *planes, hipStream_t s);
int launch_dequant_linear(const uint8_t *packed, const uint16_t *sigma16, int64_t rows, int64_t cols, const void *x,
                          int flags, int64_t m, float *y, void *workspace, size_t workspace_bytes, hipStream_t s);
size_t adam_h24_workspace_bytes(int64_t n_atoms);
int launch_adam_h24(const float *grad, float *m, float *v, float *latent, int64_t n_atoms, const float *scalars,
                    float *adam_norm_out, void *workspace, hipStream_t s);
int launch_int8_quant(const float *w, int64_t rows, int64_t cols, int8_t *q, uint16_t *mu16, hipStream_t s);
int launch_int8_dequant(const int8_t *q, const uint16_t *mu16, int64_t rows, int64_t cols, uint16_t *w16,
                        hipStream_t s);

}  // namespace plx

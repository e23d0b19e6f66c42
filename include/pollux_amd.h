/*
 * pollux_amd.h -- C ABI of the MI355X (gfx950) Leech-lattice quantization library.
 *
 * Every entry point takes plain pointers, element counts and a hipStream_t
 * (passed as void*; NULL = the legacy default stream) and returns an int
 * status: PLX_OK (0) or one of the PLX_E* codes below, with a message
 * retrievable from plx_last_error().  Device pointers must live on the
 * current HIP device.  No entry point allocates its outputs: callers own all
 * buffers.  Work is enqueued on the given stream and not synchronised.
 *
 * Each function names the reference interface it replaces
 * (alavicka/pollux, file:line).
 */
#ifndef POLLUX_AMD_H
#define POLLUX_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define PLX_OK 0
#define PLX_EINVAL 1  /* bad argument: shape, size, null pointer, mode */
#define PLX_EHIP 2    /* a HIP runtime call or kernel launch failed */
#define PLX_ENOMEM 3  /* a one-time device table allocation failed */

/* ---- nearest-neighbour semantics -------------------------------------- */
/* NN-B: bf16 operands, fp32 accumulation, score rounded to bf16, lowest index
 *       among equal maxima, origin iff 2*max < 0x407FFFFF.  The reference's
 *       non-Triton path, castor.py:544-557. */
#define PLX_NN_BF16_SCORES 0
/* NN-T: bf16 operands, fp32 accumulation and fp32 scores, lowest index among
 *       equal maxima, same origin rule.  The reference's Triton kernel,
 *       castor.py:407-460. */
#define PLX_NN_FP32_SCORES 1
/* NN-P: fp32 atoms against the fp32 codebook, first (lowest-index) maximum of
 *       the fp32 scores, origin iff ||atom||_2 < 1e-8 (no score threshold;
 *       invariant under positive scaling of the atom).  The reference's
 *       pack-time search, pack._quantize_h24_layer (pack.py:167-177). */
#define PLX_NN_PACK_FP32 2
/* Flag OR'ed into PLX_NN_BF16_SCORES (quantize / requantize entry points):
 * score every code densely on MFMA (one contraction per type-3 code and per
 * antipodal pair of type-1/2 codes) instead of the default structured
 * scorers, which score the 759 octads' sums of |x| and the 2,048 Golay
 * sign-pattern pairs and evaluate the few candidate codes exactly.  Both have
 * NN-B semantics (equal answers off near-ties); the dense sweep is kept as
 * the measured baseline of the structured one.  Ignored by the other modes. */
#define PLX_NN_DENSE_TYPE3 0x100
/* Flag OR'ed into PLX_NN_BF16_SCORES for plx_quantize (diagnostics): the
 * structured scorers find the lowest row at the best bucket by a second sweep
 * over the octads and the patterns -- the path each takes when a per-wave list
 * of surviving octads / words overflows -- instead of from those lists.  Same
 * results. */
#define PLX_NN_T3_ROWS_BY_SWEEP 0x200

/* ---- element types of plx_gather_codebook's output -------------------- */
#define PLX_DTYPE_F32 0
#define PLX_DTYPE_F16 1
#define PLX_DTYPE_BF16 2

/* ---- constants (castor.py:34-68) --------------------------------------- */
#define PLX_H24_DIM 24
#define PLX_KISSING_COUNT 196560
#define PLX_CODEBOOK_COUNT 196561
#define PLX_INDEX_BITS 18
#define PLX_INDICES_PER_CHUNK 4
#define PLX_BYTES_PER_CHUNK 9

/* Message describing the last failed call on this host thread ("" if none). */
const char *plx_last_error(void);

/* Library ABI version (monotone). */
int plx_version(void);

/* ---- codebook (host) --------------------------------------------------- */
/* Raw integer coordinates of the 196,561-row codebook, origin first, rows in
 * the reference's lexicographic order; out: int8[196561*24].
 * Replaces the generator of castor.py:74-190 (_build_codebook_cpu). */
int plx_codebook_raw(int8_t *out, int64_t n_bytes);

/* The reference's fp32 table raw*fp32(1/sqrt(8)); out: float[196561*24].
 * Replaces castor._build_codebook_cpu() / get_h24_codebook (castor.py:146-199). */
int plx_codebook_f32(float *out, int64_t n_floats);

/* First 4x4 block of the fp32 codebook; out: float[16].
 * Replaces castor.codebook_fingerprint (castor.py:263-266). */
int plx_codebook_fingerprint(float *out16);

/* Build (once per device) the device-resident codebook tables on the current
 * device and resolve the device address of plx_requantize_noalloc's scratch
 * array.  Every compute entry point except plx_requantize_noalloc builds the
 * tables lazily; calling it up front moves the one-time upload out of the
 * first timed call. */
int plx_device_init(void);

/* ---- 18-bit packing (castor.py:226-260) --------------------------------- */
/* indices: int64[n] (idx_is_i64 = 1) or int32[n] (idx_is_i64 = 0).
 * out: uint8[((n+3)/4)*9]; 72-bit big-endian groups of four 18-bit indices,
 * zero padded.  Replaces castor.pack_indices (castor.py:226-246). */
int plx_pack_indices(const void *indices, int idx_is_i64, int64_t n, uint8_t *out, void *stream);

/* packed: uint8[n_packed_bytes], n_packed_bytes % 9 == 0; out: int64[num_indices]
 * with num_indices <= 4*n_packed_bytes/9.  Replaces castor.unpack_indices
 * (castor.py:249-260). */
int plx_unpack_indices(const uint8_t *packed, int64_t n_packed_bytes, int64_t num_indices,
                       int64_t *out, void *stream);

/* ---- row scale (castor.py:309-339, pack.py:164) ------------------------ */
/* sigma[r] = sqrt(mean(w[r,:]^2) + 1e-8) in fp32; w: float[rows*cols].
 * Replaces castor.row_rms_from_matrix (castor.py:309-313). */
int plx_row_rms(const float *w, int64_t rows, int64_t cols, float *sigma, void *stream);

/* sigma16[r] = fp16(max(row_rms(w)[r] * fp32(sqrt 12), 1e-8)) as raw fp16 bits.
 * Replaces the sigma line of pack._quantize_h24_layer (pack.py:164). */
int plx_sigma16_pack(const float *w, int64_t rows, int64_t cols, uint16_t *sigma16, void *stream);

/* ---- nearest-neighbour quantizer --------------------------------------- */
/* Workspace (device bytes) plx_quantize / plx_requantize need for n_atoms. */
size_t plx_quantize_workspace_bytes(int64_t n_atoms);

/* x: float[n_atoms*24] lattice coordinates; idx_out: int32[n_atoms] codebook
 * indices (0 = origin).  mode: PLX_NN_*.  Replaces the index computation of
 * castor_quantize_leech (castor.py:487-560: _leech_nn_triton / the chunked
 * fallback loop). */
int plx_quantize(const float *x, int64_t n_atoms, int mode, int32_t *idx_out,
                 void *workspace, size_t workspace_bytes, void *stream);

/* out[i,:] = codebook[idx[i],:] cast (RNE) to out_dtype (PLX_DTYPE_*);
 * indices outside 0..196560 read row 0.  Replaces
 * codebook.to(dtype).index_select(0, indices) (castor.py:533,559). */
int plx_gather_codebook(const int32_t *idx, int64_t n, int out_dtype, void *out, void *stream);

/* The per-step requantize of one fp32 latent [rows, cols] (cols % 24 == 0):
 *   sigma = row_rms(latent); x = (latent/sigma)/fp32(1/sqrt 2);
 *   idx = NN(x); weight = (codebook[idx]*sigma)*fp32(1/sqrt 2)
 * Outputs: sigma_out float[rows] and idx_out int32[rows*cols/24] (required);
 * packed_out uint8[((N+3)/4)*9] and weight_out float[rows*cols] (nullable).
 * Replaces pollux.py:874-884 (normalize_matrix_by_row_rms ->
 * castor_quantize_leech -> scale_matrix_by_row_rms) followed by
 * castor.pack_indices. */
int plx_requantize(const float *latent, int64_t rows, int64_t cols, int mode,
                   float *sigma_out, int32_t *idx_out, uint8_t *packed_out, float *weight_out,
                   void *workspace, size_t workspace_bytes, void *stream);

/* plx_requantize without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving or
 * training loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference: it serves those callers only.  Same arguments, results and
 * errors as plx_requantize minus the workspace, which is a library-owned
 * device array of PLX_NOALLOC_MAX_ATOMS * 128 bytes (128 MiB) held by each
 * device the library runs on until the process ends.  It allocates nothing:
 * call plx_device_init() on the device first (outside any capture), which
 * builds the codebook tables and resolves the array's address; without it
 * the call fails with PLX_EINVAL.  More than PLX_NOALLOC_MAX_ATOMS atoms
 * (rows * cols / 24) fail with PLX_EINVAL.  All calls on one device share
 * the array: calls that overlap in time on one device (different streams)
 * race and must be serialised by the caller. */
#define PLX_NOALLOC_MAX_ATOMS 1048576
int plx_requantize_noalloc(const float *latent, int64_t rows, int64_t cols, int mode, float *sigma_out,
                           int32_t *idx_out, uint8_t *packed_out, float *weight_out, void *stream);

/* One matrix of plx_requantize_batch: the arguments of plx_requantize. */
typedef struct plx_requantize_item {
  const float *latent;   /* float[rows*cols], 16-byte aligned */
  int64_t rows, cols;    /* cols % 24 == 0 */
  float *sigma_out;      /* float[rows] */
  int32_t *idx_out;      /* int32[rows*cols/24] */
  uint8_t *packed_out;   /* uint8[((N+3)/4)*9] or NULL */
  float *weight_out;     /* float[rows*cols] or NULL */
} plx_requantize_item;

/* plx_requantize of n_items latents with one scoring sweep over all their
 * atoms (a layer's matrices, or every parameter of an optimiser step): the
 * results equal n_items separate plx_requantize calls (up to near-ties).
 * items is a HOST array; workspace: plx_quantize_workspace_bytes(total atoms).
 * Replaces the per-parameter requantize of the pollux_step loop
 * (pollux.py:828-884) for the H24 parameters of one step. */
int plx_requantize_batch(const plx_requantize_item *items, int n_items, int mode,
                         void *workspace, size_t workspace_bytes, void *stream);

/* Pack-time quantization of one weight [rows, cols] (cols % 24 == 0):
 *   idx = NN-P(w atoms); packed_out = pack(idx) (uint8[((N+3)/4)*9]);
 *   sigma16_out[r] = fp16(max(row_rms(w)[r] * fp32(sqrt 12), 1e-8)) (raw bits);
 * idx_out int32[N] is nullable.  Replaces pack._quantize_h24_layer
 * (pack.py:139-180) including its castor.pack_indices call. */
int plx_quantize_layer_pack(const float *w, int64_t rows, int64_t cols, uint8_t *packed_out,
                            uint16_t *sigma16_out, int32_t *idx_out, void *workspace,
                            size_t workspace_bytes, void *stream);

/* ---- fused optimiser step + requantize (pollux.py:836-884) ------------ */
/* Workspace (device bytes) plx_pollux_step_h24 needs for a [rows, cols] parameter. */
size_t plx_pollux_step_workspace_bytes(int64_t rows, int64_t cols);

/* One optimiser step of one H24 parameter [rows, cols] (cols % 24 == 0), all
 * fp32 and 16-byte aligned, m / v / latent updated in place:
 *   m = fma(g, 1-b1, m*b1);  v = fma((1-b2)*g, g, v*b2);
 *   s = neg_scale * ((m/bc1) / (sqrt(v/bc2) + 1e-8));
 *   per 24-element atom: s *= min(reciprocal(|s|_2 + 1e-8) * cap, 1);
 *   latent = latent*wdf + s;
 * then the requantize of plx_requantize on the new latent (sigma_out, idx_out
 * required; packed_out, weight_out nullable; weight_out is the parameter's
 * new data), and, if adam_norm_out is not NULL, adam_norm_out[0] = |s|_2 over
 * the whole parameter (nothing is written when rows == 0).  scalars: DEVICE
 * float[9] = {b1, 1-b1, b2, 1-b2, max(bc1, 1e-8), max(bc2, 1e-8),
 * neg_scale, wdf, cap} as the reference's
 * 0-dim fp32 tensors evaluate them (bc = 1 - b^(step+1); neg_scale =
 * -(heat*gamma/C / width_inertia); wdf = 1 - heat*gamma^2; cap =
 * KINEMATIC_LIMIT*s_lattice), so no host synchronisation is needed.
 * Replaces the H24 branch of pollux_step (pollux.py:836-884) and its
 * vector_norm contribution to adam_energy_sum (pollux.py:886-888). */
int plx_pollux_step_h24(const float *grad, float *m, float *v, float *latent, int64_t rows, int64_t cols,
                        const float *scalars, int mode, float *sigma_out, int32_t *idx_out,
                        uint8_t *packed_out, float *weight_out, float *adam_norm_out,
                        void *workspace, size_t workspace_bytes, void *stream);

/* One H24 parameter of plx_pollux_step_h24_batch: the per-parameter
 * arguments of plx_pollux_step_h24. */
typedef struct plx_pollux_step_item {
  const float *grad;     /* float[rows*cols], 16-byte aligned */
  float *m, *v, *latent; /* float[rows*cols], 16-byte aligned, updated in place */
  int64_t rows, cols;    /* cols % 24 == 0 */
  float *sigma_out;      /* float[rows] */
  int32_t *idx_out;      /* int32[rows*cols/24] */
  uint8_t *packed_out;   /* uint8[((N+3)/4)*9] or NULL */
  float *weight_out;     /* float[rows*cols] or NULL: the parameter's new data */
  float *adam_norm_out;  /* float[1] or NULL: |s|_2 over the parameter (not written when rows == 0) */
} plx_pollux_step_item;

/* Workspace (device bytes) plx_pollux_step_h24_batch needs for these items
 * (items is a HOST array). */
size_t plx_pollux_step_batch_workspace_bytes(const plx_pollux_step_item *items, int n_items);

/* One optimiser step of every H24 parameter of a pollux_step call: per
 * parameter the update of plx_pollux_step_h24 (one pass over grad, m, v and
 * the latent), then the requantize of all new latents with one scoring sweep
 * over all their atoms (plx_requantize_batch).  m, v and the latents are
 * bit-identical to n_items plx_pollux_step_h24 calls; indices equal them up
 * to near-ties.  scalars: the DEVICE float[9] of plx_pollux_step_h24, shared
 * by every item (the reference computes them once per step: one heat, one
 * step counter, one width_inertia for all matrices, pollux.py:785, 815-820,
 * 849-852).  items is a HOST array.  Replaces the loop over the H24 tensors
 * of pollux_step (pollux.py:828-888), tok_emb, pos_emb and head included. */
int plx_pollux_step_h24_batch(const plx_pollux_step_item *items, int n_items, const float *scalars, int mode,
                              void *workspace, size_t workspace_bytes, void *stream);

/* ---- dequantization (pollux.py:485-507) -------------------------------- */
/* w16 = fp16(fp16(codebook16[unpack(packed)] * sigma16[row]) * fp32(1/sqrt 2)),
 * shape [rows, cols] as raw fp16 bits.  Replaces PackedH24Linear.materialize
 * (pollux.py:485-504). */
int plx_dequant_f16(const uint8_t *packed, int64_t n_packed_bytes, const uint16_t *sigma16,
                    int64_t rows, int64_t cols, uint16_t *w16_out, void *stream);

/* plx_dequant_linear flags (0 = bf16 activations, exact fp16 weights) */
#define PLX_DQL_X_F32 1  /* x is fp32 (else bf16) */
#define PLX_DQL_W_AS_X 2 /* bf16 x: round W to bf16 first, as the reference's literal
                            F.linear(x, W.to(x.dtype)) does (pollux.py:507) */
#define PLX_DQL_GELU 4   /* y = gelu(x W^T), torch's erf form (pollux.py:645) */
#define PLX_DQL_RMS_NORM 8 /* plx_dequant_linear_multi only: RMS-normalise each fp32 x
                              row first (pre-norm of pollux.py:660-661) */
#define PLX_DQL_PLANES 16  /* `packed` is the plane layout of the weight
                              (plx_h24_plane_layout, 6 bytes per atom) instead of
                              the 18-bit stream (each target's, for
                              plx_dequant_linear_multi); taken for one token
                              (rows of at most 320 atoms) and for batches above
                              4 tokens, with the same results */

/* The plane layout of a packed weight: per atom 3 little-endian uint16
 * records (6 bytes, atom order), one per 8-coordinate plane: a 13-bit index
 * into the table of the 4,961 distinct planes of the codebook rows
 * (plx_plane_table) | 3 extra bits (record 0: the code's type, 0 origin,
 * 1 = +-4 pair, 2 = +-2 octad, 3 = one -3; records 1 and 2: bits 0-2 and 3-4 of
 * the -3 position).  Kernels decode a code from a table they keep in LDS
 * instead of gathering from the 3 MB per-code tables, so a packed layer built
 * once into this layout (6 B per atom next to its 2.25 B packed stream) runs
 * its dequant-linear without per-atom gathers.  packed: n_packed_bytes =
 * ((n_atoms+3)/4)*9 bytes (indices above 196,560 map to the origin); planes:
 * [3*n_atoms].
 * No counterpart in the reference (a derived layout of its packed buffers). */
int plx_h24_plane_layout(const uint8_t *packed, int64_t n_packed_bytes, int64_t n_atoms, uint16_t *planes,
                         void *stream);
/* Host copy of the plane table: value-id words (kp_dq order: byte i = id of
 * coordinate i | id of coordinate 4+i << 4, ids 0..7 = raw values
 * {0,1,2,4,-4,-3,-2,-1}), ascending.  Returns the number of planes; copies at
 * most `capacity` of them into ids (which may be NULL).  Needs no device. */
int64_t plx_plane_table(uint32_t *ids, int64_t capacity);

/* Workspace (device bytes, 16-byte aligned) plx_dequant_linear needs for
 * this shape, batch and flags (0 when none). */
size_t plx_dequant_linear_workspace_bytes(int64_t rows, int64_t cols, int64_t m_rows, int flags);

/* y[m, r] = sum_i x[m, i] * W[r, i] for m < m_rows, with W the fp16
 * materialisation of (packed, sigma16) above, never stored: x is bf16 or fp32
 * (PLX_DQL_X_F32) [m_rows, cols], y fp32 [m_rows, rows].  The products with
 * the fp16 weights are exact and accumulated in fp32: the numerics of
 * F.linear(x.float(), W.float()).  With PLX_DQL_W_AS_X and bf16 x the weights
 * are rounded to bf16 (RNE) first; with PLX_DQL_GELU, y = gelu(x W^T) (torch's
 * erf form).  Results are deterministic (fixed summation order).  Batches
 * above 4 tokens of fp32 x (split exactly into three bf16 parts) or above 2 of
 * bf16 x run on MFMA and need the workspace sized by
 * plx_dequant_linear_workspace_bytes (a fragment-order copy of x, plus split
 * partial tiles for narrow layers); cols <= 2^22.
 * Replaces PackedH24Linear.forward after materialize (pollux.py:506-507:
 * F.linear(x, weight.to(x.dtype))). */
int plx_dequant_linear(const uint8_t *packed, int64_t n_packed_bytes, const uint16_t *sigma16,
                       int64_t rows, int64_t cols, const void *x, int flags, int64_t m_rows,
                       float *y, void *workspace, size_t workspace_bytes, void *stream);

/* Several packed weights that share one x (e.g. the q, k and v projections,
 * pollux.py:616-621) in one call: for each target i,
 * y_i = [residual_i +] act(n(x) W_i^T) with W_i [rows_i, cols] as in
 * plx_dequant_linear (act = GELU with PLX_DQL_GELU, else identity; residual_i
 * may be NULL: the residual adds of pollux.py:660-661).  n(x) = x, or with
 * PLX_DQL_RMS_NORM (fp32 x; norm_weight fp32 [cols], 16-byte aligned)
 * x * rsqrt(mean(x^2) + norm_eps) * norm_weight per row, the block's ln1 /
 * ln2 (pollux.py:580-582); norm_weight is NULL without the flag.  Up to 16
 * targets; at m_rows <= 4 up to four of them run in one GEMV launch, which
 * normalises x in LDS.  No counterpart in the reference's FFI (separate
 * RMSNorm and F.linear calls there); results equal plx_rms_norm followed by
 * separate plx_dequant_linear calls and the epilogue, up to the summation
 * order of the norm's sum of squares. */
typedef struct {
  const uint8_t *packed;     /* ((rows*cols/24 + 3)/4)*9 bytes, 16-byte aligned */
  const uint16_t *sigma16;   /* [rows] fp16 bits */
  int64_t rows;
  float *y;                  /* [m_rows, rows] fp32 */
  const float *residual;     /* [m_rows, rows] fp32 or NULL */
} plx_dql_target;

size_t plx_dequant_linear_multi_workspace_bytes(const plx_dql_target *targets, int n_targets, int64_t cols,
                                                int64_t m_rows, int flags);
int plx_dequant_linear_multi(const plx_dql_target *targets, int n_targets, int64_t cols, const void *x,
                             int flags, int64_t m_rows, const float *norm_weight, float norm_eps,
                             void *workspace, size_t workspace_bytes, void *stream);

/* ---- packed decoder steps ------------------------------------------------
 * No counterpart in the reference's FFI: the reference runs these steps as
 * torch ops.  They serve the KV-cached decode of the packed Pollux decoder
 * (pollux_amd.model), one kernel each instead of a chain of elementwise and
 * reduction kernels. */
/* y[r, :] = x[r, :] * rsqrt(mean(x[r, :]^2) + eps) * w, fp32 x, y [rows, d] and
 * w [d], d % 4 == 0, 16-byte aligned, y not overlapping x (RMSNorm.forward,
 * pollux.py:580-582). */
int plx_rms_norm(const float *x, const float *w, float *y, int64_t rows, int64_t d, float eps, void *stream);

/* The attention of one new token per sequence (pollux.py:615-626 at the last
 * position).  q, k, v: fp32 [n, 24] projections of the new token, n = sequences
 * x heads, or with qkv_stride > 0 each sequence's row of `heads` heads
 * qkv_stride floats apart, an even number (q, k and v as column slices of one
 * stacked projection); q_norm_w, k_norm_w: fp32 [24] (q_ln, k_ln weights); q,
 * k, v and the weights 8-byte aligned; caches fp32
 * [n, max_len, 24] (16-byte aligned); *pos: the new token's position (device
 * int64).  Writes RMSNorm(k) and v at position *pos, then out fp32 [n, 24] =
 * softmax_{j <= pos}(RMSNorm(q) . K_j / sqrt 24) V_j.  A position outside
 * 0..max_len-1 writes nothing to the caches and sets out to NaN. */
int plx_decode_attention(const float *q, const float *k, const float *v, int64_t qkv_stride, const float *q_norm_w,
                         const float *k_norm_w, float eps, float *k_cache, float *v_cache, const int64_t *pos,
                         int64_t n, int64_t heads, int64_t max_len, float *out, void *stream);

/* The attention of t new positions p0 .. p0+t-1 of each of b sequences (a
 * prompt's prefill over a cached prefix: pollux.py:615-626 with is_causal,
 * positions < p0 taken from the caches).  q, k, v, out: fp32 [b, t, heads,
 * 24] (the projections' [b, t, heads*24] rows; with qkv_stride > 0 the rows of
 * q, k and v are qkv_stride floats apart, a multiple of 4: column slices of one
 * stacked projection); q_norm_w, k_norm_w: fp32 [24];
 * caches fp32 [b, heads, max_len, 24].  Writes RMSNorm(k) and v at positions
 * p0 .. p0+t-1, then out[s, i, h] = softmax_{j <= p0+i}(RMSNorm(q_i) . K_j /
 * sqrt 24) V_j.  All arrays 16-byte aligned; p0 + t <= max_len.  Replaces the
 * q_ln / k_ln calls, the cache writes and F.scaled_dot_product_attention of the
 * attention's multi-token path (no counterpart in the reference, which has no
 * cache: with p0 = 0 it is pollux.py:615-626 itself). */
int plx_prefill_attention(const float *q, const float *k, const float *v, int64_t qkv_stride, const float *q_norm_w,
                          const float *k_norm_w, float eps, float *k_cache, float *v_cache, int64_t b, int64_t heads,
                          int64_t t, int64_t p0, int64_t max_len, float *out, void *stream);

/* out[r] = the index of the maximum of x[r, :] (fp32 [rows, cols], int64 out):
 * torch.argmax's rule (the first index among equal maxima; a NaN counts as the
 * maximum).  Greedy decoding's token choice (generate.py:313-320, top_k = 1)
 * inside a captured decode step. */
int plx_argmax_rows(const float *x, int64_t rows, int64_t cols, int64_t *out, void *stream);

/* ---- per-row INT8 periphery (embeddings / LM head in .plx files) ------- */
/* q_out int8[rows*cols] = int8(clamp(rint((w / mu) * 127), -128, 127)),
 * mu16_out[r] = fp16(mu) with mu = max(max_j |w[r,j]|, 1e-8); all fp32 IEEE ops.
 * Replaces pack._quantize_int8 (pack.py:124-136). */
int plx_quantize_int8_rows(const float *w, int64_t rows, int64_t cols, int8_t *q_out,
                           uint16_t *mu16_out, void *stream);

/* w16_out[r,j] = fp16(q[r,j] * fp16(mu16[r] * fp32(1/127))) as raw fp16 bits.
 * Replaces PackedInt8Embedding/PackedInt8Linear.materialize (pollux.py:521-530,
 * 551-560) as torch evaluates it on fp16 device tensors. */
int plx_dequant_int8_rows(const int8_t *q, const uint16_t *mu16, int64_t rows, int64_t cols,
                          uint16_t *w16_out, void *stream);

/* y[m, r] = sum_j n(x)[m, j] * w16[r, j] for m < m_rows (fp32 x [m_rows, cols],
 * y fp32 [m_rows, rows]), with w16 = the materialisation above, never stored:
 * exact products accumulated in fp32, the numerics of PackedInt8Linear.forward
 * (pollux.py:562-563, F.linear(x, W.to(x.dtype))).  n(x) = x, or with a
 * norm_weight (fp32 [cols]) x * rsqrt(mean(x^2) + norm_eps) * norm_weight per
 * token (the final norm ln_f before the head, pollux.py:699-700).
 * cols % 16 == 0 and <= 4,096; q, x, norm_weight 16-byte aligned.  Up to 4
 * tokens a GEMV streams the INT8 rows once per 4 tokens; from 5 tokens an MFMA
 * kernel reads them once per 64 tokens (both exact products, fp32 sums; with a
 * norm the MFMA kernel scales each token's sums by the rsqrt at the end). */
int plx_int8_linear(const int8_t *q, const uint16_t *mu16, int64_t rows, int64_t cols, const float *x,
                    int64_t m_rows, const float *norm_weight, float norm_eps, float *y, void *stream);

/* plx_int8_linear with greedy decoding's token choice fused in: y as above,
 * then ids[t] = the index of the maximum of y[t, :] (int64 [m_rows]) by
 * torch.argmax's rule (the first index among equal maxima; a NaN counts as
 * the maximum) -- generate.py:313-320 with top_k = 1 after the head
 * (pollux.py:699-702).  With pos (device int64): history[t, *pos + 1] = ids[t]
 * (int64 [m_rows, hist_len], written when *pos + 1 lies in [0, hist_len);
 * history may be null), then *pos += 1 -- the token record and position
 * advance of a greedy decode step.  Each block of the GEMV keeps its best
 * (value, index) per token in the workspace (the size below, 8-byte
 * aligned; nothing needs clearing) and one more block picks the winner: two
 * launches instead of the GEMV, an argmax and the bookkeeping. */
size_t plx_int8_linear_argmax_workspace_bytes(int64_t rows, int64_t m_rows);
int plx_int8_linear_argmax(const int8_t *q, const uint16_t *mu16, int64_t rows, int64_t cols, const float *x,
                           int64_t m_rows, const float *norm_weight, float norm_eps, float *y, int64_t *ids,
                           int64_t *history, int64_t hist_len, int64_t *pos, void *workspace, size_t workspace_bytes,
                           void *stream);

/* out[b, i, :] = fp32(w16[ids[b, i], :]) + pos_weight[*pos0 + i, :] for b < batch,
 * i < t (fp32 out [batch, t, cols]): PackedInt8Embedding.forward plus the
 * position embedding (pollux.py:532-533, 691-693) in one kernel.  pos_weight
 * fp32 [pos_rows, cols] or NULL (no position term); pos0: device int64 start
 * position (NULL = 0), read at run time.  An id outside 0..vocab-1 or a
 * position outside 0..pos_rows-1 yields a NaN row.  cols % 4 == 0; q 4-byte,
 * pos_weight and out 16-byte aligned.  No counterpart in the reference's FFI
 * (embedding gather, cast and add are separate torch ops there). */
int plx_int8_embed(const int8_t *q, const uint16_t *mu16, int64_t vocab, int64_t cols, const int64_t *ids,
                   int64_t batch, int64_t t, const float *pos_weight, int64_t pos_rows, const int64_t *pos0,
                   float *out, void *stream);

/* ---- kernel timing (diagnostics; no counterpart in the reference) ------ */
/* While enabled, every launch of the selected kernel (default: the
 * quantizer's scoring kernel nn_kernel) is bracketed by HIP events recorded
 * on its launch stream (up to 4096 launches).  plx_profile_select() picks
 * the kernel (while recording is off); plx_profile_begin() clears and
 * enables recording; plx_profile_end() disables it, waits for the recorded
 * events and returns the summed kernel time (ms) and the number of
 * launches.  Used by bench.py for the roofline's per-launch kernel duration
 * and the HBM kernels' bandwidth. */
#define PLX_PROF_NN 0      /* nn_kernel (the dense sweep of plx_quantize / plx_requantize*) */
#define PLX_PROF_PACK 1    /* pack_kernel (plx_pack_indices) */
#define PLX_PROF_UNPACK 2  /* unpack_kernel (plx_unpack_indices) */
#define PLX_PROF_DEQUANT 3 /* dequant_kernel (plx_dequant_f16) */
#define PLX_PROF_ADAM 4    /* adam_h24_kernel (plx_pollux_step_h24*) */
#define PLX_PROF_T3 5      /* t3_kernel (the structured type-3 scorer of NN-B) */
#define PLX_PROF_T12 6     /* t12_kernel (the structured type-1/2 scorer of NN-B) */
int plx_profile_select(int kernel);
int plx_profile_begin(void);
int plx_profile_end(double *total_ms, int64_t *launches);

#ifdef __cplusplus
}
#endif
#endif /* POLLUX_AMD_H */

// extern "C" entry points: argument validation, error reporting, dispatch to
// the kernel launchers.  Validation mirrors the reference's own checks so the
// Python host layer can raise the same exception types (ValueError for shapes,
// castor.py:272-295,311-312; RuntimeError for runtime failures).

#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "plx_internal.h"

namespace plx {
namespace {
thread_local std::string g_last_error;
}

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_hip(hipError_t e, const char *what) {
  if (e == hipSuccess) return PLX_OK;
  return fail(PLX_EHIP, "%s: %s", what, hipGetErrorString(e));
}

int check_launch(const char *what) { return check_hip(hipGetLastError(), what); }

}  // namespace plx

using namespace plx;

#define PLX_REQUIRE(cond, ...) \
  do {                         \
    if (!(cond)) return fail(PLX_EINVAL, __VA_ARGS__); \
  } while (0)

static inline hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

// A quantizer mode (NN-B, NN-T, and NN-P where the entry point scores raw atoms), with the dense
// type-3 flag allowed on NN-B only.
static inline bool nn_mode_ok(int mode, bool allow_pack) {
  const int base = mode & ~(PLX_NN_DENSE_TYPE3 | PLX_NN_T3_ROWS_BY_SWEEP);
  if (mode != base && base != PLX_NN_BF16_SCORES) return false;
  return base == PLX_NN_BF16_SCORES || base == PLX_NN_FP32_SCORES || (allow_pack && base == PLX_NN_PACK_FP32);
}

extern "C" {

const char *plx_last_error(void) { return g_last_error.c_str(); }

int plx_version(void) { return 1; }

int plx_codebook_raw(int8_t *out, int64_t n_bytes) {
  PLX_REQUIRE(out != nullptr, "plx_codebook_raw: null output");
  PLX_REQUIRE(n_bytes == static_cast<int64_t>(kCodebook) * kDim, "plx_codebook_raw: need %d bytes, got %lld",
              kCodebook * kDim, static_cast<long long>(n_bytes));
  const int8_t *raw = codebook_raw_host();
  if (!raw) return fail(PLX_EINVAL, "codebook generator produced a wrong row count");
  std::memcpy(out, raw, static_cast<size_t>(n_bytes));
  return PLX_OK;
}

int plx_codebook_f32(float *out, int64_t n_floats) {
  PLX_REQUIRE(out != nullptr, "plx_codebook_f32: null output");
  PLX_REQUIRE(n_floats == static_cast<int64_t>(kCodebook) * kDim, "plx_codebook_f32: need %d floats, got %lld",
              kCodebook * kDim, static_cast<long long>(n_floats));
  const int8_t *raw = codebook_raw_host();
  if (!raw) return fail(PLX_EINVAL, "codebook generator produced a wrong row count");
  float val[9];
  for (int k = -4; k <= 4; ++k) val[k + 4] = raw_to_f32(k);
  for (int64_t i = 0; i < n_floats; ++i) out[i] = val[raw[i] + 4];
  return PLX_OK;
}

int plx_codebook_fingerprint(float *out16) {
  PLX_REQUIRE(out16 != nullptr, "plx_codebook_fingerprint: null output");
  const int8_t *raw = codebook_raw_host();
  if (!raw) return fail(PLX_EINVAL, "codebook generator produced a wrong row count");
  for (int r = 0; r < 4; ++r)
    for (int c = 0; c < 4; ++c) out16[r * 4 + c] = raw_to_f32(raw[r * kDim + c]);
  return PLX_OK;
}

int plx_device_init(void) {
  const DeviceTables *t = nullptr;
  const int st = get_tables(&t);
  if (st != PLX_OK) return st;
  return noalloc_setup();
}

int plx_pack_indices(const void *indices, int idx_is_i64, int64_t n, uint8_t *out, void *stream) {
  PLX_REQUIRE(n >= 0, "plx_pack_indices: negative count %lld", static_cast<long long>(n));
  if (n == 0) return PLX_OK;
  PLX_REQUIRE(indices != nullptr && out != nullptr, "plx_pack_indices: null pointer");
  return launch_pack(indices, idx_is_i64, n, out, as_stream(stream));
}

int plx_unpack_indices(const uint8_t *packed, int64_t n_packed_bytes, int64_t num_indices, int64_t *out,
                       void *stream) {
  PLX_REQUIRE(n_packed_bytes >= 0 && n_packed_bytes % 9 == 0,
              "plx_unpack_indices: packed length %lld is not a multiple of 9", static_cast<long long>(n_packed_bytes));
  PLX_REQUIRE(num_indices >= 0 && num_indices <= (n_packed_bytes / 9) * 4,
              "plx_unpack_indices: num_indices %lld exceeds the %lld indices held by %lld bytes",
              static_cast<long long>(num_indices), static_cast<long long>((n_packed_bytes / 9) * 4),
              static_cast<long long>(n_packed_bytes));
  if (num_indices == 0) return PLX_OK;
  PLX_REQUIRE(packed != nullptr && out != nullptr, "plx_unpack_indices: null pointer");
  return launch_unpack(packed, num_indices, out, as_stream(stream));
}

int plx_row_rms(const float *w, int64_t rows, int64_t cols, float *sigma, void *stream) {
  PLX_REQUIRE(rows >= 0 && cols > 0, "plx_row_rms: bad shape (%lld, %lld)", static_cast<long long>(rows),
              static_cast<long long>(cols));
  if (rows == 0) return PLX_OK;
  PLX_REQUIRE(w != nullptr && sigma != nullptr, "plx_row_rms: null pointer");
  return launch_row_rms(w, rows, cols, sigma, nullptr, as_stream(stream));
}

int plx_sigma16_pack(const float *w, int64_t rows, int64_t cols, uint16_t *sigma16, void *stream) {
  PLX_REQUIRE(rows >= 0 && cols > 0, "plx_sigma16_pack: bad shape (%lld, %lld)", static_cast<long long>(rows),
              static_cast<long long>(cols));
  if (rows == 0) return PLX_OK;
  PLX_REQUIRE(w != nullptr && sigma16 != nullptr, "plx_sigma16_pack: null pointer");
  return launch_row_rms(w, rows, cols, nullptr, sigma16, as_stream(stream));
}

size_t plx_quantize_workspace_bytes(int64_t n_atoms) { return quantize_workspace_bytes(n_atoms < 0 ? 0 : n_atoms); }

int plx_quantize(const float *x, int64_t n_atoms, int mode, int32_t *idx_out, void *workspace,
                 size_t workspace_bytes, void *stream) {
  PLX_REQUIRE(n_atoms >= 0, "plx_quantize: negative atom count");
  PLX_REQUIRE(nn_mode_ok(mode, true),
              "plx_quantize: unknown mode %d", mode);
  if (n_atoms == 0) return PLX_OK;
  PLX_REQUIRE(x != nullptr && idx_out != nullptr, "plx_quantize: null pointer");
  return launch_quantize(x, nullptr, n_atoms, kDim, n_atoms, mode, idx_out, nullptr, nullptr, workspace,
                         workspace_bytes, as_stream(stream));
}

int plx_gather_codebook(const int32_t *idx, int64_t n, int out_dtype, void *out, void *stream) {
  PLX_REQUIRE(n >= 0, "plx_gather_codebook: negative count");
  PLX_REQUIRE(out_dtype == PLX_DTYPE_F32 || out_dtype == PLX_DTYPE_F16 || out_dtype == PLX_DTYPE_BF16,
              "plx_gather_codebook: unknown dtype %d", out_dtype);
  if (n == 0) return PLX_OK;
  PLX_REQUIRE(idx != nullptr && out != nullptr, "plx_gather_codebook: null pointer");
  PLX_REQUIRE((reinterpret_cast<uintptr_t>(out) & (out_dtype == PLX_DTYPE_F32 ? 15u : 7u)) == 0,
              "plx_gather_codebook: output is not aligned");
  return launch_gather(idx, n, out_dtype, out, as_stream(stream));
}

int plx_requantize(const float *latent, int64_t rows, int64_t cols, int mode, float *sigma_out, int32_t *idx_out,
                   uint8_t *packed_out, float *weight_out, void *workspace, size_t workspace_bytes, void *stream) {
  PLX_REQUIRE(rows >= 0 && cols > 0, "plx_requantize: bad shape (%lld, %lld)", static_cast<long long>(rows),
              static_cast<long long>(cols));
  PLX_REQUIRE(cols % kDim == 0, "Pollux requires in_features divisible by H24_DIM=24; got %lld.",
              static_cast<long long>(cols));
  PLX_REQUIRE(nn_mode_ok(mode, false), "plx_requantize: unknown mode %d", mode);
  if (rows == 0) return PLX_OK;
  PLX_REQUIRE(latent != nullptr && sigma_out != nullptr && idx_out != nullptr, "plx_requantize: null pointer");
  const int64_t n_atoms = rows * (cols / kDim);
  int st = check_quantize_args(latent, n_atoms, workspace, workspace_bytes);  // before anything is written
  if (st != PLX_OK) return st;
  const DeviceTables *tab = nullptr;
  if ((st = get_tables(&tab)) != PLX_OK) return st;
  st = launch_row_rms(latent, rows, cols, sigma_out, nullptr, as_stream(stream));
  if (st != PLX_OK) return st;
  return launch_quantize(latent, sigma_out, rows, cols, n_atoms, mode, idx_out, packed_out, weight_out, workspace,
                         workspace_bytes, as_stream(stream));
}

int plx_requantize_noalloc(const float *latent, int64_t rows, int64_t cols, int mode, float *sigma_out,
                           int32_t *idx_out, uint8_t *packed_out, float *weight_out, void *stream) {
  PLX_REQUIRE(rows >= 0 && cols > 0, "plx_requantize_noalloc: bad shape (%lld, %lld)", static_cast<long long>(rows),
              static_cast<long long>(cols));
  PLX_REQUIRE(cols % kDim == 0, "Pollux requires in_features divisible by H24_DIM=24; got %lld.",
              static_cast<long long>(cols));
  PLX_REQUIRE(nn_mode_ok(mode, false), "plx_requantize_noalloc: unknown mode %d",
              mode);
  PLX_REQUIRE(rows <= static_cast<int64_t>(PLX_NOALLOC_MAX_ATOMS) * kDim / cols,
              "plx_requantize_noalloc: %lld x %lld is more than its maximum of %d atoms (use plx_requantize)",
              static_cast<long long>(rows), static_cast<long long>(cols), PLX_NOALLOC_MAX_ATOMS);
  if (rows == 0) return PLX_OK;
  PLX_REQUIRE(latent != nullptr && sigma_out != nullptr && idx_out != nullptr, "plx_requantize_noalloc: null pointer");
  return launch_requantize_noalloc(latent, rows, cols, mode, sigma_out, idx_out, packed_out, weight_out,
                                   as_stream(stream));
}

int plx_requantize_batch(const plx_requantize_item *items, int n_items, int mode, void *workspace,
                         size_t workspace_bytes, void *stream) {
  PLX_REQUIRE(n_items >= 0 && n_items <= 4096, "plx_requantize_batch: bad item count %d", n_items);
  PLX_REQUIRE(nn_mode_ok(mode, false), "plx_requantize_batch: unknown mode %d", mode);
  if (n_items == 0) return PLX_OK;
  PLX_REQUIRE(items != nullptr, "plx_requantize_batch: null item array");
  std::vector<RequantItem> its(static_cast<size_t>(n_items));
  for (int i = 0; i < n_items; ++i) {
    const plx_requantize_item &x = items[i];
    PLX_REQUIRE(x.rows >= 0 && x.cols > 0, "plx_requantize_batch: item %d has a bad shape (%lld, %lld)", i,
                static_cast<long long>(x.rows), static_cast<long long>(x.cols));
    PLX_REQUIRE(x.cols % kDim == 0, "Pollux requires in_features divisible by H24_DIM=24; got %lld (item %d).",
                static_cast<long long>(x.cols), i);
    PLX_REQUIRE(x.rows == 0 || (x.latent != nullptr && x.sigma_out != nullptr && x.idx_out != nullptr),
                "plx_requantize_batch: item %d has a null pointer", i);
    its[static_cast<size_t>(i)] = RequantItem{x.latent, x.rows, x.cols, x.sigma_out, x.idx_out, x.packed_out, x.weight_out};
  }
  return launch_requantize_batch(its.data(), n_items, mode, workspace, workspace_bytes, as_stream(stream));
}

size_t plx_pollux_step_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0 || cols % kDim != 0) return 0;
  const int64_t n_atoms = rows * (cols / kDim);
  return ((quantize_workspace_bytes(n_atoms) + 255) & ~static_cast<size_t>(255)) + adam_h24_workspace_bytes(n_atoms);
}

int plx_pollux_step_h24(const float *grad, float *m, float *v, float *latent, int64_t rows, int64_t cols,
                        const float *scalars, int mode, float *sigma_out, int32_t *idx_out, uint8_t *packed_out,
                        float *weight_out, float *adam_norm_out, void *workspace, size_t workspace_bytes, void *stream) {
  PLX_REQUIRE(rows >= 0 && cols > 0, "plx_pollux_step_h24: bad shape (%lld, %lld)", static_cast<long long>(rows),
              static_cast<long long>(cols));
  PLX_REQUIRE(cols % kDim == 0, "Pollux requires in_features divisible by H24_DIM=24; got %lld.",
              static_cast<long long>(cols));
  PLX_REQUIRE(nn_mode_ok(mode, false), "plx_pollux_step_h24: unknown mode %d", mode);
  if (rows == 0) return PLX_OK;
  PLX_REQUIRE(grad != nullptr && m != nullptr && v != nullptr && latent != nullptr && scalars != nullptr &&
                  sigma_out != nullptr && idx_out != nullptr,
              "plx_pollux_step_h24: null pointer");
  const size_t need = plx_pollux_step_workspace_bytes(rows, cols);
  PLX_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "plx_pollux_step_h24: workspace of %zu bytes is smaller than the %zu needed", workspace_bytes, need);
  const int64_t n_atoms = rows * (cols / kDim);
  const size_t qws = (quantize_workspace_bytes(n_atoms) + 255) & ~static_cast<size_t>(255);
  int st = check_quantize_args(latent, n_atoms, workspace, qws);  // before anything is written
  if (st != PLX_OK) return st;
  const DeviceTables *tab = nullptr;
  if ((st = get_tables(&tab)) != PLX_OK) return st;
  st = launch_adam_h24(grad, m, v, latent, n_atoms, scalars, adam_norm_out, static_cast<uint8_t *>(workspace) + qws,
                           as_stream(stream));
  if (st != PLX_OK) return st;
  st = launch_row_rms(latent, rows, cols, sigma_out, nullptr, as_stream(stream));
  if (st != PLX_OK) return st;
  return launch_quantize(latent, sigma_out, rows, cols, n_atoms, mode, idx_out, packed_out, weight_out, workspace, qws,
                         as_stream(stream));
}

size_t plx_pollux_step_batch_workspace_bytes(const plx_pollux_step_item *items, int n_items) {
  if (items == nullptr || n_items <= 0) return 0;
  int64_t total = 0;
  size_t adam = 0;
  for (int i = 0; i < n_items; ++i) {
    const plx_pollux_step_item &x = items[i];
    if (x.rows < 0 || x.cols <= 0 || x.cols % kDim != 0) return 0;
    const int64_t n = x.rows * (x.cols / kDim);
    total += n;
    adam += (adam_h24_workspace_bytes(n) + 255) & ~static_cast<size_t>(255);
  }
  return ((quantize_workspace_bytes(total) + 255) & ~static_cast<size_t>(255)) + adam;
}

int plx_pollux_step_h24_batch(const plx_pollux_step_item *items, int n_items, const float *scalars, int mode,
                              void *workspace, size_t workspace_bytes, void *stream) {
  PLX_REQUIRE(n_items >= 0 && n_items <= 4096, "plx_pollux_step_h24_batch: bad item count %d", n_items);
  PLX_REQUIRE(nn_mode_ok(mode, false), "plx_pollux_step_h24_batch: unknown mode %d",
              mode);
  if (n_items == 0) return PLX_OK;
  PLX_REQUIRE(items != nullptr && scalars != nullptr, "plx_pollux_step_h24_batch: null item array or scalars");
  // every check before the first launch: a refused call writes nothing
  int64_t total = 0;
  for (int i = 0; i < n_items; ++i) {
    const plx_pollux_step_item &x = items[i];
    PLX_REQUIRE(x.rows >= 0 && x.cols > 0, "plx_pollux_step_h24_batch: item %d has a bad shape (%lld, %lld)", i,
                static_cast<long long>(x.rows), static_cast<long long>(x.cols));
    PLX_REQUIRE(x.cols % kDim == 0, "Pollux requires in_features divisible by H24_DIM=24; got %lld (item %d).",
                static_cast<long long>(x.cols), i);
    if (x.rows == 0) continue;
    PLX_REQUIRE(x.grad != nullptr && x.m != nullptr && x.v != nullptr && x.latent != nullptr &&
                    x.sigma_out != nullptr && x.idx_out != nullptr,
                "plx_pollux_step_h24_batch: item %d has a null pointer", i);
    const uintptr_t al = reinterpret_cast<uintptr_t>(x.grad) | reinterpret_cast<uintptr_t>(x.m) |
                         reinterpret_cast<uintptr_t>(x.v) | reinterpret_cast<uintptr_t>(x.latent);
    PLX_REQUIRE((al & 15u) == 0, "plx_pollux_step_h24_batch: item %d: grad, m, v and latent must be 16-byte aligned",
                i);
    total += x.rows * (x.cols / kDim);
  }
  if (total == 0) return PLX_OK;
  const size_t need = plx_pollux_step_batch_workspace_bytes(items, n_items);
  PLX_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "plx_pollux_step_h24_batch: workspace of %zu bytes is smaller than the %zu needed", workspace_bytes, need);
  const size_t qws = (quantize_workspace_bytes(total) + 255) & ~static_cast<size_t>(255);
  int st = check_quantize_args(items[0].latent, total, workspace, qws);
  if (st != PLX_OK) return st;
  const DeviceTables *tab = nullptr;
  if ((st = get_tables(&tab)) != PLX_OK) return st;
  hipStream_t s = as_stream(stream);
  uint8_t *adam_ws = static_cast<uint8_t *>(workspace) + qws;
  std::vector<RequantItem> its;
  its.reserve(static_cast<size_t>(n_items));
  for (int i = 0; i < n_items; ++i) {
    const plx_pollux_step_item &x = items[i];
    if (x.rows == 0) continue;
    const int64_t n = x.rows * (x.cols / kDim);
    st = launch_adam_h24(x.grad, x.m, x.v, x.latent, n, scalars, x.adam_norm_out, adam_ws, s);
    if (st != PLX_OK) return st;
    adam_ws += (adam_h24_workspace_bytes(n) + 255) & ~static_cast<size_t>(255);
    its.push_back(RequantItem{x.latent, x.rows, x.cols, x.sigma_out, x.idx_out, x.packed_out, x.weight_out});
  }
  return launch_requantize_batch(its.data(), static_cast<int>(its.size()), mode, workspace, qws, s);
}

int plx_quantize_layer_pack(const float *w, int64_t rows, int64_t cols, uint8_t *packed_out, uint16_t *sigma16_out,
                            int32_t *idx_out, void *workspace, size_t workspace_bytes, void *stream) {
  PLX_REQUIRE(rows >= 0 && cols > 0, "plx_quantize_layer_pack: bad shape (%lld, %lld)", static_cast<long long>(rows),
              static_cast<long long>(cols));
  PLX_REQUIRE(cols % kDim == 0, "Pollux requires in_features divisible by H24_DIM=24; got %lld.",
              static_cast<long long>(cols));
  if (rows == 0) return PLX_OK;
  PLX_REQUIRE(w != nullptr && packed_out != nullptr && sigma16_out != nullptr, "plx_quantize_layer_pack: null pointer");
  const int64_t n_atoms = rows * (cols / kDim);
  int st = check_quantize_args(w, n_atoms, workspace, workspace_bytes);  // before anything is written
  if (st != PLX_OK) return st;
  const DeviceTables *tab = nullptr;
  if ((st = get_tables(&tab)) != PLX_OK) return st;
  st = launch_row_rms(w, rows, cols, nullptr, sigma16_out, as_stream(stream));
  if (st != PLX_OK) return st;
  return launch_quantize(w, nullptr, rows, cols, n_atoms, PLX_NN_PACK_FP32, idx_out, packed_out, nullptr, workspace,
                         workspace_bytes, as_stream(stream));
}

int plx_dequant_f16(const uint8_t *packed, int64_t n_packed_bytes, const uint16_t *sigma16, int64_t rows,
                    int64_t cols, uint16_t *w16_out, void *stream) {
  PLX_REQUIRE(rows >= 0 && cols > 0 && cols % kDim == 0, "plx_dequant_f16: bad shape (%lld, %lld)",
              static_cast<long long>(rows), static_cast<long long>(cols));
  const int64_t n_atoms = rows * (cols / kDim);
  PLX_REQUIRE(n_packed_bytes == ((n_atoms + 3) / 4) * 9,
              "plx_dequant_f16: packed length %lld does not match %lld atoms (need %lld)",
              static_cast<long long>(n_packed_bytes), static_cast<long long>(n_atoms),
              static_cast<long long>(((n_atoms + 3) / 4) * 9));
  if (rows == 0) return PLX_OK;
  PLX_REQUIRE(packed != nullptr && sigma16 != nullptr && w16_out != nullptr, "plx_dequant_f16: null pointer");
  return launch_dequant_f16(packed, sigma16, rows, cols, w16_out, as_stream(stream));
}

static_assert(sizeof(plx_dql_target) == sizeof(DqlTarget), "plx_dql_target mirrors DqlTarget");

size_t plx_dequant_linear_multi_workspace_bytes(const plx_dql_target *targets, int n, int64_t cols, int64_t m_rows,
                                                int flags) {
  if (targets == nullptr || n < 1 || n > 16 || cols <= 0 || cols % kDim != 0 || m_rows <= 0) return 0;
  int64_t rows[16];
  for (int i = 0; i < n; ++i) rows[i] = targets[i].rows;
  return dequant_linear_workspace_bytes_multi(rows, n, cols, m_rows, flags);
}

int plx_dequant_linear_multi(const plx_dql_target *targets, int n, int64_t cols, const void *x, int flags,
                             int64_t m_rows, const float *norm_weight, float norm_eps, void *workspace,
                             size_t workspace_bytes, void *stream) {
  PLX_REQUIRE(targets != nullptr && n >= 1 && n <= 16, "plx_dequant_linear_multi: %d targets (1..16)", n);
  PLX_REQUIRE(cols > 0 && cols % kDim == 0, "plx_dequant_linear_multi: bad column count %lld",
              static_cast<long long>(cols));
  PLX_REQUIRE(m_rows >= 0, "plx_dequant_linear_multi: negative batch");
  PLX_REQUIRE((flags & ~(PLX_DQL_X_F32 | PLX_DQL_W_AS_X | PLX_DQL_GELU | PLX_DQL_RMS_NORM | PLX_DQL_PLANES)) == 0,
              "plx_dequant_linear_multi: unknown flags 0x%x", flags);
  PLX_REQUIRE(!(flags & PLX_DQL_PLANES) || m_rows <= 1 || m_rows > 4,
              "plx_dequant_linear_multi: the plane layout takes one token or more than 4 (got %lld)",
              static_cast<long long>(m_rows));
  PLX_REQUIRE(((flags & PLX_DQL_RMS_NORM) != 0) == (norm_weight != nullptr),
              "plx_dequant_linear_multi: PLX_DQL_RMS_NORM needs a norm weight, and a norm weight the flag");
  PLX_REQUIRE(!(flags & PLX_DQL_RMS_NORM) || (flags & PLX_DQL_X_F32),
              "plx_dequant_linear_multi: PLX_DQL_RMS_NORM takes fp32 x");
  DqlTarget t[16];
  int live = 0;
  for (int i = 0; i < n; ++i) {
    PLX_REQUIRE(targets[i].rows >= 0, "plx_dequant_linear_multi: negative rows in target %d", i);
    if (targets[i].rows == 0) continue;
    PLX_REQUIRE(targets[i].packed && targets[i].sigma16 && targets[i].y, "plx_dequant_linear_multi: null pointer in target %d",
                i);
    t[live++] = DqlTarget{targets[i].packed, targets[i].sigma16, targets[i].rows, targets[i].y, targets[i].residual};
  }
  if (live == 0 || m_rows == 0) return PLX_OK;
  PLX_REQUIRE(x != nullptr, "plx_dequant_linear_multi: null x");
  return launch_dequant_linear_multi(t, live, cols, x, flags, m_rows, norm_weight, norm_eps, workspace, workspace_bytes,
                                     as_stream(stream));
}

int plx_rms_norm(const float *x, const float *w, float *y, int64_t rows, int64_t d, float eps, void *stream) {
  PLX_REQUIRE(rows >= 0 && d > 0, "plx_rms_norm: bad shape (%lld, %lld)", static_cast<long long>(rows),
              static_cast<long long>(d));
  if (rows == 0) return PLX_OK;
  PLX_REQUIRE(x != nullptr && w != nullptr && y != nullptr, "plx_rms_norm: null pointer");
  return launch_rms_norm(x, w, y, rows, d, eps, as_stream(stream));
}

int plx_argmax_rows(const float *x, int64_t rows, int64_t cols, int64_t *out, void *stream) {
  PLX_REQUIRE(rows >= 0 && cols > 0, "plx_argmax_rows: bad shape (%lld, %lld)", static_cast<long long>(rows),
              static_cast<long long>(cols));
  if (rows == 0) return PLX_OK;
  PLX_REQUIRE(x != nullptr && out != nullptr, "plx_argmax_rows: null pointer");
  return launch_argmax_rows(x, rows, cols, out, as_stream(stream));
}

int plx_decode_attention(const float *q, const float *k, const float *v, int64_t qkv_stride, const float *q_norm_w,
                         const float *k_norm_w, float eps, float *k_cache, float *v_cache, const int64_t *pos,
                         int64_t n, int64_t heads, int64_t max_len, float *out, void *stream) {
  PLX_REQUIRE(n >= 0 && qkv_stride >= 0, "plx_decode_attention: negative head count or stride");
  if (n == 0) return PLX_OK;
  PLX_REQUIRE(q && k && v && q_norm_w && k_norm_w && k_cache && v_cache && pos && out,
              "plx_decode_attention: null pointer");
  return launch_decode_attention(q, k, v, qkv_stride, heads, q_norm_w, k_norm_w, eps, k_cache, v_cache, pos, n,
                                 max_len, out, as_stream(stream));
}

int plx_prefill_attention(const float *q, const float *k, const float *v, int64_t qkv_stride, const float *q_norm_w,
                          const float *k_norm_w, float eps, float *k_cache, float *v_cache, int64_t b, int64_t heads,
                          int64_t t, int64_t p0, int64_t max_len, float *out, void *stream) {
  PLX_REQUIRE(qkv_stride >= 0, "plx_prefill_attention: negative stride");
  PLX_REQUIRE(b >= 0 && heads >= 0 && t >= 0, "plx_prefill_attention: negative shape (%lld, %lld, %lld)",
              static_cast<long long>(b), static_cast<long long>(t), static_cast<long long>(heads));
  if (b == 0 || heads == 0 || t == 0) return PLX_OK;
  PLX_REQUIRE(q && k && v && q_norm_w && k_norm_w && k_cache && v_cache && out, "plx_prefill_attention: null pointer");
  return launch_prefill_attention(q, k, v, qkv_stride, q_norm_w, k_norm_w, eps, k_cache, v_cache, b, heads, t, p0,
                                  max_len, out, as_stream(stream));
}

size_t plx_dequant_linear_workspace_bytes(int64_t rows, int64_t cols, int64_t m_rows, int flags) {
  if (rows <= 0 || cols <= 0 || cols % kDim != 0 || m_rows <= 0) return 0;
  return dequant_linear_workspace_bytes(rows, cols, m_rows, flags);
}

int plx_dequant_linear(const uint8_t *packed, int64_t n_packed_bytes, const uint16_t *sigma16, int64_t rows,
                       int64_t cols, const void *x, int flags, int64_t m_rows, float *y, void *workspace,
                       size_t workspace_bytes, void *stream) {
  PLX_REQUIRE(rows >= 0 && cols > 0 && cols % kDim == 0, "plx_dequant_linear: bad shape (%lld, %lld)",
              static_cast<long long>(rows), static_cast<long long>(cols));
  PLX_REQUIRE(m_rows >= 0, "plx_dequant_linear: negative batch");
  PLX_REQUIRE((flags & ~(PLX_DQL_X_F32 | PLX_DQL_W_AS_X | PLX_DQL_GELU | PLX_DQL_PLANES)) == 0,
              "plx_dequant_linear: unknown flags 0x%x", flags);
  const int64_t n_atoms = rows * (cols / kDim);
  if (flags & PLX_DQL_PLANES) {
    PLX_REQUIRE(n_packed_bytes == 6 * n_atoms, "plx_dequant_linear: plane layout of %lld bytes does not match %lld atoms",
                static_cast<long long>(n_packed_bytes), static_cast<long long>(n_atoms));
    PLX_REQUIRE(m_rows > 4 || m_rows <= 1,
                "plx_dequant_linear: the plane layout takes one token or more than 4 (got %lld)",
                static_cast<long long>(m_rows));
  } else {
    PLX_REQUIRE(n_packed_bytes == ((n_atoms + 3) / 4) * 9,
                "plx_dequant_linear: packed length %lld does not match %lld atoms",
                static_cast<long long>(n_packed_bytes), static_cast<long long>(n_atoms));
  }
  if (rows == 0 || m_rows == 0) return PLX_OK;
  PLX_REQUIRE(packed != nullptr && sigma16 != nullptr && x != nullptr && y != nullptr, "plx_dequant_linear: null pointer");
  return launch_dequant_linear(packed, sigma16, rows, cols, x, flags, m_rows, y, workspace, workspace_bytes,
                               as_stream(stream));
}

int plx_h24_plane_layout(const uint8_t *packed, int64_t n_packed_bytes, int64_t n_atoms, uint16_t *planes,
                         void *stream) {
  PLX_REQUIRE(n_atoms >= 0, "plx_h24_plane_layout: negative atom count");
  PLX_REQUIRE(n_packed_bytes == ((n_atoms + 3) / 4) * 9, "plx_h24_plane_layout: packed length %lld does not match %lld atoms",
              static_cast<long long>(n_packed_bytes), static_cast<long long>(n_atoms));
  if (n_atoms == 0) return PLX_OK;
  PLX_REQUIRE(packed != nullptr && planes != nullptr, "plx_h24_plane_layout: null pointer");
  return launch_plane_layout(packed, n_atoms, planes, as_stream(stream));
}

int64_t plx_plane_table(uint32_t *ids, int64_t capacity) {
  const PlaneTables *pt = plane_tables_host();
  if (!pt) return fail(PLX_EINVAL, "plane table construction failed");
  const int64_t n = static_cast<int64_t>(pt->ids.size());
  if (ids && capacity > 0) std::memcpy(ids, pt->ids.data(), static_cast<size_t>(std::min(n, capacity)) * 4);
  return n;
}

int plx_int8_linear(const int8_t *q, const uint16_t *mu16, int64_t rows, int64_t cols, const float *x, int64_t m_rows,
                    const float *norm_weight, float norm_eps, float *y, void *stream) {
  PLX_REQUIRE(rows >= 0 && cols > 0 && m_rows >= 0, "plx_int8_linear: bad shape (%lld, %lld) x %lld tokens",
              static_cast<long long>(rows), static_cast<long long>(cols), static_cast<long long>(m_rows));
  if (rows == 0 || m_rows == 0) return PLX_OK;
  PLX_REQUIRE(q != nullptr && mu16 != nullptr && x != nullptr && y != nullptr, "plx_int8_linear: null pointer");
  return launch_int8_linear(q, mu16, rows, cols, x, m_rows, norm_weight, norm_eps, y, nullptr, as_stream(stream));
}

size_t plx_int8_linear_argmax_workspace_bytes(int64_t rows, int64_t m_rows) {
  return int8_linear_argmax_workspace_bytes(rows, m_rows);
}

int plx_int8_linear_argmax(const int8_t *q, const uint16_t *mu16, int64_t rows, int64_t cols, const float *x,
                           int64_t m_rows, const float *norm_weight, float norm_eps, float *y, int64_t *ids,
                           int64_t *history, int64_t hist_len, int64_t *pos, void *workspace, size_t workspace_bytes,
                           void *stream) {
  PLX_REQUIRE(rows > 0 && cols > 0 && m_rows >= 0 && hist_len >= 0,
              "plx_int8_linear_argmax: bad shape (%lld, %lld) x %lld tokens", static_cast<long long>(rows),
              static_cast<long long>(cols), static_cast<long long>(m_rows));
  if (m_rows == 0) return PLX_OK;
  PLX_REQUIRE(q != nullptr && mu16 != nullptr && x != nullptr && y != nullptr && ids != nullptr,
              "plx_int8_linear_argmax: null pointer");
  PLX_REQUIRE(history == nullptr || pos != nullptr, "plx_int8_linear_argmax: a history needs the position");
  return launch_int8_linear_argmax(q, mu16, rows, cols, x, m_rows, norm_weight, norm_eps, y, ids, history, hist_len,
                                   pos, workspace, workspace_bytes, as_stream(stream));
}

int plx_int8_embed(const int8_t *q, const uint16_t *mu16, int64_t vocab, int64_t cols, const int64_t *ids,
                   int64_t batch, int64_t t, const float *pos_weight, int64_t pos_rows, const int64_t *pos0, float *out,
                   void *stream) {
  PLX_REQUIRE(vocab >= 0 && cols > 0 && batch >= 0 && t >= 0 && pos_rows >= 0, "plx_int8_embed: bad shape");
  if (batch == 0 || t == 0) return PLX_OK;
  PLX_REQUIRE(q != nullptr && mu16 != nullptr && ids != nullptr && out != nullptr, "plx_int8_embed: null pointer");
  return launch_int8_embed(q, mu16, vocab, cols, ids, batch * t, t, pos_weight, pos_rows, pos0, out, as_stream(stream));
}

int plx_quantize_int8_rows(const float *w, int64_t rows, int64_t cols, int8_t *q_out, uint16_t *mu16_out,
                           void *stream) {
  PLX_REQUIRE(rows >= 0 && cols > 0, "plx_quantize_int8_rows: bad shape (%lld, %lld)", static_cast<long long>(rows),
              static_cast<long long>(cols));
  if (rows == 0) return PLX_OK;
  PLX_REQUIRE(w != nullptr && q_out != nullptr && mu16_out != nullptr, "plx_quantize_int8_rows: null pointer");
  return launch_int8_quant(w, rows, cols, q_out, mu16_out, as_stream(stream));
}

int plx_dequant_int8_rows(const int8_t *q, const uint16_t *mu16, int64_t rows, int64_t cols, uint16_t *w16_out,
                          void *stream) {
  PLX_REQUIRE(rows >= 0 && cols > 0, "plx_dequant_int8_rows: bad shape (%lld, %lld)", static_cast<long long>(rows),
              static_cast<long long>(cols));
  if (rows == 0) return PLX_OK;
  PLX_REQUIRE(q != nullptr && mu16 != nullptr && w16_out != nullptr, "plx_dequant_int8_rows: null pointer");
  return launch_int8_dequant(q, mu16, rows, cols, w16_out, as_stream(stream));
}

}  // extern "C"

// cmk_iq2.cpp — implementation of the C ABI declared in include/cmk_iq2.h.
//
// Host-side dispatch for the IQ2_XXS path: argument validation with the
// reference's error texts (src/iq2_matmul.rs:210-311, 367-433, 559-591), kernel
// selection by shape, and thin HIP runtime wrappers.  Nothing here allocates
// device memory on a launch path.
#include "cmk_iq2.h"

#include <hip/hip_runtime.h>

#include <cinttypes>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "iq2xxs_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return CMK_OK;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(CMK_ERR_HIP, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}

// bytes_per_block / scales_per_block (src/iq2_matmul.rs:13-29,39-57).
size_t bytes_per_block(int v) { return v == CMK_IQ2_XXS ? 64 : cmk::variant_bytes_per_block(v); }
size_t scales_per_block(int v) { return v == CMK_IQ2_XXS ? 2 : cmk::variant_scales_per_block(v); }

// Largest m served by the GEMV family (above it: the MFMA GEMM).  The GEMV
// multiplies exact weights (the GEMM rounds them to f16) and takes up to 16
// rows in one launch, which at 9-16 rows is also faster than the GEMM for
// f16 / bf16 x at the decode shapes (K=4096: 18.9-19.9 against 23.1-27.9 us at
// N=14336; K=8192, N=28672: 54 against 86 us), the one exception measured being
// N=4096 (16.1 against 13.2 us at 16 rows).
constexpr size_t kGemvMaxM = 16;
constexpr size_t kGemvMaxMF32 = 16;
// W8A8 activations are int8 on the multi-row kernel, 32 rows per launch: at
// 24 to 32 rows it is level in time with the GEMM (which rounds the weights
// to f16) and its sums are exact.
constexpr size_t kGemvMaxMW8A8 = 32;
constexpr size_t kWorkspaceAlign = 256;

bool checked_mul(size_t a, size_t b, size_t* out) {
  if (a != 0 && b > SIZE_MAX / a) return false;
  *out = a * b;
  return true;
}

struct Dims {
  uint32_t m, out_dim, in_dim, bpr;
};

// Per-device CU counts, read once.
std::mutex g_dev_mu;
int g_cu_count[64] = {0};

int current_cu_count(int* cus) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= 64) return fail(CMK_ERR_NO_DEVICE, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_dev_mu);
  if (g_cu_count[dev] == 0) {
    int n = 0;
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
    g_cu_count[dev] = n > 0 ? n : 1;
  }
  *cus = g_cu_count[dev];
  return CMK_OK;
}

// Path decision shared by the launch, the workspace query and the path query.
enum class Path { Gemv, Gemm, Simple, Variant };

// Null pointers stand for allocator-aligned buffers (queries made before the
// buffers exist).
Path choose_path(int x_dtype, size_t m, uint32_t out_dim, uint32_t in_dim, const void* x,
                 const void* wb, const void* ws, bool w8a8) {
  auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; };
  // f32 rows beyond the GEMV's range are staged as scaled f16 head / tail row
  // pairs for the GEMM (twice the rows).
  const size_t gemm_rows = x_dtype == CMK_F32 ? 2 * m : m;
  const size_t gemv_max_m =
      w8a8 ? kGemvMaxMW8A8 : (x_dtype == CMK_F32 ? kGemvMaxMF32 : kGemvMaxM);
  if (m > gemv_max_m && gemm_rows <= UINT32_MAX &&
      cmk::gemm_supported((uint32_t)gemm_rows, out_dim, in_dim) && al(x, 16) && al(wb, 16) &&
      al(ws, 2))
    return Path::Gemm;
  if (m <= UINT32_MAX && cmk::gemv_supported((uint32_t)m, out_dim, in_dim, x_dtype) &&
      al(wb, 16) && al(ws, 2))
    return Path::Gemv;
  return Path::Simple;
}

// Row scales first (256-byte aligned), then for the GEMM the quantised rows.
size_t row_scale_bytes(size_t m) {
  return ((m * sizeof(float) + kWorkspaceAlign - 1) / kWorkspaceAlign) * kWorkspaceAlign;
}

// Row scales and staged rows at the head of the workspace: the GEMM stages
// f32 rows (as head / tail pairs), bf16 rows (as scaled f16) and W8A8 rows;
// Simple and Variant need the W8A8 row scales only.
size_t workspace_head(Path p, bool w8a8, int x_dtype, size_t m, uint32_t in_dim) {
  if (p == Path::Gemm && x_dtype == CMK_F32)
    return row_scale_bytes(m) + cmk::gemm_f32_scratch_bytes((uint32_t)m, in_dim, w8a8);
  if (p == Path::Gemm && (w8a8 || x_dtype == CMK_BF16))  // (bf16 rows staged as f16)
    return row_scale_bytes(m) + cmk::gemm_w8a8_scratch_bytes((uint32_t)m, in_dim);
  if (!w8a8 || p == Path::Gemv) return 0;
  return row_scale_bytes(m);
}

// What a launch needs: the head, then for a GEMM split over k its partial
// products.
size_t workspace_required(Path p, bool w8a8, int x_dtype, size_t m, uint32_t out_dim,
                          uint32_t in_dim) {
  const size_t head = workspace_head(p, w8a8, x_dtype, m, in_dim);
  if (p != Path::Gemm) return head;
  const size_t rows = x_dtype == CMK_F32 && !w8a8 ? 2 * m : m;
  return head + cmk::gemm_split_scratch_bytes((uint32_t)rows, (uint32_t)m, out_dim, in_dim);
}

// The multi-row decode kernel splits K over several workgroups per row group
// when the row groups leave CUs idle (N <= 4096 on 256 CUs); the split is
// used when the workspace holds its bytes after the required ones (256-byte
// aligned) and skipped otherwise.  The query assumes 256 CUs, the most a
// gfx950 device has: fewer CUs never split more.
constexpr int kMaxCusForQuery = 256;
size_t split_offset(size_t required) {
  return (required + kWorkspaceAlign - 1) / kWorkspaceAlign * kWorkspaceAlign;
}
size_t rows_split_bytes(Path p, bool w8a8, size_t m, uint32_t out_dim, uint32_t in_dim,
                        int cus) {
  if ((p != Path::Gemv && p != Path::Variant) || m < 2 || m > UINT32_MAX) return 0;
  return cmk::gemv_rows_split_bytes((uint32_t)m, out_dim, in_dim, w8a8, cus);
}

// The workspace the query reports: the required bytes, then the split's.
size_t workspace_for(Path p, bool w8a8, int x_dtype, size_t m, uint32_t out_dim,
                     uint32_t in_dim) {
  const size_t req = workspace_required(p, w8a8, x_dtype, m, out_dim, in_dim);
  const size_t split = rows_split_bytes(p, w8a8, m, out_dim, in_dim, kMaxCusForQuery);
  return split ? split_offset(req) + split : req;
}

// Shared validation of cmk_iq2_matmul / cmk_iq2_matmul_workspace_size.
// Resolves the activation mode (W4A8 non-strict runs as OFF).
int validate_matmul(int x_dtype, size_t m, size_t out_dim, size_t in_dim, int variant, int* mode,
                    int strict, size_t wb_len, size_t ws_len, bool check_sizes, Dims* dims) {
  // iq2_matmul_with_activation_quant (src/iq2_matmul.rs:559-591)
  if (*mode == CMK_ACT_QUANT_W4A8) {
    if (strict)
      return fail(CMK_ERR_UNSUPPORTED,
                  "activation quant mode W4A8 requested in strict mode, but W4A8 kernel path is "
                  "not implemented yet");
    *mode = CMK_ACT_QUANT_OFF;
  }
  if (*mode != CMK_ACT_QUANT_OFF && *mode != CMK_ACT_QUANT_W8A8)
    return fail(CMK_ERR_INVALID_ARGUMENT, "invalid activation quant mode: %d", *mode);
  // iq2_matmul_metal guards (src/iq2_matmul.rs:210-311)
  if (out_dim == 0 || in_dim == 0)
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_matmul expects non-zero dimensions");
  if (variant < CMK_IQ2_XXS || variant > CMK_IQ3_S)
    return fail(CMK_ERR_INVALID_ARGUMENT, "invalid iq2 variant: %d", variant);
  if (x_dtype != CMK_F32 && x_dtype != CMK_F16 && x_dtype != CMK_BF16)
    return fail(CMK_ERR_INVALID_ARGUMENT,
                *mode == CMK_ACT_QUANT_W8A8 ? "iq2_matmul_w8a8 unsupported x dtype: %d"
                                            : "iq2_matmul unsupported x dtype: %d",
                x_dtype);
  const size_t bpr = (in_dim + 255) / 256;
  size_t blocks, expected_bytes, expected_scales;
  if (!checked_mul(out_dim, bpr, &blocks) ||
      !checked_mul(blocks, bytes_per_block(variant), &expected_bytes))
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_matmul bytes size overflow");
  if (!checked_mul(blocks, scales_per_block(variant), &expected_scales))
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_matmul scales size overflow");
  if (check_sizes) {
    if (wb_len < expected_bytes)
      return fail(CMK_ERR_INVALID_ARGUMENT,
                  "iq2_matmul weight_bytes too small: got %zu expected at least %zu", wb_len,
                  expected_bytes);
    if (ws_len < expected_scales)
      return fail(CMK_ERR_INVALID_ARGUMENT,
                  "iq2_matmul weight_scales too small: got %zu expected at least %zu", ws_len,
                  expected_scales);
  }
  size_t total;
  if (!checked_mul(m, out_dim, &total))
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_matmul output size overflow");
  if (m > UINT32_MAX) return fail(CMK_ERR_INVALID_ARGUMENT, "m too large");
  if (out_dim > UINT32_MAX) return fail(CMK_ERR_INVALID_ARGUMENT, "out_dim too large");
  if (in_dim > UINT32_MAX) return fail(CMK_ERR_INVALID_ARGUMENT, "in_dim too large");
  if (bpr > UINT32_MAX) return fail(CMK_ERR_INVALID_ARGUMENT, "blocks_per_row too large");
  dims->m = (uint32_t)m;
  dims->out_dim = (uint32_t)out_dim;
  dims->in_dim = (uint32_t)in_dim;
  dims->bpr = (uint32_t)bpr;
  return CMK_OK;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace

// ---------------------------------------------------------------------------
// Scratch of cmk_iq2_matmul_noalloc: one array per device, part of the code
// object, so it exists on every device the library runs on until the process
// ends.  In host code `scratch` only names the symbol; the device address of
// each device's copy comes from hipGetSymbolAddress, called once per device
// (with that device current) on the first call there, and is kept below.
static __device__ __align__(256) uint8_t scratch[CMK_IQ2_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

// Device address of the current device's scratch array.
int device_scratch(void** ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(CMK_ERR_NO_DEVICE, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(CMK_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address");
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return CMK_OK;
}

}  // namespace

extern "C" {

const char* cmk_last_error(void) { return g_last_error.c_str(); }

int cmk_abi_version(void) { return CMK_IQ2_ABI_VERSION; }

int cmk_iq2_matmul_workspace_size(cmk_dtype x_dtype, size_t m, size_t out_dim, size_t in_dim,
                                  cmk_iq2_variant variant, cmk_act_quant_mode mode,
                                  size_t* bytes) {
  if (!bytes) return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_matmul null pointer argument");
  int md = (int)mode;
  Dims dims;
  int rc = validate_matmul((int)x_dtype, m, out_dim, in_dim, (int)variant, &md, 0, 0, 0, false,
                           &dims);
  if (rc != CMK_OK) return rc;
  // Assume allocator-aligned buffers (hipMalloc gives 256-byte alignment).
  Path p = variant != CMK_IQ2_XXS
               ? Path::Variant
               : choose_path((int)x_dtype, m, dims.out_dim, dims.in_dim, nullptr, nullptr, nullptr,
                             md == CMK_ACT_QUANT_W8A8);
  // The simple path can still be chosen at launch for unaligned weights; report
  // the larger need so either choice is covered.
  size_t need =
      workspace_for(p, md == CMK_ACT_QUANT_W8A8, (int)x_dtype, m, dims.out_dim, dims.in_dim);
  size_t need_simple = workspace_for(Path::Simple, md == CMK_ACT_QUANT_W8A8, (int)x_dtype, m,
                                     dims.out_dim, dims.in_dim);
  *bytes = need > need_simple ? need : need_simple;
  return ok();
}

int cmk_iq2_matmul_path(cmk_dtype x_dtype, size_t m, size_t out_dim, size_t in_dim,
                        cmk_act_quant_mode mode) {
  return choose_path((int)x_dtype, m, (uint32_t)(out_dim > UINT32_MAX ? UINT32_MAX : out_dim),
                     (uint32_t)(in_dim > UINT32_MAX ? UINT32_MAX : in_dim), nullptr, nullptr,
                     nullptr, mode == CMK_ACT_QUANT_W8A8) == Path::Gemm
             ? 1
             : 0;
}

int cmk_iq2_matmul(const void* x, cmk_dtype x_dtype, size_t x_len, size_t m,
                   const uint8_t* weight_bytes, size_t weight_bytes_len,
                   const uint8_t* weight_scales, size_t weight_scales_len, size_t out_dim,
                   size_t in_dim, cmk_iq2_variant variant, cmk_act_quant_mode mode, int strict,
                   float* out, void* workspace, size_t workspace_bytes, void* stream) {
  int md = (int)mode;
  Dims dims;
  int rc = validate_matmul((int)x_dtype, m, out_dim, in_dim, (int)variant, &md, strict,
                           weight_bytes_len, weight_scales_len, true, &dims);
  if (rc != CMK_OK) return rc;
  if (m == 0) return ok();  // empty activation: nothing to compute (src/iq2_matmul.rs:265-267)
  size_t need_x;
  if (!checked_mul(m, in_dim, &need_x))
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_matmul x size overflow");
  if (x_len < need_x)
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_matmul x too small: got %zu expected at least %zu",
                x_len, need_x);
  if (!x || !weight_bytes || !weight_scales || !out)
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_matmul null pointer argument");
  const size_t esize = x_dtype == CMK_F32 ? 4 : 2;
  if (!aligned(x, esize))
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_matmul x must be aligned to its element size");
  if (!aligned(out, 4))
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_matmul out must be 4-byte aligned");

  const bool w8a8 = md == CMK_ACT_QUANT_W8A8;
  Path p = variant != CMK_IQ2_XXS ? Path::Variant
                                  : choose_path((int)x_dtype, m, dims.out_dim, dims.in_dim, x,
                                                weight_bytes, weight_scales, w8a8);
  const size_t need_ws =
      workspace_required(p, w8a8, (int)x_dtype, m, dims.out_dim, dims.in_dim);
  const size_t head_ws = workspace_head(p, w8a8, (int)x_dtype, m, dims.in_dim);
  if (need_ws > 0 && (workspace == nullptr || workspace_bytes < need_ws))
    return fail(CMK_ERR_INVALID_ARGUMENT,
                "iq2_matmul workspace too small: got %zu expected at least %zu (see "
                "cmk_iq2_matmul_workspace_size)",
                workspace ? workspace_bytes : (size_t)0, need_ws);
  const size_t ws_align = p == Path::Gemm ? 16 : 4;
  if (need_ws > 0 && !aligned(workspace, ws_align))
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_matmul workspace must be %zu-byte aligned", ws_align);

  int cus = 0;
  rc = current_cu_count(&cus);
  if (rc != CMK_OK) return rc;
  // the multi-row kernel's split over K, when the workspace has room for it
  void* split_ws = nullptr;
  size_t split_ws_bytes = 0;
  const size_t split_need = rows_split_bytes(p, w8a8, m, dims.out_dim, dims.in_dim, cus);
  if (split_need > 0 && workspace != nullptr && aligned(workspace, 16) &&
      workspace_bytes >= split_offset(need_ws) + split_need) {
    split_ws = static_cast<uint8_t*>(workspace) + split_offset(need_ws);
    split_ws_bytes = workspace_bytes - split_offset(need_ws);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = hipSuccess;
  float* row_inv = head_ws > 0 ? static_cast<float*>(workspace) : nullptr;
  float* partials =
      need_ws > head_ws ? reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + head_ws)
                        : nullptr;
  // IQ2_XS / IQ2_S / IQ3_S with aligned weights: the multi-row decode kernel
  // (W8A8 scales computed there; the workspace stays unused)
  const bool variant_rows = p == Path::Variant && aligned(weight_bytes, 16) &&
                            aligned(weight_scales, 2) &&
                            cmk::variant_rows_supported((int)variant, dims.out_dim, dims.in_dim,
                                                        (int)x_dtype);
  // IQ2_XS, IQ2_S and IQ3_S at m = 1 take the one-row GEMV where it fits
  const bool variant_one_row = p == Path::Variant && dims.m == 1 &&
                          cmk::iq_variant_gemv_fits((int)variant, x, weight_bytes, weight_scales,
                                                    dims.out_dim, dims.in_dim, (int)x_dtype, cus);
  if (row_inv && w8a8 && !variant_rows && !variant_one_row) {  // (f32 rows staged for the GEMM get their scales there)
    e = cmk::launch_iq2xxs_row_inv_scale(x, (int)x_dtype, dims.m, dims.in_dim, row_inv, s);
    if (e != hipSuccess) return hip_fail(e, "iq2_matmul row scale launch");
  }
  switch (p) {
    case Path::Gemv:
      e = cmk::launch_iq2xxs_gemv(x, (int)x_dtype, dims.m, weight_bytes, weight_scales, out,
                                  dims.out_dim, dims.in_dim, w8a8, cus, s, nullptr, split_ws,
                                  split_ws_bytes);
      break;
    case Path::Gemm:
      e = cmk::launch_iq2xxs_gemm(
          x, (int)x_dtype, dims.m, weight_bytes, weight_scales, out, dims.out_dim, dims.in_dim,
          row_inv, row_inv ? static_cast<uint8_t*>(workspace) + row_scale_bytes(m) : nullptr, w8a8,
          partials, s);
      break;
    case Path::Simple:
      e = cmk::launch_iq2xxs_matmul_simple(x, (int)x_dtype, dims.m, weight_bytes, weight_scales,
                                           out, dims.out_dim, dims.in_dim, row_inv, cus, s);
      break;
    case Path::Variant:
      e = variant_one_row
              ? cmk::launch_iq_variant_gemv((int)variant, x, (int)x_dtype, weight_bytes,
                                            weight_scales, out, dims.out_dim, dims.in_dim, w8a8,
                                            cus, s)
          : variant_rows
              ? cmk::launch_iq_variant_rows((int)variant, x, (int)x_dtype, dims.m, weight_bytes,
                                            weight_scales, out, dims.out_dim, dims.in_dim, w8a8,
                                            cus, s, split_ws, split_ws_bytes)
              : cmk::launch_iq_variant_matmul((int)variant, x, (int)x_dtype, dims.m,
                                              weight_bytes, weight_scales, out, dims.out_dim,
                                              dims.in_dim, row_inv, cus, s);
      break;
  }
  if (e != hipSuccess) return hip_fail(e, "iq2_matmul launch");
  return ok();
}

int cmk_iq2_matmul_noalloc(const void* x, cmk_dtype x_dtype, size_t x_len, size_t m,
                           const uint8_t* weight_bytes, size_t weight_bytes_len,
                           const uint8_t* weight_scales, size_t weight_scales_len, size_t out_dim,
                           size_t in_dim, cmk_iq2_variant variant, cmk_act_quant_mode mode,
                           int strict, float* out, void* stream) {
  int md = (int)mode;
  Dims dims;
  int rc = validate_matmul((int)x_dtype, m, out_dim, in_dim, (int)variant, &md, strict,
                           weight_bytes_len, weight_scales_len, true, &dims);
  if (rc != CMK_OK) return rc;
  if (m == 0) return ok();
  const Path p = variant != CMK_IQ2_XXS ? Path::Variant
                                        : choose_path((int)x_dtype, m, dims.out_dim, dims.in_dim,
                                                      x, weight_bytes, weight_scales,
                                                      md == CMK_ACT_QUANT_W8A8);
  const size_t need =
      workspace_for(p, md == CMK_ACT_QUANT_W8A8, (int)x_dtype, m, dims.out_dim, dims.in_dim);
  if (need > (size_t)CMK_IQ2_NOALLOC_SCRATCH_BYTES)
    return fail(CMK_ERR_INVALID_ARGUMENT,
                "cmk_iq2_matmul_noalloc needs %zu bytes of scratch for these arguments, more "
                "than its fixed %zu (call cmk_iq2_matmul with a workspace instead)",
                need, (size_t)CMK_IQ2_NOALLOC_SCRATCH_BYTES);
  void* work = nullptr;
  if (need > 0) {
    rc = device_scratch(&work);
    if (rc != CMK_OK) return rc;
  }
  return cmk_iq2_matmul(x, x_dtype, x_len, m, weight_bytes, weight_bytes_len, weight_scales,
                        weight_scales_len, out_dim, in_dim, variant, mode, strict, out, work,
                        need > 0 ? (size_t)CMK_IQ2_NOALLOC_SCRATCH_BYTES : 0, stream);
}

int cmk_iq2_dequantize(const uint8_t* weight_bytes, size_t weight_bytes_len,
                       const uint8_t* weight_scales, size_t weight_scales_len, size_t out_dim,
                       size_t in_dim, cmk_iq2_variant variant, cmk_dtype out_dtype, void* out,
                       void* stream) {
  // iq2_dequantize_to_f16_metal guards (src/iq2_matmul.rs:367-433)
  if (out_dim == 0 || in_dim == 0)
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_dequantize_to_f16 expects non-zero dimensions");
  if ((int)variant < CMK_IQ2_XXS || (int)variant > CMK_IQ3_S)
    return fail(CMK_ERR_INVALID_ARGUMENT, "invalid iq2 variant: %d", (int)variant);
  if (out_dtype != CMK_F32 && out_dtype != CMK_F16 && out_dtype != CMK_BF16)
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_dequantize unsupported output dtype: %d",
                (int)out_dtype);
  const size_t bpr = (in_dim + 255) / 256;
  size_t blocks, expected_bytes, expected_scales, total;
  if (!checked_mul(out_dim, bpr, &blocks) ||
      !checked_mul(blocks, bytes_per_block((int)variant), &expected_bytes))
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_dequantize_to_f16 bytes size overflow");
  if (!checked_mul(blocks, scales_per_block((int)variant), &expected_scales))
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_dequantize_to_f16 scales size overflow");
  if (weight_bytes_len < expected_bytes)
    return fail(CMK_ERR_INVALID_ARGUMENT,
                "iq2_dequantize_to_f16 weight_bytes too small: got %zu expected at least %zu",
                weight_bytes_len, expected_bytes);
  if (weight_scales_len < expected_scales)
    return fail(CMK_ERR_INVALID_ARGUMENT,
                "iq2_dequantize_to_f16 weight_scales too small: got %zu expected at least %zu",
                weight_scales_len, expected_scales);
  if (!checked_mul(out_dim, in_dim, &total))
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_dequantize_to_f16 output size overflow");
  if (out_dim > UINT32_MAX) return fail(CMK_ERR_INVALID_ARGUMENT, "out_dim too large");
  if (in_dim > UINT32_MAX) return fail(CMK_ERR_INVALID_ARGUMENT, "in_dim too large");
  if (!weight_bytes || !weight_scales || !out)
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_dequantize_to_f16 null pointer argument");
  if (variant == CMK_IQ2_XXS && (!aligned(weight_bytes, 8) || !aligned(weight_scales, 2)))
    return fail(CMK_ERR_INVALID_ARGUMENT,
                "iq2_dequantize_to_f16 needs 8-byte aligned weight_bytes and 2-byte aligned "
                "weight_scales");
  if (!aligned(out, out_dtype == CMK_F32 ? 4 : 2))
    return fail(CMK_ERR_INVALID_ARGUMENT, "iq2_dequantize_to_f16 out is misaligned");
  int cus = 0;
  int rc = current_cu_count(&cus);
  if (rc != CMK_OK) return rc;
  hipError_t e =
      variant == CMK_IQ2_XXS
          ? cmk::launch_iq2xxs_dequant(weight_bytes, weight_scales, out, (int)out_dtype,
                                       (uint32_t)out_dim, (uint32_t)in_dim, cus,
                                       static_cast<hipStream_t>(stream))
          : cmk::launch_iq_variant_dequant((int)variant, weight_bytes, weight_scales, out,
                                           (int)out_dtype, (uint32_t)out_dim, (uint32_t)in_dim,
                                           cus, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "iq2_dequantize launch");
  return ok();
}

int cmk_iq2_split_gguf_blocks(const uint8_t* blocks, size_t blocks_len, size_t n_blocks,
                              cmk_iq2_variant variant, uint8_t* weight_bytes,
                              size_t weight_bytes_len, uint8_t* weight_scales,
                              size_t weight_scales_len, void* stream) {
  if ((int)variant < CMK_IQ2_XXS || (int)variant > CMK_IQ3_S)
    return fail(CMK_ERR_INVALID_ARGUMENT, "invalid iq2 variant: %d", (int)variant);
  const size_t cb = bytes_per_block((int)variant), sb = scales_per_block((int)variant);
  size_t need_src, need_b, need_s;
  if (!checked_mul(n_blocks, cb + sb, &need_src) || !checked_mul(n_blocks, cb, &need_b) ||
      !checked_mul(n_blocks, sb, &need_s))
    return fail(CMK_ERR_INVALID_ARGUMENT, "split_gguf_blocks size overflow");
  if (blocks_len < need_src)
    return fail(CMK_ERR_INVALID_ARGUMENT,
                "split_gguf_blocks blocks too small: got %zu expected at least %zu", blocks_len,
                need_src);
  if (weight_bytes_len < need_b)
    return fail(CMK_ERR_INVALID_ARGUMENT,
                "split_gguf_blocks weight_bytes too small: got %zu expected at least %zu",
                weight_bytes_len, need_b);
  if (weight_scales_len < need_s)
    return fail(CMK_ERR_INVALID_ARGUMENT,
                "split_gguf_blocks weight_scales too small: got %zu expected at least %zu",
                weight_scales_len, need_s);
  if (n_blocks == 0) return ok();
  if (!blocks || !weight_bytes || !weight_scales)
    return fail(CMK_ERR_INVALID_ARGUMENT, "split_gguf_blocks null pointer argument");
  int cus = 0;
  int rc = current_cu_count(&cus);
  if (rc != CMK_OK) return rc;
  hipError_t e = cmk::launch_gguf_split(blocks, n_blocks, (uint32_t)cb, (uint32_t)sb, weight_bytes,
                                        weight_scales, cus, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "split_gguf_blocks launch");
  return ok();
}

int cmk_swiglu(const float* gate, const float* up, size_t n, cmk_dtype out_dtype, void* out,
               void* stream) {
  if (out_dtype != CMK_F32 && out_dtype != CMK_F16 && out_dtype != CMK_BF16)
    return fail(CMK_ERR_INVALID_ARGUMENT, "swiglu unsupported output dtype: %d", (int)out_dtype);
  if (n == 0) return ok();
  if (!gate || !up || !out) return fail(CMK_ERR_INVALID_ARGUMENT, "swiglu null pointer argument");
  if (!aligned(gate, 4) || !aligned(up, 4) || !aligned(out, out_dtype == CMK_F32 ? 4 : 2))
    return fail(CMK_ERR_INVALID_ARGUMENT, "swiglu buffers must be aligned to their element size");
  int cus = 0;
  int rc = current_cu_count(&cus);
  if (rc != CMK_OK) return rc;
  hipError_t e = cmk::launch_swiglu(gate, up, out, (int)out_dtype, n, cus,
                                    static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "swiglu launch");
  return ok();
}

int cmk_iq2_matmul_swiglu(const void* x, cmk_dtype x_dtype, size_t x_len, size_t m,
                          const uint8_t* weight_bytes, size_t weight_bytes_len,
                          const uint8_t* weight_scales, size_t weight_scales_len,
                          size_t out_dim, size_t in_dim, const float* gate, size_t gate_len,
                          float* out, void* workspace, size_t workspace_bytes, void* stream) {
  int md = CMK_ACT_QUANT_OFF;
  Dims dims;
  int rc = validate_matmul((int)x_dtype, m, out_dim, in_dim, CMK_IQ2_XXS, &md, 0,
                           weight_bytes_len, weight_scales_len, true, &dims);
  if (rc != CMK_OK) return rc;
  if (m == 0) return ok();
  size_t need_x, need_out;
  if (!checked_mul(m, in_dim, &need_x) || !checked_mul(m, out_dim, &need_out))
    return fail(CMK_ERR_INVALID_ARGUMENT, "matmul_swiglu size overflow");
  if (x_len < need_x)
    return fail(CMK_ERR_INVALID_ARGUMENT,
                "matmul_swiglu x too small: got %zu expected at least %zu", x_len, need_x);
  if (gate_len < need_out)
    return fail(CMK_ERR_INVALID_ARGUMENT,
                "matmul_swiglu gate too small: got %zu expected at least %zu", gate_len,
                need_out);
  if (!x || !weight_bytes || !weight_scales || !gate || !out)
    return fail(CMK_ERR_INVALID_ARGUMENT, "matmul_swiglu null pointer argument");
  const size_t esize = x_dtype == CMK_F32 ? 4 : 2;
  if (!aligned(x, esize) || !aligned(gate, 4) || !aligned(out, 4))
    return fail(CMK_ERR_INVALID_ARGUMENT,
                "matmul_swiglu x, gate and out must be aligned to their element size");
  const uintptr_t g0 = reinterpret_cast<uintptr_t>(gate), o0 = reinterpret_cast<uintptr_t>(out);
  if (g0 < o0 + need_out * 4 && o0 < g0 + need_out * 4)
    return fail(CMK_ERR_INVALID_ARGUMENT, "matmul_swiglu gate must not overlap out");
  if (choose_path((int)x_dtype, m, dims.out_dim, dims.in_dim, x, weight_bytes, weight_scales,
                  false) != Path::Gemv)
    return fail(CMK_ERR_UNSUPPORTED,
                "matmul_swiglu serves the decode-shaped kernels (m <= %zu, aligned weights): use "
                "cmk_iq2_matmul and cmk_swiglu",
                kGemvMaxM);
  int cus = 0;
  rc = current_cu_count(&cus);
  if (rc != CMK_OK) return rc;
  // the split over K as cmk_iq2_matmul takes it (the GEMV path needs no other
  // workspace)
  const size_t split_need = rows_split_bytes(Path::Gemv, false, m, dims.out_dim, dims.in_dim, cus);
  const bool split = split_need > 0 && workspace != nullptr && aligned(workspace, 16) &&
                     workspace_bytes >= split_need;
  const hipError_t e = cmk::launch_iq2xxs_gemv(
      x, (int)x_dtype, dims.m, weight_bytes, weight_scales, out, dims.out_dim, dims.in_dim, false,
      cus, static_cast<hipStream_t>(stream), gate, split ? workspace : nullptr,
      split ? workspace_bytes : 0);
  if (e != hipSuccess) return hip_fail(e, "matmul_swiglu launch");
  return ok();
}

// ---- runtime wrappers -----------------------------------------------------

int cmk_device_count(int* count) {
  if (!count) return fail(CMK_ERR_INVALID_ARGUMENT, "null pointer argument");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    *count = 0;
    return fail(CMK_ERR_NO_DEVICE, "hipGetDeviceCount failed: %s", hipGetErrorString(e));
  }
  *count = n;
  return ok();
}

int cmk_set_device(int ordinal) {
  hipError_t e = hipSetDevice(ordinal);
  return e == hipSuccess ? ok() : hip_fail(e, "hipSetDevice");
}

int cmk_device_props(char* name, size_t name_len, int* cu_count, size_t* lds_bytes,
                     int* mem_clock_khz, int* mem_bus_bits) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  hipDeviceProp_t p;
  e = hipGetDeviceProperties(&p, dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  if (name && name_len) snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
  if (cu_count) *cu_count = p.multiProcessorCount;
  if (lds_bytes) *lds_bytes = p.maxSharedMemoryPerMultiProcessor;
  if (mem_clock_khz) *mem_clock_khz = p.memoryClockRate;
  if (mem_bus_bits) *mem_bus_bits = p.memoryBusWidth;
  return ok();
}

int cmk_malloc(void** ptr, size_t bytes) {
  if (!ptr) return fail(CMK_ERR_INVALID_ARGUMENT, "null pointer argument");
  hipError_t e = hipMalloc(ptr, bytes);
  return e == hipSuccess ? ok() : hip_fail(e, "hipMalloc");
}

int cmk_free(void* ptr) {
  hipError_t e = hipFree(ptr);
  return e == hipSuccess ? ok() : hip_fail(e, "hipFree");
}

int cmk_memcpy_htod(void* dst, const void* src, size_t bytes, void* stream) {
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice,
                                static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "hipMemcpyAsync(H2D)");
}

int cmk_memcpy_dtoh(void* dst, const void* src, size_t bytes, void* stream) {
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost,
                                static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "hipMemcpyAsync(D2H)");
}

int cmk_memset(void* dst, int value, size_t bytes, void* stream) {
  hipError_t e = hipMemsetAsync(dst, value, bytes, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "hipMemsetAsync");
}

int cmk_stream_create(void** stream) {
  if (!stream) return fail(CMK_ERR_INVALID_ARGUMENT, "null pointer argument");
  hipStream_t s = nullptr;
  hipError_t e = hipStreamCreate(&s);  // default priority
  if (e != hipSuccess) return hip_fail(e, "hipStreamCreate");
  *stream = s;
  return ok();
}

int cmk_stream_destroy(void* stream) {
  hipError_t e = hipStreamDestroy(static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "hipStreamDestroy");
}

int cmk_stream_synchronize(void* stream) {
  hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "hipStreamSynchronize");
}

int cmk_device_synchronize(void) {
  hipError_t e = hipDeviceSynchronize();
  return e == hipSuccess ? ok() : hip_fail(e, "hipDeviceSynchronize");
}

int cmk_event_create(void** event) {
  if (!event) return fail(CMK_ERR_INVALID_ARGUMENT, "null pointer argument");
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreate(&ev);
  if (e != hipSuccess) return hip_fail(e, "hipEventCreate");
  *event = ev;
  return ok();
}

int cmk_event_destroy(void* event) {
  hipError_t e = hipEventDestroy(static_cast<hipEvent_t>(event));
  return e == hipSuccess ? ok() : hip_fail(e, "hipEventDestroy");
}

int cmk_event_record(void* event, void* stream) {
  hipError_t e = hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "hipEventRecord");
}

int cmk_event_elapsed_ms(void* start, void* stop, float* ms) {
  if (!ms) return fail(CMK_ERR_INVALID_ARGUMENT, "null pointer argument");
  hipError_t e = hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                     static_cast<hipEvent_t>(stop));
  return e == hipSuccess ? ok() : hip_fail(e, "hipEventElapsedTime");
}

}  // extern "C"

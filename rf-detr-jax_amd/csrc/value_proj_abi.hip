// value_proj_abi.hip — C ABI of the value projection with its fused epilogue (include/msda.h):
// validation, launch planning, kernel launches. Validation runs before any HIP call.
#include "msda.h"
#include "msda_launch.h"
#include "msda_kernels.h"  // bf16_t
#include "value_proj_kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>

namespace {

using msda_host::aligned_to;
using msda_host::fail;

int vp_validate(int dtype, int batch, int len_in, int in_features, int n_heads, int head_dim) {
  if (dtype != MSDA_DTYPE_F32 && dtype != MSDA_DTYPE_BF16) return fail(MSDA_ERR_UNSUPPORTED, "input: unsupported dtype code %d", dtype);
  if (batch < 0 || len_in < 0) return fail(MSDA_ERR_INVALID_ARGUMENT, "batch (%d) and len_in (%d) must be >= 0", batch, len_in);
  if (in_features < 1 || n_heads < 1 || head_dim < 1)
    return fail(MSDA_ERR_INVALID_ARGUMENT, "in_features (%d), n_heads (%d) and head_dim (%d) must be >= 1", in_features, n_heads, head_dim);
  const int64_t m = static_cast<int64_t>(batch) * len_in, n = static_cast<int64_t>(n_heads) * head_dim;
  if (m >= (int64_t{1} << 31) || n >= (int64_t{1} << 24) || in_features >= (1 << 24) || m * std::max<int64_t>(n, in_features) >= (int64_t{1} << 40))
    return fail(MSDA_ERR_UNSUPPORTED, "value projection too large");
  // channel n of a row splits into (head, d), and row m into (batch, position), by multiply-highs,
  // exact while n * head_dim and m * len_in stay below 2^32; element offsets are 32-bit
  if (n * head_dim >= (int64_t{1} << 32) || m * len_in >= (int64_t{1} << 32))
    return fail(MSDA_ERR_UNSUPPORTED, "n_heads * head_dim^2 or batch * len_in^2 reaches 2^32");
  if (m * n >= (int64_t{1} << 32) || m * in_features >= (int64_t{1} << 32) || n * (static_cast<int64_t>(in_features) + 1) >= (int64_t{1} << 32))
    return fail(MSDA_ERR_UNSUPPORTED, "a value-projection tensor reaches 2^32 elements");
  return MSDA_OK;
}

// grad_weight's product is split over m into slices of at least 256 rows (at most 64 slices); the
// partial sums [splits][N][K + 1] are the workspace. A function of the shape only.
int vp_splits(int64_t m) { return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(64, (m + 255) / 256))); }

int64_t vp_workspace(int batch, int len_in, int in_features, int n_heads, int head_dim) {
  const int64_t m = static_cast<int64_t>(batch) * len_in;
  return static_cast<int64_t>(vp_splits(m)) * n_heads * head_dim * (in_features + 1) * 4;
}

int tiles(int64_t rows, int64_t cols) {
  return static_cast<int>(((rows + msda::kGemmBM - 1) / msda::kGemmBM) * ((cols + msda::kGemmBN - 1) / msda::kGemmBN));
}

}  // namespace

extern "C" {

int msda_value_proj_fwd(const void* input, int dtype, const float* weight, const float* bias, const uint8_t* padding_mask, void* value,
                        int batch, int len_in, int in_features, int n_heads, int head_dim, void* stream) {
  msda_host::clear_error();
  int rc = vp_validate(dtype, batch, len_in, in_features, n_heads, head_dim);
  if (rc != MSDA_OK) return rc;
  if (batch == 0 || len_in == 0) return MSDA_OK;
  if (input == nullptr || weight == nullptr || value == nullptr) return fail(MSDA_ERR_INVALID_ARGUMENT, "msda_value_proj_fwd: NULL tensor pointer");
  const size_t eb = dtype == MSDA_DTYPE_BF16 ? 2 : 4;
  if (!aligned_to(input, eb) || !aligned_to(value, eb) || !aligned_to(weight, 4) || !aligned_to(bias, 4))
    return fail(MSDA_ERR_INVALID_ARGUMENT, "tensors must be aligned to their element size");
  msda::ValueProjParams p{};
  p.x = input;
  p.w = weight;
  p.bias = bias;
  p.mask = padding_mask;
  p.value = value;
  p.bf16 = dtype == MSDA_DTYPE_BF16;
  p.batch = batch;
  p.seq = len_in;
  p.k = in_features;
  p.n = n_heads * head_dim;
  p.heads = n_heads;
  p.dim = head_dim;
  p.dim_magic = static_cast<uint32_t>(((uint64_t{1} << 32) + head_dim - 1) / head_dim);
  p.seq_magic = static_cast<uint32_t>(((uint64_t{1} << 32) + len_in - 1) / len_in);
  const int g = tiles(static_cast<int64_t>(batch) * len_in, p.n);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (p.bf16) hipLaunchKernelGGL((msda::gemm_kernel<msda::kGemmForward, msda::bf16_t>), dim3(g), dim3(256), 0, st, p);
  else hipLaunchKernelGGL((msda::gemm_kernel<msda::kGemmForward, float>), dim3(g), dim3(256), 0, st, p);
  return msda_host::check_launch("value projection forward");
}

int64_t msda_value_proj_bwd_workspace_size(int batch, int len_in, int in_features, int n_heads, int head_dim) {
  msda_host::clear_error();
  const int rc = vp_validate(MSDA_DTYPE_F32, batch, len_in, in_features, n_heads, head_dim);
  if (rc != MSDA_OK) return rc;
  return vp_workspace(batch, len_in, in_features, n_heads, head_dim);
}

int msda_value_proj_bwd(const void* input, int dtype, const float* weight, const uint8_t* padding_mask, const void* grad_value,
                        void* grad_input, float* grad_weight, float* grad_bias, int batch, int len_in, int in_features, int n_heads,
                        int head_dim, void* workspace, int64_t workspace_bytes, void* stream) {
  msda_host::clear_error();
  int rc = vp_validate(dtype, batch, len_in, in_features, n_heads, head_dim);
  if (rc != MSDA_OK) return rc;
  const bool want_w = grad_weight != nullptr || grad_bias != nullptr;
  if (grad_input == nullptr && !want_w) return MSDA_OK;
  const int64_t m = static_cast<int64_t>(batch) * len_in;
  const size_t eb = dtype == MSDA_DTYPE_BF16 ? 2 : 4;
  if (m > 0) {
    if (grad_value == nullptr || weight == nullptr || (want_w && input == nullptr))
      return fail(MSDA_ERR_INVALID_ARGUMENT, "msda_value_proj_bwd: NULL tensor pointer");
    if (!aligned_to(input, eb) || !aligned_to(grad_value, eb) || !aligned_to(grad_input, eb) || !aligned_to(weight, 4) ||
        !aligned_to(grad_weight, 4) || !aligned_to(grad_bias, 4))
      return fail(MSDA_ERR_INVALID_ARGUMENT, "tensors must be aligned to their element size");
  }
  const int64_t ws = vp_workspace(batch, len_in, in_features, n_heads, head_dim);
  if (want_w) {
    if (workspace == nullptr) return fail(MSDA_ERR_INVALID_ARGUMENT, "workspace is NULL (see msda_value_proj_bwd_workspace_size)");
    if (!aligned_to(workspace, 16)) return fail(MSDA_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
    if (workspace_bytes < ws)
      return fail(MSDA_ERR_INVALID_ARGUMENT, "workspace of %lld bytes needed, got %lld", static_cast<long long>(ws),
                  static_cast<long long>(workspace_bytes));
  }
  msda::ValueProjParams p{};
  p.x = input;
  p.w = weight;
  p.mask = padding_mask;
  p.gvalue = grad_value;
  p.gx = grad_input;
  p.gw = grad_weight;
  p.gb = grad_bias;
  p.gw_part = static_cast<float*>(workspace);
  p.bf16 = dtype == MSDA_DTYPE_BF16;
  p.batch = batch;
  p.seq = len_in;
  p.k = in_features;
  p.n = n_heads * head_dim;
  p.heads = n_heads;
  p.dim = head_dim;
  p.splits = vp_splits(m);
  p.dim_magic = static_cast<uint32_t>(((uint64_t{1} << 32) + head_dim - 1) / head_dim);
  p.seq_magic = len_in > 0 ? static_cast<uint32_t>(((uint64_t{1} << 32) + len_in - 1) / len_in) : 0u;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (grad_input != nullptr && m > 0) {
    if (p.bf16) hipLaunchKernelGGL((msda::gemm_kernel<msda::kGemmGradInput, msda::bf16_t>), dim3(tiles(m, in_features)), dim3(256), 0, st, p);
    else hipLaunchKernelGGL((msda::gemm_kernel<msda::kGemmGradInput, float>), dim3(tiles(m, in_features)), dim3(256), 0, st, p);
    if ((rc = msda_host::check_launch("value projection backward (input)")) != MSDA_OK) return rc;
  }
  if (want_w) {
    // with no rows the partial sums are zero: the product still runs (every partial is written)
    const int64_t g = static_cast<int64_t>(tiles(p.n, static_cast<int64_t>(in_features) + 1)) * p.splits;
    if (p.bf16) hipLaunchKernelGGL((msda::gemm_kernel<msda::kGemmGradWeight, msda::bf16_t>), dim3(static_cast<unsigned>(g)), dim3(256), 0, st, p);
    else hipLaunchKernelGGL((msda::gemm_kernel<msda::kGemmGradWeight, float>), dim3(static_cast<unsigned>(g)), dim3(256), 0, st, p);
    if ((rc = msda_host::check_launch("value projection backward (weight)")) != MSDA_OK) return rc;
    const int64_t total = static_cast<int64_t>(p.n) * (in_features + 1);
    hipLaunchKernelGGL(msda::wg_reduce_kernel, dim3(static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 4096))), dim3(256), 0, st,
                       p);
    if ((rc = msda_host::check_launch("value projection backward (weight reduction)")) != MSDA_OK) return rc;
  }
  return MSDA_OK;
}

}  // extern "C"

// value_proj_abi.hip — C ABI of the value projection with its fused epilogue (include/msda.h):
// validation, launch planning, kernel launches. Validation runs before any HIP call.
#include "msda.h"
#include "msda_launch.h"
#include "msda_kernels.h"  // bf16_t
#include "value_proj_kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>

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

// ceil(2^32 / divisor) for the kernels' multiply-high divisions (vp_div); 0 marks a divisor of 1
// (and an empty extent), whose magic 2^32 does not fit 32 bits.
uint32_t vp_magic(int divisor) {
  return divisor > 1 ? static_cast<uint32_t>(((uint64_t{1} << 32) + static_cast<uint64_t>(divisor) - 1) / static_cast<uint64_t>(divisor)) : 0u;
}

// grad_weight's product is split over m into slices of at least 256 rows (at most 64 slices); the
// partial sums [splits][N][K + 1] are the workspace. A function of the shape only.
int vp_splits(int64_t m) { return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(64, (m + 255) / 256))); }

int64_t vp_workspace(int batch, int len_in, int in_features, int n_heads, int head_dim) {
  const int64_t m = static_cast<int64_t>(batch) * len_in;
  return static_cast<int64_t>(vp_splits(m)) * n_heads * head_dim * (in_features + 1) * 4;
}

// The 16-byte operand kernels need every 4-element vector they load contiguous and aligned: the
// reduction and column extents K and D multiples of 4 (so N is too), and the tensors they read
// aligned to 4 elements. MSDA_VP_SCALAR forces the element-wise kernels.
bool vec_path(const msda::ValueProjParams& p, size_t eb, const void* a, const void* b) {
  if (msda_host::env_flag("MSDA_VP_SCALAR")) return false;
  return p.k % 4 == 0 && p.dim % 4 == 0 && aligned_to(p.w, 16) && (a == nullptr || aligned_to(a, 4 * eb)) &&
         (b == nullptr || aligned_to(b, 4 * eb));
}

template <int KIND, typename VT, int BM>
int launch_g4(const msda::ValueProjParams& p, int grid, hipStream_t st) {
  static std::atomic<int> granted[msda_host::kMaxDevices];  // per instantiation
  auto k = msda::gemm4_kernel<KIND, VT, BM>;
  const int rc = msda_host::allow_lds(k, msda::G4<BM>::kLdsBytes, granted);
  if (rc != MSDA_OK) return rc;
  hipLaunchKernelGGL(k, dim3(grid), dim3(msda::G4<BM>::kThreads), msda::G4<BM>::kLdsBytes, st, p);
  return MSDA_OK;
}

// One product: rows x cols outputs (times `splits` slices of the reduction). The 16-byte kernels
// take 32-row tiles when 64-row tiles would be fewer than four per CU (a CU with one tile more
// than another finishes a whole tile later; smaller tiles even that out), else 64-row tiles;
// MSDA_VP_BM=32 or 64 forces one.
template <int KIND, typename VT>
int launch_gemm(const msda::ValueProjParams& p, int64_t rows, int64_t cols, int splits, bool vec, hipStream_t st, const char* what) {
  int rc = MSDA_OK;
  const int64_t ct = (cols + msda::kGemmBN - 1) / msda::kGemmBN;
  if (vec) {
    int lds = 0, cus = 0;
    if ((rc = msda_host::device_attrs(&lds, &cus)) != MSDA_OK) return rc;
    const int64_t t64 = (rows + 63) / 64 * ct * splits;
    int bm = t64 < 4 * static_cast<int64_t>(cus) ? 32 : 64;
    const int e = msda_host::knob("MSDA_VP_BM", 0);
    bm = e == 32 ? 32 : e == 64 ? 64 : bm;
    if (bm == 32) rc = launch_g4<KIND, VT, 32>(p, static_cast<int>((rows + 31) / 32 * ct * splits), st);
    else rc = launch_g4<KIND, VT, 64>(p, static_cast<int>(t64), st);
    if (rc != MSDA_OK) return rc;
  } else {
    hipLaunchKernelGGL((msda::gemm_kernel<KIND, VT>), dim3(static_cast<unsigned>((rows + 63) / 64 * ct * splits)), dim3(256), 0, st, p);
  }
  return msda_host::check_launch(what);
}

template <int KIND>
int launch_gemm_dt(const msda::ValueProjParams& p, int64_t rows, int64_t cols, int splits, bool vec, hipStream_t st, const char* what) {
  return p.bf16 ? launch_gemm<KIND, msda::bf16_t>(p, rows, cols, splits, vec, st, what)
                : launch_gemm<KIND, float>(p, rows, cols, splits, vec, st, what);
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
  p.dim_magic = vp_magic(head_dim);
  p.seq_magic = vp_magic(len_in);
  return launch_gemm_dt<msda::kGemmForward>(p, static_cast<int64_t>(batch) * len_in, p.n, 1, vec_path(p, eb, input, nullptr),
                                            static_cast<hipStream_t>(stream), "value projection forward");
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
  p.dim_magic = vp_magic(head_dim);
  p.seq_magic = vp_magic(len_in);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (grad_input != nullptr && m > 0) {
    const bool vec = vec_path(p, eb, grad_value, nullptr);
    if ((rc = launch_gemm_dt<msda::kGemmGradInput>(p, m, in_features, 1, vec, st, "value projection backward (input)")) != MSDA_OK)
      return rc;
  }
  if (want_w) {
    // with no rows the partial sums are zero: the product still runs (every partial is written).
    // The element-wise kernel forms the bias gradient as a column of ones (K + 1 columns); the
    // 16-byte kernel sums dY^T rows instead (K columns).
    const bool vec = vec_path(p, eb, grad_value, input);
    if ((rc = launch_gemm_dt<msda::kGemmGradWeight>(p, p.n, static_cast<int64_t>(in_features) + (vec ? 0 : 1), p.splits, vec, st,
                                                     "value projection backward (weight)")) != MSDA_OK)
      return rc;
    const int64_t total = static_cast<int64_t>(p.n) * (in_features + 1);
    hipLaunchKernelGGL(msda::wg_reduce_kernel, dim3(static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 4096))), dim3(256), 0, st,
                       p);
    if ((rc = msda_host::check_launch("value projection backward (weight reduction)")) != MSDA_OK) return rc;
  }
  return MSDA_OK;
}

}  // extern "C"

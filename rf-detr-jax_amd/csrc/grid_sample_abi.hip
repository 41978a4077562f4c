// grid_sample_abi.hip — C ABI of bilinear_grid_sample / point_sample (include/msda.h): argument
// validation, launch planning, kernel launches. Validation runs before any HIP call.
#include "grid_sample_kernels.h"
#include "msda.h"
#include "msda_launch.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>

namespace {

using msda_host::aligned_to;
using msda_host::fail;

int gs_validate(int dtype, int n, int channels, int height, int width, int n_points, int grid_kind, int padding_mode,
                int sample_mode) {
  if (dtype != MSDA_DTYPE_F32 && dtype != MSDA_DTYPE_BF16) return fail(MSDA_ERR_UNSUPPORTED, "input: unsupported dtype code %d", dtype);
  if (n < 0 || n_points < 0) return fail(MSDA_ERR_INVALID_ARGUMENT, "n (%d) and n_points (%d) must be >= 0", n, n_points);
  if (channels < 1 || height < 1 || width < 1)
    return fail(MSDA_ERR_INVALID_ARGUMENT, "channels (%d), height (%d) and width (%d) must be >= 1", channels, height, width);
  if (grid_kind != MSDA_GRID_COORDS && grid_kind != MSDA_GRID_UNIT_POINTS)
    return fail(MSDA_ERR_INVALID_ARGUMENT, "grid_kind must be MSDA_GRID_COORDS or MSDA_GRID_UNIT_POINTS, got %d", grid_kind);
  if (padding_mode != MSDA_PADDING_ZEROS && padding_mode != MSDA_PADDING_BORDER)
    return fail(MSDA_ERR_INVALID_ARGUMENT, "padding_mode must be 'zeros' or 'border' (got code %d)", padding_mode);
  if (sample_mode != MSDA_SAMPLE_BILINEAR && sample_mode != MSDA_SAMPLE_NEAREST)
    return fail(MSDA_ERR_INVALID_ARGUMENT, "sample mode must be bilinear or nearest (got code %d)", sample_mode);
  if (sample_mode == MSDA_SAMPLE_NEAREST && padding_mode != MSDA_PADDING_BORDER)
    return fail(MSDA_ERR_UNSUPPORTED, "nearest sampling is defined with border padding only (segmentation.py:173-186)");
  if (static_cast<int64_t>(height) * width >= (int64_t{1} << 31)) return fail(MSDA_ERR_UNSUPPORTED, "height * width reaches 2^31");
  // lanes index (slice, point) pairs in 32 bits
  if (static_cast<int64_t>(n) * n_points >= (int64_t{1} << 31)) return fail(MSDA_ERR_UNSUPPORTED, "n * n_points reaches 2^31");
  return MSDA_OK;
}

msda::GridSampleParams gs_params(const void* input, int dtype, const float* grid, int grid_kind, int n, int channels, int height,
                                 int width, int n_points, int padding_mode, int sample_mode) {
  msda::GridSampleParams p{};
  p.input = input;
  p.grid = grid;
  p.bf16 = dtype == MSDA_DTYPE_BF16;
  p.n = n;
  p.c = channels;
  p.h = height;
  p.w = width;
  p.points = n_points;
  p.unit_points = grid_kind == MSDA_GRID_UNIT_POINTS;
  p.border = padding_mode == MSDA_PADDING_BORDER;
  p.nearest = sample_mode == MSDA_SAMPLE_NEAREST;
  return p;
}

int lane_grid(int64_t lanes) {
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>((lanes + 255) / 256, int64_t{1} << 20)));
}

}  // namespace

extern "C" {

int msda_grid_sample_fwd(const void* input, int dtype, const float* grid, int grid_kind, void* output, int n, int channels,
                         int height, int width, int n_points, int padding_mode, int sample_mode, void* stream) {
  msda_host::clear_error();
  int rc = gs_validate(dtype, n, channels, height, width, n_points, grid_kind, padding_mode, sample_mode);
  if (rc != MSDA_OK) return rc;
  if (n == 0 || n_points == 0) return MSDA_OK;
  if (input == nullptr || grid == nullptr || output == nullptr) return fail(MSDA_ERR_INVALID_ARGUMENT, "msda_grid_sample_fwd: NULL tensor pointer");
  const size_t eb = dtype == MSDA_DTYPE_BF16 ? 2 : 4;
  if (!aligned_to(grid, 8) || !aligned_to(input, eb) || !aligned_to(output, eb))
    return fail(MSDA_ERR_INVALID_ARGUMENT, "grid must be 8-byte aligned and input/output aligned to their element size");
  msda::GridSampleParams p = gs_params(input, dtype, grid, grid_kind, n, channels, height, width, n_points, padding_mode, sample_mode);
  p.out = output;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int lds_bytes = 0, cus = 0;
  if ((rc = msda_host::device_attrs(&lds_bytes, &cus)) != MSDA_OK) return rc;
  // Staged when one plane fits in a third of the LDS (three workgroups per CU) and there are enough
  // points per plane to pay for the copy (measured on MI355X, 400 one-channel 112x112 f32 planes:
  // 2352 points 9.4 us staged against 21 us gathered through L2; 784 points 9.4 against 8.2).
  const int budget = std::min(lds_bytes / 3, 64 * 1024);
  const int64_t plane_bytes = static_cast<int64_t>(height) * width * static_cast<int64_t>(eb);
  if (plane_bytes <= budget && static_cast<int64_t>(n_points) * 12 >= static_cast<int64_t>(height) * width &&
      !msda_host::env_flag("MSDA_GS_NO_LDS")) {
    p.fwd_chunk = static_cast<int>(std::min<int64_t>(channels, budget / plane_bytes));
    const int64_t units = static_cast<int64_t>(n) * ((channels + p.fwd_chunk - 1) / p.fwd_chunk);
    // share a (slice, chunk)'s points among workgroups until the grid fills three per CU, each
    // keeping at least 256 points
    const int64_t want = (3 * static_cast<int64_t>(cus) + units - 1) / units;
    p.fwd_split = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(want, n_points / 256)));
    const int64_t groups = units * p.fwd_split;
    if (groups <= 0x7fffffff) {
      const int lds = static_cast<int>(p.fwd_chunk * plane_bytes);
      // 16-byte copies when the input and every plane start on 16 bytes
      p.fwd_vec16 = aligned_to(input, 16) && plane_bytes % 16 == 0;
      static std::atomic<int> granted_f[msda_host::kMaxDevices], granted_b[msda_host::kMaxDevices];
      if (dtype == MSDA_DTYPE_BF16) {
        if ((rc = msda_host::allow_lds(msda::gs_fwd_lds_kernel<msda::bf16_t>, lds, granted_b)) != MSDA_OK) return rc;
        hipLaunchKernelGGL(msda::gs_fwd_lds_kernel<msda::bf16_t>, dim3(static_cast<unsigned>(groups)), dim3(512), lds, st, p);
      } else {
        if ((rc = msda_host::allow_lds(msda::gs_fwd_lds_kernel<float>, lds, granted_f)) != MSDA_OK) return rc;
        hipLaunchKernelGGL(msda::gs_fwd_lds_kernel<float>, dim3(static_cast<unsigned>(groups)), dim3(512), lds, st, p);
      }
      return msda_host::check_launch("grid sample forward (staged)");
    }
  }
  hipLaunchKernelGGL(msda::gs_fwd_kernel, dim3(lane_grid(static_cast<int64_t>(n) * n_points)), dim3(256), 0, st, p);
  return msda_host::check_launch("grid sample forward");
}

int msda_grid_sample_bwd(const void* input, int dtype, const float* grid, int grid_kind, const void* grad_output, void* grad_input,
                         float* grad_grid, int n, int channels, int height, int width, int n_points, int padding_mode,
                         int sample_mode, void* stream) {
  msda_host::clear_error();
  int rc = gs_validate(dtype, n, channels, height, width, n_points, grid_kind, padding_mode, sample_mode);
  if (rc != MSDA_OK) return rc;
  if (n == 0 || (grad_input == nullptr && grad_grid == nullptr)) return MSDA_OK;
  if (n_points > 0 && (grid == nullptr || grad_output == nullptr))
    return fail(MSDA_ERR_INVALID_ARGUMENT, "msda_grid_sample_bwd: NULL tensor pointer");
  if (grad_grid != nullptr && n_points > 0 && input == nullptr) return fail(MSDA_ERR_INVALID_ARGUMENT, "msda_grid_sample_bwd: input is NULL");
  const size_t eb = dtype == MSDA_DTYPE_BF16 ? 2 : 4;
  if (!aligned_to(grid, 8) || !aligned_to(grad_grid, 8) || !aligned_to(input, eb) || !aligned_to(grad_output, eb) ||
      !aligned_to(grad_input, eb))
    return fail(MSDA_ERR_INVALID_ARGUMENT, "grid tensors must be 8-byte aligned and the others aligned to their element size");
  int lds_bytes = 0, cus = 0;
  if (grad_input != nullptr && (rc = msda_host::device_attrs(&lds_bytes, &cus)) != MSDA_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  msda::GridSampleParams p = gs_params(input, dtype, grid, grid_kind, n, channels, height, width, n_points, padding_mode, sample_mode);
  p.gout = grad_output;
  if (grad_input != nullptr) {
    // the accumulator of one workgroup: a chunk of channels x a band of rows, within 64 KB so
    // that several workgroups share a CU; whole planes when they fit
    const int budget = std::min(lds_bytes, 64 * 1024);
    const int64_t row_bytes = static_cast<int64_t>(width) * 4;
    if (row_bytes > budget) return fail(MSDA_ERR_UNSUPPORTED, "width %d exceeds the grad_input accumulator (%d bytes of LDS)", width, budget);
    const int64_t plane_bytes = row_bytes * height;
    if (plane_bytes <= budget) {
      p.band_rows = height;
      p.chunk = static_cast<int>(std::min<int64_t>(channels, budget / plane_bytes));
    } else {
      p.chunk = 1;
      p.band_rows = static_cast<int>(budget / row_bytes);
    }
    // at least four workgroups per CU (measured on MI355X with 400 one-channel 112x112 masks: 400
    // whole-plane workgroups leave CUs idle); each band re-reads the slice's points, which are few
    const int64_t chunks = (channels + p.chunk - 1) / p.chunk;
    const int64_t want_bands = (4 * static_cast<int64_t>(cus) + n * chunks - 1) / std::max<int64_t>(1, n * chunks);
    const int64_t bands_now = (height + p.band_rows - 1) / p.band_rows;
    if (want_bands > bands_now) p.band_rows = static_cast<int>(std::max<int64_t>(1, (height + want_bands - 1) / want_bands));
    const int64_t groups = static_cast<int64_t>(n) * ((channels + p.chunk - 1) / p.chunk) * ((height + p.band_rows - 1) / p.band_rows);
    if (groups > 0x7fffffff) return fail(MSDA_ERR_UNSUPPORTED, "grad_input grid too large");
    p.ginput = grad_input;
    const int lds = static_cast<int>(static_cast<int64_t>(p.chunk) * p.band_rows * row_bytes);
    static std::atomic<int> granted[msda_host::kMaxDevices];
    if ((rc = msda_host::allow_lds(msda::gs_bwd_input_kernel, lds, granted)) != MSDA_OK) return rc;
    hipLaunchKernelGGL(msda::gs_bwd_input_kernel, dim3(static_cast<unsigned>(groups)), dim3(256), lds, st, p);
    if ((rc = msda_host::check_launch("grid sample backward (input)")) != MSDA_OK) return rc;
  }
  if (grad_grid != nullptr && n_points > 0) {
    p.ggrid = grad_grid;
    hipLaunchKernelGGL(msda::gs_bwd_grid_kernel, dim3(lane_grid(static_cast<int64_t>(n) * n_points)), dim3(256), 0, st, p);
    if ((rc = msda_host::check_launch("grid sample backward (grid)")) != MSDA_OK) return rc;
  }
  return MSDA_OK;
}

}  // extern "C"

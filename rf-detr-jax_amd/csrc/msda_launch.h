// msda_launch.h — host-side launchers and kernel dispatch, shared by the translation units that
// instantiate the kernels (one per value dtype and direction, so the build compiles them in
// parallel) and by the C ABI (msda_abi.hip), which sees only the extern declarations below.
#pragma once

#include "msda.h"
#include "msda_band_kernels.h"
#include "msda_gather_kernels.h"
#include "msda_kernels.h"

#include <hip/hip_runtime.h>

#include <atomic>

namespace msda_host {

constexpr int kMaxDevices = 64;

// Defined in msda_abi.hip.
int fail(int code, const char* fmt, ...);  // records the message for msda_last_error(), returns code
void clear_error();                          // at the start of every C-ABI call
int raise_lds_limit(const void* kernel, int bytes, std::atomic<int>* granted);
int check_launch(const char* what);
int device_attrs(int* lds_bytes, int* cus);  // of the current device, cached per device
bool env_flag(const char* name);              // a tuning switch (MSDA_* knob) set to a non-zero integer
int knob(const char* name, int dflt);         // a tuning knob's value, or dflt when unset

inline bool aligned_to(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Allow a kernel instantiation to use more than 64 KB of dynamic LDS (once per instantiation and
// device; `granted` is that instantiation's per-device record).
template <typename K>
int allow_lds(K kernel, int bytes, std::atomic<int> (&granted)[kMaxDevices]) {
  return raise_lds_limit(reinterpret_cast<const void*>(kernel), bytes, granted);
}

template <typename VT, int VEC, int NS, bool STAGED, bool FUSED>
int launch_fwd(const msda::SampleParams& p, int grid, int threads, int lds, hipStream_t stream) {
  static std::atomic<int> granted[kMaxDevices];  // per instantiation
  auto k = msda::fwd_kernel<VT, VEC, NS, STAGED, FUSED>;
  int rc = allow_lds(k, lds, granted);
  if (rc != MSDA_OK) return rc;
  hipLaunchKernelGGL(k, dim3(grid), dim3(threads), lds, stream, p);
  return check_launch("msda forward");
}

template <typename VT, typename GT, int CH, int KD, bool FZ = false>
int launch_bwd_band(const msda::BandParams& p, int grid, int threads, int lds, hipStream_t stream) {
  static std::atomic<int> granted[kMaxDevices];
  auto k = msda::bwd_band_kernel<VT, GT, CH, KD, FZ>;
  int rc = allow_lds(k, lds, granted);
  if (rc != MSDA_OK) return rc;
  hipLaunchKernelGGL(k, dim3(grid), dim3(threads), lds, stream, p);
  return check_launch("msda backward");
}

// Channels per lane of the backward kernel (16, 8, 4, 2 or 1); head_dim 16 and 32 with 8- or
// 16-channel lanes have kernels that know head_dim at compile time.
// fused: the instantiations with the MSDeformAttn prologue and epilogue (8-channel lanes, head_dim
// 16 or 32; the host checks the rest of the conditions).
template <typename VT, typename GT>
int dispatch_bwd_band_g(int ch, const msda::BandParams& p, int grid, int threads, int lds, hipStream_t st, bool fused) {
  if (fused) {
    if (ch == 8 && p.dim == 16) return launch_bwd_band<VT, GT, 8, 16, true>(p, grid, threads, lds, st);
    if (ch == 8 && p.dim == 32) return launch_bwd_band<VT, GT, 8, 32, true>(p, grid, threads, lds, st);
    return fail(MSDA_ERR_UNSUPPORTED, "no fused backward kernel for %d channels per lane, head_dim %d", ch, p.dim);
  }
  switch (ch) {
    case 1: return launch_bwd_band<VT, GT, 1, 0>(p, grid, threads, lds, st);
    case 2: return launch_bwd_band<VT, GT, 2, 0>(p, grid, threads, lds, st);
    case 4: return launch_bwd_band<VT, GT, 4, 0>(p, grid, threads, lds, st);
    case 8:
      if (p.dim == 16) return launch_bwd_band<VT, GT, 8, 16>(p, grid, threads, lds, st);
      if (p.dim == 32) return launch_bwd_band<VT, GT, 8, 32>(p, grid, threads, lds, st);
      return launch_bwd_band<VT, GT, 8, 0>(p, grid, threads, lds, st);
    case 16:
      if (p.dim == 16) return launch_bwd_band<VT, GT, 16, 16>(p, grid, threads, lds, st);
      if (p.dim == 32) return launch_bwd_band<VT, GT, 16, 32>(p, grid, threads, lds, st);
      return launch_bwd_band<VT, GT, 16, 0>(p, grid, threads, lds, st);
  }
  return fail(MSDA_ERR_UNSUPPORTED, "no backward kernel for %d channels per lane", ch);
}

template <typename VT>
int launch_part_sum(const float* part, int nqb, int64_t n, int64_t stride, void* dv, int vec, int grid, hipStream_t st,
                    const float* rpart, float* dref, int heads, int64_t nref) {
  hipLaunchKernelGGL(msda::bwd_part_sum_kernel<VT>, dim3(grid), dim3(256), 0, st, part, nqb, n, stride, static_cast<VT*>(dv), vec,
                     rpart, dref, heads, nref);
  return check_launch("msda backward (partial sums)");
}

template <typename VT>
int dispatch_bwd_band(int ch, const msda::BandParams& p, int grid, int threads, int lds, hipStream_t st, bool fused) {
  return p.gout_bf16 ? dispatch_bwd_band_g<VT, msda::bf16_t>(ch, p, grid, threads, lds, st, fused)
                     : dispatch_bwd_band_g<VT, float>(ch, p, grid, threads, lds, st, fused);
}

template <typename VT, typename GT, int KD, int NT>
int launch_bwd_gather(const msda::GatherParams& p, int grid, int threads, int lds, hipStream_t stream) {
  static std::atomic<int> granted[kMaxDevices];
  auto k = msda::bwd_gather_kernel<VT, GT, KD, NT>;
  int rc = allow_lds(k, lds, granted);
  if (rc != MSDA_OK) return rc;
  hipLaunchKernelGGL(k, dim3(grid), dim3(threads), lds, stream, p);
  return check_launch("msda backward (sorted gather)");
}

// head_dim 16 (up to 1024 threads) or 32 (up to 512: twice the registers per thread).
template <typename VT>
int dispatch_bwd_gather(int dim, bool gout_bf16, const msda::GatherParams& p, int grid, int threads, int lds, hipStream_t st) {
  if (dim == 16)
    return gout_bf16 ? launch_bwd_gather<VT, msda::bf16_t, 16, 1024>(p, grid, threads, lds, st)
                     : launch_bwd_gather<VT, float, 16, 1024>(p, grid, threads, lds, st);
  if (dim == 32)
    return gout_bf16 ? launch_bwd_gather<VT, msda::bf16_t, 32, 512>(p, grid, threads, lds, st)
                     : launch_bwd_gather<VT, float, 32, 512>(p, grid, threads, lds, st);
  return fail(MSDA_ERR_UNSUPPORTED, "no sorted-gather backward for head_dim %d", dim);
}

// Grouped-query forward kernels come in two forms: every level staged in LDS (no L2 gather path)
// or not; NS = 0 handles any sample count and either kind of level.
template <typename VT, int VEC, bool FUSED>
int fwd_ns(int ns, const msda::SampleParams& p, int grid, int threads, int lds, hipStream_t st) {
  const bool staged = p.all_staged != 0;
  switch (ns) {
    case 2: return staged ? launch_fwd<VT, VEC, 2, true, FUSED>(p, grid, threads, lds, st)
                          : launch_fwd<VT, VEC, 2, false, FUSED>(p, grid, threads, lds, st);
    case 4: return staged ? launch_fwd<VT, VEC, 4, true, FUSED>(p, grid, threads, lds, st)
                          : launch_fwd<VT, VEC, 4, false, FUSED>(p, grid, threads, lds, st);
    default: return launch_fwd<VT, VEC, 0, false, FUSED>(p, grid, threads, lds, st);
  }
}

template <typename VT>
int dispatch_fwd(int vec, int ns, bool fused, const msda::SampleParams& p, int grid, int threads, int lds, hipStream_t st) {
  switch (vec) {
    case 1: return fused ? fwd_ns<VT, 1, true>(ns, p, grid, threads, lds, st) : fwd_ns<VT, 1, false>(ns, p, grid, threads, lds, st);
    case 2: return fused ? fwd_ns<VT, 2, true>(ns, p, grid, threads, lds, st) : fwd_ns<VT, 2, false>(ns, p, grid, threads, lds, st);
    case 4: return fused ? fwd_ns<VT, 4, true>(ns, p, grid, threads, lds, st) : fwd_ns<VT, 4, false>(ns, p, grid, threads, lds, st);
    case 8: return fused ? fwd_ns<VT, 8, true>(ns, p, grid, threads, lds, st) : fwd_ns<VT, 8, false>(ns, p, grid, threads, lds, st);
    case 16: return fused ? fwd_ns<VT, 16, true>(ns, p, grid, threads, lds, st) : fwd_ns<VT, 16, false>(ns, p, grid, threads, lds, st);
  }
  return fail(MSDA_ERR_UNSUPPORTED, "no kernel for %d channels per lane", vec);
}

// Instantiated in msda_fwd_f32.hip, msda_fwd_bf16.hip, msda_bwd_f32.hip and msda_bwd_bf16.hip.
extern template int dispatch_fwd<float>(int, int, bool, const msda::SampleParams&, int, int, int, hipStream_t);
extern template int dispatch_fwd<msda::bf16_t>(int, int, bool, const msda::SampleParams&, int, int, int, hipStream_t);
extern template int dispatch_bwd_band<float>(int, const msda::BandParams&, int, int, int, hipStream_t, bool);
extern template int dispatch_bwd_band<msda::bf16_t>(int, const msda::BandParams&, int, int, int, hipStream_t, bool);
extern template int launch_part_sum<float>(const float*, int, int64_t, int64_t, void*, int, int, hipStream_t, const float*, float*, int, int64_t);
extern template int launch_part_sum<msda::bf16_t>(const float*, int, int64_t, int64_t, void*, int, int, hipStream_t, const float*, float*, int, int64_t);
extern template int dispatch_bwd_gather<float>(int, bool, const msda::GatherParams&, int, int, int, hipStream_t);
extern template int dispatch_bwd_gather<msda::bf16_t>(int, bool, const msda::GatherParams&, int, int, int, hipStream_t);

}  // namespace msda_host

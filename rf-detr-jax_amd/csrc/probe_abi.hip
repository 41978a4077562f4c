// probe_abi.hip — LDS probes of the device (read bandwidth, f64 and f32 atomic-add rates), for the
// benchmark's LDS rooflines.
//
// Every wave of every workgroup streams 16-byte LDS reads (ds_read_b128: the 64 lanes of a wave
// read one contiguous 1 KB block per instruction; eight instructions in flight before one wait)
// over a 32 KB buffer. The loads are written as the instructions themselves so that the compiler
// neither narrows nor drops them, and one VALU operation per load folds a 32-bit word of it into
// the result, so the measured rate is the LDS's rather than the vector ALU's.
#include "msda_probe.h"

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeBytes = 32768;  // LDS per workgroup: several workgroups fit a CU

typedef unsigned probe_u4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(kProbeThreads) lds_read_probe_kernel(unsigned* out, int reps) {
  __shared__ __align__(16) unsigned buf[kProbeBytes / 4];
  for (int i = threadIdx.x; i < kProbeBytes / 4; i += kProbeThreads) buf[i] = static_cast<unsigned>(i) * 2654435761u;
  __syncthreads();
  const unsigned lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const unsigned base = static_cast<unsigned>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned*)(buf)));
  unsigned acc = 0;
  unsigned off = (wave * 8192u) & (kProbeBytes - 1);
  for (int r = 0; r < reps; ++r) {
    // eight consecutive 1 KB blocks [off, off + 8 KB), inside the buffer (off is 8 KB aligned)
    const unsigned a = base + off + lane * 16u;
    probe_u4 x0, x1, x2, x3, x4, x5, x6, x7;
    asm volatile(
        "ds_read_b128 %0, %8\n\t"
        "ds_read_b128 %1, %8 offset:1024\n\t"
        "ds_read_b128 %2, %8 offset:2048\n\t"
        "ds_read_b128 %3, %8 offset:3072\n\t"
        "ds_read_b128 %4, %8 offset:4096\n\t"
        "ds_read_b128 %5, %8 offset:5120\n\t"
        "ds_read_b128 %6, %8 offset:6144\n\t"
        "ds_read_b128 %7, %8 offset:7168\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3), "=&v"(x4), "=&v"(x5), "=&v"(x6), "=&v"(x7)
        : "v"(a)
        : "memory");
    acc += x0.x ^ x1.y ^ x2.z ^ x3.w ^ x4.x ^ x5.y ^ x6.z ^ x7.w;
    off = (off + 8192u) & (kProbeBytes - 1);
  }
  out[blockIdx.x * kProbeThreads + threadIdx.x] = acc;
}

// LDS f64 atomic-add rate: every lane adds 1.0 with ds_add_f64 (no return) 16 times per repetition,
// instruction u of a wave to the 64 consecutive doubles [64 u, 64 u + 64) of the wave's 8 KB
// region (the lanes of an instruction cover every bank pair, each address once), then the thread
// writes the sum of 16 of the doubles (the workgroup's total is 256 * 16 * reps).
constexpr int kAtomicUnroll = 16;

__global__ void __launch_bounds__(kProbeThreads) lds_atomic_probe_kernel(double* out, int reps) {
  __shared__ __align__(16) double acc[kProbeThreads * kAtomicUnroll];  // 32 KB
  for (int i = threadIdx.x; i < kProbeThreads * kAtomicUnroll; i += kProbeThreads) acc[i] = 0.0;
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  double* region = acc + wave * 64 * kAtomicUnroll + lane;
  for (int r = 0; r < reps; ++r) {
#pragma unroll
    for (int u = 0; u < kAtomicUnroll; ++u) __hip_atomic_fetch_add(region + 64 * u, 1.0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __syncthreads();
  const double* mine = acc + threadIdx.x * kAtomicUnroll;
  double sum = 0.0;
  for (int i = 0; i < kAtomicUnroll; ++i) sum += mine[i];
  out[blockIdx.x * kProbeThreads + threadIdx.x] = sum;
}

// The same with 32-bit floats (ds_add_f32 through an explicit LDS pointer, the instruction the
// compiler emits for atomicAdd on __shared__ floats): instruction u of a wave adds 1.0f to the 64
// consecutive floats [64 u, 64 u + 64) of the wave's 4 KB region (every bank once). Measured on
// MI355X this instruction is about 20 times slower than ds_add_f64 whatever the addresses, which is
// why grad_value accumulates in f64.
__global__ void __launch_bounds__(kProbeThreads) lds_atomic_f32_probe_kernel(float* out, int reps) {
  __shared__ __align__(16) float acc[kProbeThreads * kAtomicUnroll];  // 16 KB
  for (int i = threadIdx.x; i < kProbeThreads * kAtomicUnroll; i += kProbeThreads) acc[i] = 0.0f;
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __attribute__((address_space(3))) float* region = (__attribute__((address_space(3))) float*)(acc) + wave * 64 * kAtomicUnroll + lane;
  for (int r = 0; r < reps; ++r) {
#pragma unroll
    for (int u = 0; u < kAtomicUnroll; ++u) __hip_atomic_fetch_add(region + 64 * u, 1.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __syncthreads();
  const float* mine = acc + threadIdx.x * kAtomicUnroll;
  float sum = 0.0f;
  for (int i = 0; i < kAtomicUnroll; ++i) sum += mine[i];
  out[blockIdx.x * kProbeThreads + threadIdx.x] = sum;
}

}  // namespace

extern "C" int msda_probe_lds_atomic_f32(float* out, int blocks, int reps, void* stream) {
  if (out == nullptr || blocks < 1 || reps < 1) return -1;
  hipLaunchKernelGGL(lds_atomic_f32_probe_kernel, dim3(blocks), dim3(kProbeThreads), 0, static_cast<hipStream_t>(stream), out, reps);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

extern "C" int msda_probe_lds_atomic(double* out, int blocks, int reps, void* stream) {
  if (out == nullptr || blocks < 1 || reps < 1) return -1;
  hipLaunchKernelGGL(lds_atomic_probe_kernel, dim3(blocks), dim3(kProbeThreads), 0, static_cast<hipStream_t>(stream), out, reps);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

extern "C" int64_t msda_probe_lds_atomic_ops(int blocks, int reps) {
  return static_cast<int64_t>(blocks) * kProbeThreads * reps * kAtomicUnroll;
}

extern "C" int msda_probe_lds_read(unsigned* out, int blocks, int reps, void* stream) {
  if (out == nullptr || blocks < 1 || reps < 1) return -1;
  hipLaunchKernelGGL(lds_read_probe_kernel, dim3(blocks), dim3(kProbeThreads), 0, static_cast<hipStream_t>(stream), out, reps);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

extern "C" int64_t msda_probe_lds_read_bytes(int blocks, int reps) {
  return static_cast<int64_t>(blocks) * kProbeThreads * reps * 8 * 16;
}

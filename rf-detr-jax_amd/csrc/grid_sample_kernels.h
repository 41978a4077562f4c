// grid_sample_kernels.h — gfx950 device code for RF-DETR-JAX's bilinear_grid_sample and
// point_sample (src/rfdetr_jax/models/ops.py:64-134, :189-205; models/heads/segmentation.py:146-186).
//
// Layouts are the reference's: input [N, C, H, W] (channels first), grid [N, P, 2] (P = Hg * Wg;
// either grid coordinates in [-1, 1] or point_sample's points in [0, 1], from which the kernel forms
// grid = 2 p - 1), output [N, C, P].
//
// Kernels:
//  * gs_fwd_lds_kernel — when a channel plane fits in LDS (the segmentation loss's mask logits):
//    one workgroup per (slice, chunk of channels, share of the points) stages the planes in LDS
//    and samples every point from there; out[n, c, p] is written by consecutive lanes.
//  * gs_fwd_kernel — otherwise: one lane per (slice n, point p), the point's corners and weights
//    once, then every channel's four corner values gathered through L2.
//  * gs_bwd_input_kernel — one workgroup per (slice, chunk of channels, band of rows): an f32
//    accumulator for the band's pixels of those channels in LDS, every point of the slice scattered
//    into it (LDS float atomics), then the band written once in the input dtype. grad_input needs
//    no zero-fill and no global atomics; each element has one writer.
//  * gs_bwd_grid_kernel — one lane per point: the gradient of the sample position, summed over
//    channels (bilinear only; nearest sampling has none).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "msda_kernels.h"  // stage_copy, bf16_to_f32, MSDA_LDS

namespace msda {

struct GridSampleParams {
  const void* input;      // [N, C, H, W]
  const float* grid;      // [N, P, 2]
  void* out;              // forward: [N, C, P]
  const void* gout;       // backward: grad_output [N, C, P]
  void* ginput;           // backward: grad_input [N, C, H, W], or null
  float* ggrid;           // backward: grad_grid [N, P, 2], or null
  int bf16;               // input / output / grad dtype is bf16 (else f32)
  int n, c, h, w, points;
  int unit_points;        // grid holds point_sample's [0, 1] points (grid = 2 p - 1 formed here)
  int border;             // padding_mode "border" (else "zeros")
  int nearest;            // nearest sampling (border padding; segmentation.py:173-186)
  int chunk, band_rows;   // gs_bwd_input_kernel: channels and image rows per workgroup
  int fwd_chunk;          // gs_fwd_lds_kernel: channel planes staged per workgroup
  int fwd_split;          // gs_fwd_lds_kernel: workgroups sharing one (slice, chunk)'s points
  int fwd_vec16;          // gs_fwd_lds_kernel: the staged planes may be copied 16 bytes at a time
};

__device__ __forceinline__ float gs_load(const void* base, int64_t i, bool bf16) {
  if (bf16) return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(base)[i]) << 16);
  return static_cast<const float*>(base)[i];
}

__device__ __forceinline__ void gs_store(void* base, int64_t i, float v, bool bf16) {
  if (bf16) {
    uint32_t u = __float_as_uint(v);
    uint16_t r;
    if ((u & 0x7fffffffu) > 0x7f800000u) r = static_cast<uint16_t>((u >> 16) | 0x40u);  // quiet NaN
    else r = static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);          // nearest even
    static_cast<uint16_t*>(base)[i] = r;
  } else {
    static_cast<float*>(base)[i] = v;
  }
}

// One sample position's corners: clipped flat indices in the (H, W) plane, weights (masked for
// zero padding, unmasked for border padding, ops.py:123-132), masks, fractions. Nearest sampling
// uses c00 alone with weight one.
struct GsCorners {
  int c00, c10, c01, c11;
  float w00, w10, w01, w11;
  float m00, m10, m01, m11;
  float fx, fy;
};

// ops.py:83-84: ix = ((g + 1) W - 1) / 2, one IEEE rounding per operation (the division by two
// is exact). point_sample's grid = 2 p - 1 (segmentation.py:166) is rounded once first.
__device__ __forceinline__ float gs_coord(float g, float size, bool unit) {
#pragma clang fp contract(off)
  if (unit) g = 2.0f * g - 1.0f;
  return ((g + 1.0f) * size - 1.0f) * 0.5f;
}

__device__ __forceinline__ GsCorners gs_corners(float gx, float gy, const GridSampleParams& p) {
  GsCorners k;
  const int h = p.h, w = p.w;
  const float ix = gs_coord(gx, static_cast<float>(w), p.unit_points != 0);
  const float iy = gs_coord(gy, static_cast<float>(h), p.unit_points != 0);
  if (p.nearest) {
    // segmentation.py:177-180: round half to even, then clip to the map
    const int xi = static_cast<int>(fminf(fmaxf(rintf(ix), 0.0f), static_cast<float>(w - 1)));
    const int yi = static_cast<int>(fminf(fmaxf(rintf(iy), 0.0f), static_cast<float>(h - 1)));
    k.c00 = k.c10 = k.c01 = k.c11 = yi * w + xi;
    k.w00 = 1.0f;
    k.w10 = k.w01 = k.w11 = 0.0f;
    k.m00 = k.m10 = k.m01 = k.m11 = 0.0f;
    k.fx = k.fy = 0.0f;
    return k;
  }
  const float x0f = floorf(ix), y0f = floorf(iy);
  k.fx = ix - x0f;  // ops.py:88-89
  k.fy = iy - y0f;
  // clamp before the conversion so huge or NaN coordinates stay defined (beyond [-1, size] every
  // corner is out of bounds or clipped to the edge either way)
  const int x0 = static_cast<int>(fminf(fmaxf(x0f, -2.0f), static_cast<float>(w)));
  const int y0 = static_cast<int>(fminf(fmaxf(y0f, -2.0f), static_cast<float>(h)));
  const int x1 = x0 + 1, y1 = y0 + 1;
  const int cx0 = min(max(x0, 0), w - 1), cx1 = min(max(x1, 0), w - 1);
  const int cy0 = min(max(y0, 0), h - 1), cy1 = min(max(y1, 0), h - 1);
  k.c00 = cy0 * w + cx0;
  k.c10 = cy0 * w + cx1;
  k.c01 = cy1 * w + cx0;
  k.c11 = cy1 * w + cx1;
  if (p.border) {
    k.m00 = k.m10 = k.m01 = k.m11 = 1.0f;
  } else {
    const bool mx0 = static_cast<unsigned>(x0) < static_cast<unsigned>(w), mx1 = static_cast<unsigned>(x1) < static_cast<unsigned>(w);
    const bool my0 = static_cast<unsigned>(y0) < static_cast<unsigned>(h), my1 = static_cast<unsigned>(y1) < static_cast<unsigned>(h);
    k.m00 = (mx0 && my0) ? 1.0f : 0.0f;
    k.m10 = (mx1 && my0) ? 1.0f : 0.0f;
    k.m01 = (mx0 && my1) ? 1.0f : 0.0f;
    k.m11 = (mx1 && my1) ? 1.0f : 0.0f;
  }
  const float gxw = 1.0f - k.fx, gyw = 1.0f - k.fy;
  k.w00 = (gxw * gyw) * k.m00;
  k.w10 = (k.fx * gyw) * k.m10;
  k.w01 = (gxw * k.fy) * k.m01;
  k.w11 = (k.fx * k.fy) * k.m11;
  return k;
}

// One lane per (slice, point); n * points < 2^31 (checked on the host), so indices are 32-bit.
__global__ void __launch_bounds__(256) gs_fwd_kernel(const GridSampleParams p) {
  const uint32_t total = static_cast<uint32_t>(p.n) * static_cast<uint32_t>(p.points);
  const int64_t plane = static_cast<int64_t>(p.h) * p.w;
  const bool bf = p.bf16 != 0;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const uint32_t n32 = i / static_cast<uint32_t>(p.points);
    const int64_t n = n32;
    const int pt = static_cast<int>(i - n32 * static_cast<uint32_t>(p.points));
    const float2 g = reinterpret_cast<const float2*>(p.grid)[i];
    const GsCorners k = gs_corners(g.x, g.y, p);
    for (int c = 0; c < p.c; ++c) {
      const int64_t base = (n * p.c + c) * plane;
      float v;
      if (p.nearest) {
        v = gs_load(p.input, base + k.c00, bf);
      } else {
        const float v00 = gs_load(p.input, base + k.c00, bf), v10 = gs_load(p.input, base + k.c10, bf);
        const float v01 = gs_load(p.input, base + k.c01, bf), v11 = gs_load(p.input, base + k.c11, bf);
        v = ((v00 * k.w00 + v10 * k.w10) + v01 * k.w01) + v11 * k.w11;  // corner order of ops.py:133-134
      }
      gs_store(p.out, (n * p.c + c) * p.points + pt, v, bf);
    }
  }
}

// Staged forward: workgroup = (slice n, chunk of channels, share of the points). The chunk's
// planes (consecutive in [N, C, H, W]) are copied into LDS once in the input dtype (stage_copy:
// global_load_lds_dwordx4 when rows allow 16-byte copies), then each lane samples its points from
// LDS: the corner gathers of a wave touch random words, which from L2 would cost a cache line each.
// The workgroups of one slice are consecutive ids, so they run on one XCD and share its L2.
template <typename VT>
__global__ void __launch_bounds__(512) gs_fwd_lds_kernel(const GridSampleParams p) {
  extern __shared__ __align__(16) unsigned char gs_raw[];
  VT* plane_lds = reinterpret_cast<VT*>(gs_raw);
  const int nchunks = (p.c + p.fwd_chunk - 1) / p.fwd_chunk;
  int id = blockIdx.x;
  const int share = id % p.fwd_split;
  id /= p.fwd_split;
  const int chunk = id % nchunks;
  const int n = id / nchunks;
  const int c0 = chunk * p.fwd_chunk, c1 = min(p.c, c0 + p.fwd_chunk);
  const int plane = p.h * p.w;
  const bool bf = p.bf16 != 0;
  const VT* src = static_cast<const VT*>(p.input) + (static_cast<int64_t>(n) * p.c + c0) * plane;
  stage_copy<VT>(plane_lds, src, (c1 - c0) * plane, p.fwd_vec16 != 0);
  __syncthreads();
  const int per = (p.points + p.fwd_split - 1) / p.fwd_split;
  const int pt0 = share * per, pt1 = min(p.points, pt0 + per);
  const float2* grid = reinterpret_cast<const float2*>(p.grid) + static_cast<int64_t>(n) * p.points;
  const MSDA_LDS VT* pl_all = (const MSDA_LDS VT*)(plane_lds);
  auto rd = [&](const MSDA_LDS VT* pl, int i) -> float {
    if constexpr (std::is_same<VT, float>::value) return pl[i];
    else return bf16_to_f32(pl[i]);
  };
  for (int pt = pt0 + threadIdx.x; pt < pt1; pt += blockDim.x) {
    const float2 g = grid[pt];
    const GsCorners k = gs_corners(g.x, g.y, p);
    for (int c = c0; c < c1; ++c) {
      const MSDA_LDS VT* pl = pl_all + (c - c0) * plane;
      float v;
      if (p.nearest) {
        v = rd(pl, k.c00);
      } else {
        v = ((rd(pl, k.c00) * k.w00 + rd(pl, k.c10) * k.w10) + rd(pl, k.c01) * k.w01) + rd(pl, k.c11) * k.w11;
      }
      gs_store(p.out, (static_cast<int64_t>(n) * p.c + c) * p.points + pt, v, bf);
    }
  }
}

// Workgroup = (slice n, channel chunk, row band); LDS: chunk x band_rows x W floats.
__global__ void __launch_bounds__(256) gs_bwd_input_kernel(const GridSampleParams p) {
  extern __shared__ __align__(16) float gs_acc[];
  const int nchunks = (p.c + p.chunk - 1) / p.chunk;
  const int nbands = (p.h + p.band_rows - 1) / p.band_rows;
  int id = blockIdx.x;
  const int band = id % nbands;
  id /= nbands;
  const int chunk = id % nchunks;
  const int n = id / nchunks;
  const int c0 = chunk * p.chunk, c1 = min(p.c, c0 + p.chunk);
  const int r0 = band * p.band_rows, r1 = min(p.h, r0 + p.band_rows);
  const int w = p.w;
  const int band_px = (r1 - r0) * w;
  const int cells = (c1 - c0) * band_px;
  for (int i = threadIdx.x; i < cells; i += blockDim.x) gs_acc[i] = 0.0f;
  __syncthreads();
  const bool bf = p.bf16 != 0;
  const int lo = r0 * w, hi = r1 * w;  // the band's flat pixel range in the plane
  for (int pt = threadIdx.x; pt < p.points; pt += blockDim.x) {
    const float2 g = reinterpret_cast<const float2*>(p.grid)[static_cast<int64_t>(n) * p.points + pt];
    const GsCorners k = gs_corners(g.x, g.y, p);
    for (int c = c0; c < c1; ++c) {
      const float go = gs_load(p.gout, (static_cast<int64_t>(n) * p.c + c) * p.points + pt, bf);
      float* acc = gs_acc + (c - c0) * band_px - lo;
      auto add = [&](int idx, float wt) {
        if (wt != 0.0f && idx >= lo && idx < hi) atomicAdd(acc + idx, wt * go);
      };
      add(k.c00, k.w00);
      if (!p.nearest) {
        add(k.c10, k.w10);
        add(k.c01, k.w01);
        add(k.c11, k.w11);
      }
    }
  }
  __syncthreads();
  const int64_t plane = static_cast<int64_t>(p.h) * w;
  for (int i = threadIdx.x; i < cells; i += blockDim.x) {
    const int cc = i / band_px, px = i - cc * band_px;
    gs_store(p.ginput, (static_cast<int64_t>(n) * p.c + c0 + cc) * plane + lo + px, gs_acc[i], bf);
  }
}

// d out / d ix = gy (m10 v10 - m00 v00) + fy (m11 v11 - m01 v01), and the same for iy; d ix / d g
// = W / 2 (ops.py:83), d g / d p = 2 for point_sample's points. Floor, masks and clipping are
// piecewise constant and contribute nothing.
__global__ void __launch_bounds__(256) gs_bwd_grid_kernel(const GridSampleParams p) {
  const uint32_t total = static_cast<uint32_t>(p.n) * static_cast<uint32_t>(p.points);
  const int64_t plane = static_cast<int64_t>(p.h) * p.w;
  const bool bf = p.bf16 != 0;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const uint32_t n32 = i / static_cast<uint32_t>(p.points);
    const int64_t n = n32;
    const int pt = static_cast<int>(i - n32 * static_cast<uint32_t>(p.points));
    float2 grad = make_float2(0.0f, 0.0f);
    if (!p.nearest) {
      const float2 g = reinterpret_cast<const float2*>(p.grid)[i];
      const GsCorners k = gs_corners(g.x, g.y, p);
      float sx = 0.0f, sy = 0.0f;
      for (int c = 0; c < p.c; ++c) {
        const int64_t base = (n * p.c + c) * plane;
        const float go = gs_load(p.gout, (n * p.c + c) * p.points + pt, bf);
        const float v00 = k.m00 * gs_load(p.input, base + k.c00, bf), v10 = k.m10 * gs_load(p.input, base + k.c10, bf);
        const float v01 = k.m01 * gs_load(p.input, base + k.c01, bf), v11 = k.m11 * gs_load(p.input, base + k.c11, bf);
        sx += go * ((1.0f - k.fy) * (v10 - v00) + k.fy * (v11 - v01));
        sy += go * ((1.0f - k.fx) * (v01 - v00) + k.fx * (v11 - v10));
      }
      const float scale = p.unit_points ? 1.0f : 0.5f;
      grad = make_float2(sx * (static_cast<float>(p.w) * scale), sy * (static_cast<float>(p.h) * scale));
    }
    reinterpret_cast<float2*>(p.ggrid)[i] = grad;
  }
}

}  // namespace msda

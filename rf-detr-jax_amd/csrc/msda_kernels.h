// msda_kernels.h — gfx950 device code for multi-scale deformable attention (forward and VJP).
//
// Semantics follow RF-DETR-JAX's gather sampler, src/rfdetr_jax/models/ops.py:64-134 and
// ops.py:208-292: grid_sample(bilinear, zeros, align_corners=False) of each (batch, head) value
// slice at 2*loc-1, corner order (x0,y0),(x1,y0),(x0,y1),(x1,y1), masked weights multiplied onto
// values read at clipped indices, level-major point sum. Gradients are the VJP of those lines.
//
// Work decomposition (MI355X: 256 CUs in 8 XCDs, 160 KB LDS per CU, 64-lane waves):
//  * Forward: one workgroup per (slice n = b*H+h, chunk of queries). Levels that fit the LDS
//    budget are staged once per workgroup with 16-byte loads; the rest are gathered from global
//    memory (L2). A group of `lpq` adjacent lanes owns one query; each lane owns VEC contiguous
//    channels, so a corner read is one 16-byte LDS/global load per lane.
//  * Backward: one workgroup per (slice, level, band of image rows). The workgroup stages the
//    band's value rows (+1 halo row) and keeps an f32 grad_value accumulator for the band's rows
//    in LDS. It scans every query of its slice: a sample whose floor row lies in the band is
//    "owned" and gets its grad_location / grad_weight computed here (the 4 corner values are all
//    in the staged rows); every sample with a corner row in the band adds that corner's
//    contribution to the LDS accumulator with ds_add_f32. The accumulator is then written to
//    grad_value once, in the value dtype. Each grad element therefore has exactly one writer:
//    no global atomics, no zero-fill pass, no cross-workgroup reduction, and levels larger than
//    LDS are handled by using more bands.
//  * Workgroups are re-numbered so each XCD receives a contiguous range of logical work items;
//    the logical order puts the heads of one (batch, query range) next to each other, so the
//    workgroups that share cache lines of sampling_locations / attention_weights / output (all
//    laid out [B, Q, H, ...]) run on the same XCD and share its L2.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace msda {

constexpr int kMaxLevels = 16;
constexpr int kXcds = 8;  // MI355X: 8 accelerator complex dies, workgroups dispatched round-robin
constexpr int kFwdThreads = 256;
constexpr int kBwdThreads = 512;

using bf16_t = uint16_t;

struct LevelDesc {
  int h, w;        // level height and width
  int start;       // first position of the level in the value slice
  int lds;         // forward: element offset of the staged level in LDS, -1 = read from global memory
  int band_rows;   // backward: image rows per band
  int band_first;  // backward: index of the level's first band among a slice's (level, band) items
};

struct FwdParams {
  const void* value;
  const float* loc;
  const float* attn;
  void* out;
  int out_bf16;
  int heads, dim, queries, levels, points;
  int64_t len_value;
  int lpq_shift;  // log2(lanes per query)
  int qchunk;     // queries per workgroup
  int nqc;        // query chunks per slice
  int vec16;      // staging may use 16-byte vectors
  LevelDesc lv[kMaxLevels];
};

struct BwdParams {
  const void* value;
  const float* loc;
  const float* attn;
  const void* gout;
  void* dvalue;
  float* dloc;
  float* dattn;
  int gout_bf16;
  int heads, dim, queries, levels, points;
  int64_t len_value;
  int lpq_shift;
  int nwork;  // (level, band) items per slice
  int vec16;
  LevelDesc lv[kMaxLevels];
};

// ---------------------------------------------------------------------------------------------
// scalar helpers

__device__ __forceinline__ float bf16_to_f32(bf16_t x) { return __uint_as_float(static_cast<uint32_t>(x) << 16); }

__device__ __forceinline__ bf16_t f32_to_bf16(float f) {  // round to nearest even, quiet NaNs
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<bf16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<bf16_t>(u >> 16);
}

// Map the hardware workgroup id to a logical work item so that each XCD (hardware id mod 8)
// processes one contiguous range of logical ids. A bijection on [0, G) for any G.
__device__ __forceinline__ int xcd_logical(int hw, int G) {
  const int x = hw % kXcds, k = hw / kXcds;
  const int base = G / kXcds, extra = G % kXcds;
  return x * base + min(x, extra) + k;
}

// ops.py:270 then ops.py:83-84: grid = 2*loc - 1; pixel = ((grid + 1) * size - 1) / 2.
// One IEEE rounding per operation (no FMA contraction), as the reference's f32 run computes it,
// so that floor() decides the same cell. Dividing by two is exact, so it is written as * 0.5f.
__device__ __forceinline__ float pixel_coord(float loc, float size) {
#pragma clang fp contract(off)
  const float grid = 2.0f * loc - 1.0f;
  return ((grid + 1.0f) * size - 1.0f) * 0.5f;
}

struct Bilinear {
  int i00, i10, i01, i11;      // clipped flat indices inside the level
  float w00, w10, w01, w11;    // masked corner weights
  float m00, m10, m01, m11;    // in-bounds masks
  float fx, fy;                // fractional parts
  int y0c, y1c;                // clipped rows of the two corner rows
  float y0f;                   // floor of the row coordinate
};

// ops.py:85-128 for one sample position.
__device__ __forceinline__ Bilinear bilinear(float lx, float ly, int h, int w) {
  Bilinear c;
  const float ix = pixel_coord(lx, static_cast<float>(w));
  const float iy = pixel_coord(ly, static_cast<float>(h));
  const float x0f = floorf(ix), y0f = floorf(iy);
  c.fx = ix - x0f;  // rounded in f32 like ops.py:88-89 (inexact only for ix in (-1, 0))
  c.fy = iy - y0f;
  const float gx = 1.0f - c.fx, gy = 1.0f - c.fy;
  // Clamp before the integer conversion so huge or NaN coordinates stay defined; the clamp does
  // not change any in-bounds decision (values below -1 or above size-1 are out of bounds anyway).
  const int x0 = static_cast<int>(fminf(fmaxf(x0f, -2.0f), static_cast<float>(w)));
  const int y0 = static_cast<int>(fminf(fmaxf(y0f, -2.0f), static_cast<float>(h)));
  const int x1 = x0 + 1, y1 = y0 + 1;
  const bool mx0 = static_cast<unsigned>(x0) < static_cast<unsigned>(w);
  const bool mx1 = static_cast<unsigned>(x1) < static_cast<unsigned>(w);
  const bool my0 = static_cast<unsigned>(y0) < static_cast<unsigned>(h);
  const bool my1 = static_cast<unsigned>(y1) < static_cast<unsigned>(h);
  const int cx0 = min(max(x0, 0), w - 1), cx1 = min(max(x1, 0), w - 1);
  const int cy0 = min(max(y0, 0), h - 1), cy1 = min(max(y1, 0), h - 1);
  c.i00 = cy0 * w + cx0;
  c.i10 = cy0 * w + cx1;
  c.i01 = cy1 * w + cx0;
  c.i11 = cy1 * w + cx1;
  c.m00 = (mx0 && my0) ? 1.0f : 0.0f;
  c.m10 = (mx1 && my0) ? 1.0f : 0.0f;
  c.m01 = (mx0 && my1) ? 1.0f : 0.0f;
  c.m11 = (mx1 && my1) ? 1.0f : 0.0f;
  // weight = (wx * wy) * inside, ops.py:123-128 (NaN coordinates give NaN weights, as there)
  c.w00 = (gx * gy) * c.m00;
  c.w10 = (c.fx * gy) * c.m10;
  c.w01 = (gx * c.fy) * c.m01;
  c.w11 = (c.fx * c.fy) * c.m11;
  c.y0c = cy0;
  c.y1c = cy1;
  c.y0f = y0f;
  return c;
}

// ---------------------------------------------------------------------------------------------
// vector loads / stores of VEC channels

template <typename VT, int VEC>
__device__ __forceinline__ void load_vec(const VT* __restrict__ p, float (&o)[VEC]) {
  if constexpr (VEC == 1) {
    if constexpr (std::is_same<VT, float>::value) o[0] = *p;
    else o[0] = bf16_to_f32(*p);
  } else if constexpr (std::is_same<VT, float>::value) {
    typedef float V __attribute__((ext_vector_type(VEC)));
    const V v = *reinterpret_cast<const V*>(p);
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = v[k];
  } else {
    typedef bf16_t V __attribute__((ext_vector_type(VEC)));
    const V v = *reinterpret_cast<const V*>(p);
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = bf16_to_f32(v[k]);
  }
}

template <int VEC>
__device__ __forceinline__ void load_any(const void* base, int64_t off, bool is_bf16, float (&o)[VEC]) {
  if (is_bf16) load_vec<bf16_t, VEC>(static_cast<const bf16_t*>(base) + off, o);
  else load_vec<float, VEC>(static_cast<const float*>(base) + off, o);
}

template <typename VT, int VEC>
__device__ __forceinline__ void store_vec(VT* __restrict__ p, const float (&a)[VEC]) {
  if constexpr (VEC == 1) {
    if constexpr (std::is_same<VT, float>::value) *p = a[0];
    else *p = f32_to_bf16(a[0]);
  } else if constexpr (std::is_same<VT, float>::value) {
    typedef float V __attribute__((ext_vector_type(VEC)));
    V v;
#pragma unroll
    for (int k = 0; k < VEC; ++k) v[k] = a[k];
    *reinterpret_cast<V*>(p) = v;
  } else {
    typedef bf16_t V __attribute__((ext_vector_type(VEC)));
    V v;
#pragma unroll
    for (int k = 0; k < VEC; ++k) v[k] = f32_to_bf16(a[k]);
    *reinterpret_cast<V*>(p) = v;
  }
}

template <int VEC>
__device__ __forceinline__ void store_any(void* base, int64_t off, bool is_bf16, const float (&a)[VEC]) {
  if (is_bf16) store_vec<bf16_t, VEC>(static_cast<bf16_t*>(base) + off, a);
  else store_vec<float, VEC>(static_cast<float*>(base) + off, a);
}

// Cooperative copy global -> LDS of `count` elements (16-byte vectors when allowed).
template <typename VT>
__device__ __forceinline__ void stage_copy(VT* dst, const VT* __restrict__ src, int count, bool vec16) {
  if (vec16) {
    const int n16 = static_cast<int>((static_cast<int64_t>(count) * sizeof(VT)) / 16);
    const uint4* s = reinterpret_cast<const uint4*>(src);
    uint4* d = reinterpret_cast<uint4*>(dst);
    for (int i = threadIdx.x; i < n16; i += blockDim.x) d[i] = s[i];
  } else {
    for (int i = threadIdx.x; i < count; i += blockDim.x) dst[i] = src[i];
  }
}

__device__ __forceinline__ float group_sum(float v, int lpq) {
  for (int o = 1; o < lpq; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ---------------------------------------------------------------------------------------------
// forward

template <typename VT, int VEC>
__global__ void __launch_bounds__(kFwdThreads) fwd_kernel(const FwdParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  VT* lds = reinterpret_cast<VT*>(lds_raw);

  const int lid = xcd_logical(blockIdx.x, gridDim.x);
  const int h = lid % p.heads;
  const int rest = lid / p.heads;
  const int qc = rest % p.nqc;
  const int b = rest / p.nqc;
  const int64_t n = static_cast<int64_t>(b) * p.heads + h;
  const VT* __restrict__ vs = static_cast<const VT*>(p.value) + n * p.len_value * p.dim;

  for (int l = 0; l < p.levels; ++l) {
    const LevelDesc L = p.lv[l];
    if (L.lds >= 0) stage_copy(lds + L.lds, vs + static_cast<int64_t>(L.start) * p.dim, L.h * L.w * p.dim, p.vec16);
  }
  __syncthreads();

  const int lpq = 1 << p.lpq_shift;
  const int j = threadIdx.x & (lpq - 1);
  const int slot = threadIdx.x >> p.lpq_shift;
  const int nslots = blockDim.x >> p.lpq_shift;
  const bool lane_on = j * VEC < p.dim;
  const int c0 = lane_on ? j * VEC : 0;
  const int LP = p.levels * p.points;
  const int q_lo = qc * p.qchunk;
  const int q_hi = min(p.queries, q_lo + p.qchunk);

  for (int q = q_lo + slot; q < q_hi; q += nslots) {
    const int64_t bqh = (static_cast<int64_t>(b) * p.queries + q) * p.heads + h;
    const float* __restrict__ lq = p.loc + bqh * LP * 2;
    const float* __restrict__ aq = p.attn + bqh * LP;
    float acc[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc[k] = 0.0f;
    for (int l = 0; l < p.levels; ++l) {
      const LevelDesc L = p.lv[l];
      for (int pt = 0; pt < p.points; ++pt) {
        const int s = l * p.points + pt;
        const float2 xy = *reinterpret_cast<const float2*>(lq + 2 * s);
        const float a = aq[s];
        const Bilinear c = bilinear(xy.x, xy.y, L.h, L.w);
        float v00[VEC], v10[VEC], v01[VEC], v11[VEC];
        if (L.lds >= 0) {
          const VT* base = lds + L.lds + c0;
          load_vec<VT, VEC>(base + c.i00 * p.dim, v00);
          load_vec<VT, VEC>(base + c.i10 * p.dim, v10);
          load_vec<VT, VEC>(base + c.i01 * p.dim, v01);
          load_vec<VT, VEC>(base + c.i11 * p.dim, v11);
        } else {
          const VT* base = vs + static_cast<int64_t>(L.start) * p.dim + c0;
          load_vec<VT, VEC>(base + static_cast<int64_t>(c.i00) * p.dim, v00);
          load_vec<VT, VEC>(base + static_cast<int64_t>(c.i10) * p.dim, v10);
          load_vec<VT, VEC>(base + static_cast<int64_t>(c.i01) * p.dim, v01);
          load_vec<VT, VEC>(base + static_cast<int64_t>(c.i11) * p.dim, v11);
        }
#pragma unroll
        for (int k = 0; k < VEC; ++k)
          acc[k] += a * (v00[k] * c.w00 + v10[k] * c.w10 + v01[k] * c.w01 + v11[k] * c.w11);
      }
    }
    if (lane_on) store_any<VEC>(p.out, bqh * p.dim + c0, p.out_bf16 != 0, acc);
  }
}

// ---------------------------------------------------------------------------------------------
// backward

template <typename VT, int VEC>
__global__ void __launch_bounds__(kBwdThreads) bwd_kernel(const BwdParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];

  const int lid = xcd_logical(blockIdx.x, gridDim.x);
  const int h = lid % p.heads;
  const int rest = lid / p.heads;
  const int wk = rest % p.nwork;
  const int b = rest / p.nwork;
  int l = 0;
  while (l + 1 < p.levels && wk >= p.lv[l + 1].band_first) ++l;
  const LevelDesc L = p.lv[l];
  const int r0 = (wk - L.band_first) * L.band_rows;  // band rows [r0, r1); staged rows [r0, rs1)
  const int r1 = min(L.h, r0 + L.band_rows);
  const int rs1 = min(L.h, r1 + 1);
  const int rowlen = L.w * p.dim;
  const int64_t n = static_cast<int64_t>(b) * p.heads + h;
  const int64_t band_off = (n * p.len_value + L.start + static_cast<int64_t>(r0) * L.w) * p.dim;

  VT* sv = reinterpret_cast<VT*>(lds_raw);
  const int nstage = (rs1 - r0) * rowlen;
  const int stage_bytes = ((nstage * static_cast<int>(sizeof(VT))) + 15) & ~15;
  float* acc = reinterpret_cast<float*>(lds_raw + stage_bytes);
  const int nacc = (r1 - r0) * rowlen;
  const bool want_dv = p.dvalue != nullptr;

  stage_copy(sv, static_cast<const VT*>(p.value) + band_off, nstage, p.vec16);
  if (want_dv) {
    for (int i = threadIdx.x; i < nacc; i += blockDim.x) acc[i] = 0.0f;
  }
  __syncthreads();

  const int lpq = 1 << p.lpq_shift;
  const int j = threadIdx.x & (lpq - 1);
  const int slot = threadIdx.x >> p.lpq_shift;
  const int nslots = blockDim.x >> p.lpq_shift;
  const bool lane_on = j * VEC < p.dim;
  const int c0 = lane_on ? j * VEC : 0;
  const int LP = p.levels * p.points;
  const int band_base = r0 * L.w;  // flat index of the band's first pixel inside the level
  const float fw = static_cast<float>(L.w), fh = static_cast<float>(L.h);
  const bool gbf = p.gout_bf16 != 0;

  for (int q = slot; q < p.queries; q += nslots) {
    const int64_t bqh = (static_cast<int64_t>(b) * p.queries + q) * p.heads + h;
    const int64_t s0 = bqh * LP + l * p.points;
    float g[VEC];
    bool have_g = false;
    for (int pt = 0; pt < p.points; ++pt) {
      const float2 xy = *reinterpret_cast<const float2*>(p.loc + 2 * (s0 + pt));
      const Bilinear c = bilinear(xy.x, xy.y, L.h, L.w);
      // The owner band of a sample is the one holding its floor row, clamped into the level
      // (NaN -> row 0); both of its clipped corner rows are then among the staged rows.
      const int yo = static_cast<int>(fminf(fmaxf(c.y0f, 0.0f), fh - 1.0f));
      const bool own = yo >= r0 && yo < r1;
      const bool in0 = c.y0c >= r0 && c.y0c < r1;
      const bool in1 = c.y1c >= r0 && c.y1c < r1;
      const bool touch = want_dv && ((in0 && (c.w00 != 0.0f || c.w10 != 0.0f)) ||
                                     (in1 && (c.w01 != 0.0f || c.w11 != 0.0f)));
      if (!own && !touch) continue;
      const float a = p.attn[s0 + pt];
      if (!have_g) {
        load_any<VEC>(p.gout, bqh * p.dim + c0, gbf, g);
        if (!lane_on) {
#pragma unroll
          for (int k = 0; k < VEC; ++k) g[k] = 0.0f;
        }
        have_g = true;
      }
      if (own) {
        float v00[VEC], v10[VEC], v01[VEC], v11[VEC];
        const VT* base = sv + c0;
        load_vec<VT, VEC>(base + (c.i00 - band_base) * p.dim, v00);
        load_vec<VT, VEC>(base + (c.i10 - band_base) * p.dim, v10);
        load_vec<VT, VEC>(base + (c.i01 - band_base) * p.dim, v01);
        load_vec<VT, VEC>(base + (c.i11 - band_base) * p.dim, v11);
        const float gx = 1.0f - c.fx, gy = 1.0f - c.fy;
        float da = 0.0f, dx = 0.0f, dy = 0.0f;
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          const float m00 = v00[k] * c.m00, m10 = v10[k] * c.m10, m01 = v01[k] * c.m01, m11 = v11[k] * c.m11;
          const float smp = v00[k] * c.w00 + v10[k] * c.w10 + v01[k] * c.w01 + v11[k] * c.w11;
          da += g[k] * smp;
          dx += g[k] * (gy * (m10 - m00) + c.fy * (m11 - m01));
          dy += g[k] * (gx * (m01 - m00) + c.fx * (m11 - m10));
        }
        da = group_sum(da, lpq);
        dx = group_sum(dx, lpq);
        dy = group_sum(dy, lpq);
        if (j == 0) {
          if (p.dattn) p.dattn[s0 + pt] = da;
          if (p.dloc) *reinterpret_cast<float2*>(p.dloc + 2 * (s0 + pt)) = make_float2(a * fw * dx, a * fh * dy);
        }
      }
      if (touch && lane_on) {
        float* arow;
        if (in0) {
          if (c.w00 != 0.0f) {
            const float aw = a * c.w00;
            arow = acc + (c.i00 - band_base) * p.dim + c0;
#pragma unroll
            for (int k = 0; k < VEC; ++k) atomicAdd(arow + k, aw * g[k]);
          }
          if (c.w10 != 0.0f) {
            const float aw = a * c.w10;
            arow = acc + (c.i10 - band_base) * p.dim + c0;
#pragma unroll
            for (int k = 0; k < VEC; ++k) atomicAdd(arow + k, aw * g[k]);
          }
        }
        if (in1) {
          if (c.w01 != 0.0f) {
            const float aw = a * c.w01;
            arow = acc + (c.i01 - band_base) * p.dim + c0;
#pragma unroll
            for (int k = 0; k < VEC; ++k) atomicAdd(arow + k, aw * g[k]);
          }
          if (c.w11 != 0.0f) {
            const float aw = a * c.w11;
            arow = acc + (c.i11 - band_base) * p.dim + c0;
#pragma unroll
            for (int k = 0; k < VEC; ++k) atomicAdd(arow + k, aw * g[k]);
          }
        }
      }
    }
  }

  if (want_dv) {
    __syncthreads();
    VT* dst = static_cast<VT*>(p.dvalue) + band_off;
    if constexpr (std::is_same<VT, float>::value) {
      for (int i = threadIdx.x; i < nacc; i += blockDim.x) dst[i] = acc[i];
    } else {
      for (int i = threadIdx.x; i < nacc; i += blockDim.x) dst[i] = f32_to_bf16(acc[i]);
    }
  }
}

}  // namespace msda

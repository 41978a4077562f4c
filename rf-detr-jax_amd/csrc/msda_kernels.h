// msda_kernels.h — gfx950 device code for multi-scale deformable attention (forward and VJP).
//
// Semantics follow RF-DETR-JAX's gather sampler, src/rfdetr_jax/models/ops.py:64-134 and
// ops.py:208-292: grid_sample(bilinear, zeros, align_corners=False) of each (batch, head) value
// slice at 2*loc-1, corner order (x0,y0),(x1,y0),(x0,y1),(x1,y1), masked weights multiplied onto
// values read at clipped indices, level-major point sum. Gradients are the VJP of those lines.
//
// Measured on MI355X (per CU): random 64-byte-row ds_read_b128 gathers run at ~220 B/clk (close to
// the ~260 B/clk of contiguous reads), random ds_write_b128 at ~66 B/clk, ds_add_f32 at one lane
// per ~3 cycles, and device-wide f32 atomics to L2 at ~1.3 TB/s. The design therefore gathers from
// LDS freely, never uses atomics, and keeps every lane busy with useful work:
//
//  * Forward: one workgroup per (slice n = b*H+h, chunk of queries). The levels that fit the LDS
//    budget and the chunk's sampling locations / weights are staged into LDS with all global loads
//    in flight at once; levels that do not fit are gathered through L2. Each group of `lpq` lanes
//    (normally one lane) owns a query and VEC channels of it, and computes each sample position
//    once.
//  * Backward: one workgroup per (slice, level, band of image rows). It stages the band's value
//    rows (+1 halo row) and keeps one f32 grad_value accumulator per wave for the band. Each wave
//    scans queries with one lane per query, computing only the row of each sample to decide
//    whether the query matters to this band; the relevant queries are compacted (ballot + mbcnt)
//    into a per-wave ring of records, which is processed one record per lane group once a full
//    wave of records is available. A sample whose floor row lies in the band is "owned": its
//    grad_location / grad_weight are computed here from the staged rows. Every sample with a
//    corner row in the band adds a * w_c * g to its wave's accumulator. At the end the wave
//    accumulators are summed and written once, in the value dtype: each grad element has one
//    writer, with no atomics, no zero-fill pass and no cross-workgroup reduction.
//  * Inside a wave, lane groups that target the same accumulator pixel in the same step are
//    serialised by a write-tag / read-back round (write own id to the pixel's tag, read it back,
//    the surviving id does a plain read-modify-write, the others retry). LDS instructions of one
//    wave execute in order, so every round sees the previous round's writes.
//  * Workgroups are re-numbered so each XCD receives a contiguous range of logical work items;
//    the heads of one (batch, query range) are adjacent in that order, so the workgroups that
//    share cache lines of sampling_locations / attention_weights / output / grad_output (all laid
//    out [B, Q, H, ...]) run on the same XCD and share its L2.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace msda {

constexpr int kMaxLevels = 16;
constexpr int kXcds = 8;  // MI355X: 8 accelerator complex dies, workgroups dispatched round-robin
constexpr int kFwdThreads = 256;
constexpr int kBwdThreads = 256;

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
  int vec16;      // value staging may use 16-byte vectors
  int loc_lds;    // byte offset of the staged locations/weights in LDS, -1 = read them from global memory
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
  int lpq_shift;  // log2(lanes per sample) in the owner pass
  int nwork;      // (level, band) items per slice
  int vec16;
  int chunk_m;    // relevant queries whose inputs are staged in LDS at a time
  int scan_seg;   // queries scanned per segment (capacity of the relevant-query list)
  int g_vec4;     // grad_output rows may be read 4 channels at a time
  LevelDesc lv[kMaxLevels];
};

// LDS carve-up of one backward workgroup; shared by the host planner and the kernel so both
// agree on the size. Every region starts on a 16-byte boundary.
struct BwdLayout {
  int sv, acc, cnt, off, misc, rel, cg, cl, ca, skey, srank, swt, rslot, rw, total;
};

__host__ __device__ inline int bwd_align16(int x) { return (x + 15) & ~15; }

__host__ __device__ inline BwdLayout bwd_layout(int staged_rows, int band_rows, int w, int dim, int vbytes, int points,
                                                int chunk_m, int scan_seg) {
  BwdLayout L;
  const int ncell = (band_rows + 1) * (w + 1);
  const int ns = chunk_m * points;  // samples per chunk
  int o = 0;
  L.sv = o;    o += bwd_align16(staged_rows * w * dim * vbytes);
  L.acc = o;   o += bwd_align16(band_rows * w * dim * 4);
  L.cnt = o;   o += bwd_align16(ncell * 4);
  L.off = o;   o += bwd_align16((ncell + 1) * 4);
  L.misc = o;  o += 64;
  L.rel = o;   o += bwd_align16(scan_seg * 2);
  L.cg = o;    o += bwd_align16(chunk_m * dim * 4);
  L.cl = o;    o += bwd_align16(ns * 8);
  L.ca = o;    o += bwd_align16(ns * 4);
  L.skey = o;  o += bwd_align16(ns * 4);
  L.srank = o; o += bwd_align16(ns * 4);
  L.swt = o;   o += bwd_align16(ns * 16);
  L.rslot = o; o += bwd_align16(ns * 4);
  L.rw = o;    o += bwd_align16(ns * 16);
  L.total = o;
  return L;
}

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
// vector loads / stores of VEC channels (at most 16-byte alignment is assumed, so VEC*size > 16
// becomes several 16-byte accesses)

template <typename T, int N>
struct VecT {
  static constexpr int kAlign = (N * sizeof(T) < 16) ? N * sizeof(T) : 16;
  typedef T type __attribute__((ext_vector_type(N), aligned(kAlign)));
};

template <typename VT, int VEC>
__device__ __forceinline__ void load_vec(const VT* __restrict__ p, float (&o)[VEC]) {
  if constexpr (VEC == 1) {
    if constexpr (std::is_same<VT, float>::value) o[0] = *p;
    else o[0] = bf16_to_f32(*p);
  } else if constexpr (std::is_same<VT, float>::value) {
    const typename VecT<float, VEC>::type v = *reinterpret_cast<const typename VecT<float, VEC>::type*>(p);
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = v[k];
  } else {
    const typename VecT<bf16_t, VEC>::type v = *reinterpret_cast<const typename VecT<bf16_t, VEC>::type*>(p);
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
    typename VecT<float, VEC>::type v;
#pragma unroll
    for (int k = 0; k < VEC; ++k) v[k] = a[k];
    *reinterpret_cast<typename VecT<float, VEC>::type*>(p) = v;
  } else {
    typename VecT<bf16_t, VEC>::type v;
#pragma unroll
    for (int k = 0; k < VEC; ++k) v[k] = f32_to_bf16(a[k]);
    *reinterpret_cast<typename VecT<bf16_t, VEC>::type*>(p) = v;
  }
}

template <int VEC>
__device__ __forceinline__ void store_any(void* base, int64_t off, bool is_bf16, const float (&a)[VEC]) {
  if (is_bf16) store_vec<bf16_t, VEC>(static_cast<bf16_t*>(base) + off, a);
  else store_vec<float, VEC>(static_cast<float*>(base) + off, a);
}

// Cooperative copy global -> LDS of `count` elements. Each thread issues a batch of loads before
// any store, so the copy is bounded by bandwidth rather than by one load latency per step.
template <typename VT>
__device__ __forceinline__ void stage_copy(VT* dst, const VT* __restrict__ src, int count, bool vec16) {
  constexpr int U = 8;
  const int nt = blockDim.x;
  if (vec16) {
    const int n16 = static_cast<int>((static_cast<int64_t>(count) * sizeof(VT)) / 16);
    const uint4* s = reinterpret_cast<const uint4*>(src);
    uint4* d = reinterpret_cast<uint4*>(dst);
    int i = threadIdx.x;
    for (; i + (U - 1) * nt < n16; i += U * nt) {
      uint4 r[U];
#pragma unroll
      for (int u = 0; u < U; ++u) r[u] = s[i + u * nt];
#pragma unroll
      for (int u = 0; u < U; ++u) d[i + u * nt] = r[u];
    }
    for (; i < n16; i += nt) d[i] = s[i];
  } else {
    int i = threadIdx.x;
    for (; i + (U - 1) * nt < count; i += U * nt) {
      VT r[U];
#pragma unroll
      for (int u = 0; u < U; ++u) r[u] = src[i + u * nt];
#pragma unroll
      for (int u = 0; u < U; ++u) dst[i + u * nt] = r[u];
    }
    for (; i < count; i += nt) dst[i] = src[i];
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
  const int LP = p.levels * p.points;
  const int q_lo = qc * p.qchunk;
  const int q_hi = min(p.queries, q_lo + p.qchunk);

  // The chunk's sampling locations [q][LP] (float2) and weights [q][LP], contiguous per query in
  // LDS. Their loads are issued first, in batches held in registers, so they overlap the value
  // staging below; the LDS stores happen after it.
  const bool loc_in_lds = p.loc_lds >= 0;
  float2* sl = reinterpret_cast<float2*>(lds_raw + (loc_in_lds ? p.loc_lds : 0));
  float* sa = reinterpret_cast<float*>(sl + p.qchunk * LP);
  constexpr int UL = 4;
  const int nt = blockDim.x;
  const int E = loc_in_lds ? (q_hi - q_lo) * LP : 0;
  const int64_t row0 = (static_cast<int64_t>(b) * p.queries + q_lo) * p.heads + h;
  const float2* lsrc = reinterpret_cast<const float2*>(p.loc) + row0 * LP;
  const float* asrc = p.attn + row0 * LP;
  const int64_t qstride = static_cast<int64_t>(p.heads) * LP;  // samples between consecutive queries
  float2 rl[UL];
  float ra[UL];
#pragma unroll
  for (int u = 0; u < UL; ++u) {
    const int i = threadIdx.x + u * nt;
    if (i < E) {
      const int qq = i / LP, k = i - qq * LP;
      rl[u] = lsrc[qq * qstride + k];
      ra[u] = asrc[qq * qstride + k];
    }
  }
  for (int l = 0; l < p.levels; ++l) {
    const LevelDesc L = p.lv[l];
    if (L.lds >= 0) stage_copy(lds + L.lds, vs + static_cast<int64_t>(L.start) * p.dim, L.h * L.w * p.dim, p.vec16);
  }
#pragma unroll
  for (int u = 0; u < UL; ++u) {
    const int i = threadIdx.x + u * nt;
    if (i < E) {
      sl[i] = rl[u];
      sa[i] = ra[u];
    }
  }
  for (int base = threadIdx.x + UL * nt; base < E; base += UL * nt) {  // chunks larger than UL * nt
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      const int i = base + u * nt;
      if (i < E) {
        const int qq = i / LP, k = i - qq * LP;
        rl[u] = lsrc[qq * qstride + k];
        ra[u] = asrc[qq * qstride + k];
      }
    }
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      const int i = base + u * nt;
      if (i < E) {
        sl[i] = rl[u];
        sa[i] = ra[u];
      }
    }
  }
  __syncthreads();

  const int lpq = 1 << p.lpq_shift;
  const int j = threadIdx.x & (lpq - 1);
  const int slot = threadIdx.x >> p.lpq_shift;
  const int nslots = blockDim.x >> p.lpq_shift;
  const bool lane_on = j * VEC < p.dim;
  const int c0 = lane_on ? j * VEC : 0;

  for (int q = q_lo + slot; q < q_hi; q += nslots) {
    const int64_t bqh = (static_cast<int64_t>(b) * p.queries + q) * p.heads + h;
    const float2* lq = loc_in_lds ? sl + (q - q_lo) * LP : reinterpret_cast<const float2*>(p.loc) + bqh * LP;
    const float* aq = loc_in_lds ? sa + (q - q_lo) * LP : p.attn + bqh * LP;
    float acc[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc[k] = 0.0f;
    for (int l = 0; l < p.levels; ++l) {
      const LevelDesc L = p.lv[l];
      for (int pt = 0; pt < p.points; ++pt) {
        const int s = l * p.points + pt;
        const float2 xy = lq[s];
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
        const float a00 = a * c.w00, a10 = a * c.w10, a01 = a * c.w01, a11 = a * c.w11;
#pragma unroll
        for (int k = 0; k < VEC; ++k) acc[k] += v00[k] * a00 + v10[k] * a10 + v01[k] * a01 + v11[k] * a11;
      }
    }
    if (lane_on) store_any<VEC>(p.out, bqh * p.dim + c0, p.out_bf16 != 0, acc);
  }
}

// ---------------------------------------------------------------------------------------------
// backward
//
// One workgroup per (slice, level, band of rows [r0, r1)). Phases:
//  0. stage the band's value rows (+1 halo row); zero the f32 accumulator of the band's pixels.
//  1. scan: the row coordinate of every sample of the slice on this level is loaded (all loads of
//     a round in flight) and tested against the band; queries with a relevant sample are
//     compacted into a list (ballot per wave, one LDS atomic per wave to reserve space).
//  2. per chunk of `chunk_m` listed queries:
//     a. stage grad_output rows, locations and weights of the chunk into LDS;
//     b. one lane group per sample: owned samples (floor row in the band) get their grad_weight
//        and grad_location from the staged value rows; samples with a corner pixel in the band
//        are bucketed by bilinear cell (x0, y0): ds_add_rtn_u32 on the cell's count gives the
//        sample's rank inside the cell;
//     c. exclusive scan of the cell counts (cells are ordered row-major);
//     d. samples are written into cell order;
//     e. pixel-major gather: one lane per (band pixel, 4 channels) sums, in registers, a * w_k * g
//        over the samples of the four cells that have this pixel as corner k, and adds the sum to
//        its own accumulator slot. Every accumulator element has exactly one writer per chunk.
//  3. the accumulator is written to grad_value in the value dtype.
// Integer LDS atomics are cheap on gfx950 (~10 lanes/clk); float ones are not, and none are used.

// Exclusive prefix sum of cnt[0, n) into off[0, n] (off[n] = total); block-wide, ends in a barrier.
// cnt is cleared for reuse. `tmp` holds one int per wave.
__device__ __forceinline__ void block_scan_counts(int* cnt, int* off, int n, int* tmp) {
  const int nt = blockDim.x, t = threadIdx.x, lane = t & 63;
  const int per = (n + nt - 1) / nt;
  const int b0 = min(n, t * per), b1 = min(n, b0 + per);
  int sum = 0;
  for (int i = b0; i < b1; ++i) sum += cnt[i];
  int incl = sum;
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  if (lane == 63) tmp[t >> 6] = incl;
  __syncthreads();
  int run = incl - sum;
  for (int w = 0; w < (t >> 6); ++w) run += tmp[w];
  for (int i = b0; i < b1; ++i) {
    off[i] = run;
    run += cnt[i];
    cnt[i] = 0;
  }
  if (t == nt - 1) off[n] = run;
  __syncthreads();
}

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
  const int W = L.w;
  const int r0 = (wk - L.band_first) * L.band_rows;  // band rows [r0, r1); staged rows [r0, rs1)
  const int r1 = min(L.h, r0 + L.band_rows);
  const int rs1 = min(L.h, r1 + 1);
  const int rb = r1 - r0;
  const int D = p.dim;
  const int P = p.points;
  const int LP = p.levels * P;
  const int Q = p.queries;
  const int ncell = (rb + 1) * (W + 1);
  const int64_t n = static_cast<int64_t>(b) * p.heads + h;
  const int64_t band_off = (n * p.len_value + L.start + static_cast<int64_t>(r0) * W) * D;
  const int nt = blockDim.x, t = threadIdx.x, lane = t & 63;

  const BwdLayout lay = bwd_layout(rs1 - r0, rb, W, D, static_cast<int>(sizeof(VT)), P, p.chunk_m, p.scan_seg);
  VT* sv = reinterpret_cast<VT*>(lds_raw + lay.sv);
  float* acc = reinterpret_cast<float*>(lds_raw + lay.acc);
  int* cnt = reinterpret_cast<int*>(lds_raw + lay.cnt);
  int* off = reinterpret_cast<int*>(lds_raw + lay.off);
  int* misc = reinterpret_cast<int*>(lds_raw + lay.misc);  // [0] list size, [4..] scan scratch
  uint16_t* rel = reinterpret_cast<uint16_t*>(lds_raw + lay.rel);
  float* cg = reinterpret_cast<float*>(lds_raw + lay.cg);
  float2* cl = reinterpret_cast<float2*>(lds_raw + lay.cl);
  float* ca = reinterpret_cast<float*>(lds_raw + lay.ca);
  int* skey = reinterpret_cast<int*>(lds_raw + lay.skey);
  int* srank = reinterpret_cast<int*>(lds_raw + lay.srank);
  float4* swt = reinterpret_cast<float4*>(lds_raw + lay.swt);
  int* rslot = reinterpret_cast<int*>(lds_raw + lay.rslot);
  float4* rw = reinterpret_cast<float4*>(lds_raw + lay.rw);

  const bool want_dv = p.dvalue != nullptr;
  const bool want_dl = p.dloc != nullptr || p.dattn != nullptr;
  const float fw = static_cast<float>(W), fh = static_cast<float>(L.h);
  const int64_t qstride = static_cast<int64_t>(p.heads) * LP;                    // samples between queries
  const int64_t srow0 = (static_cast<int64_t>(b) * Q * p.heads + h) * LP + l * P;  // sample (q=0, pt=0)
  const float2* loc2 = reinterpret_cast<const float2*>(p.loc);
  const bool gbf = p.gout_bf16 != 0;

  // ---- phase 0
  stage_copy(sv, static_cast<const VT*>(p.value) + band_off, (rs1 - r0) * W * D, p.vec16);
  {
    const int na = rb * W * D;
    float4* a4 = reinterpret_cast<float4*>(acc);
    for (int i = t; i < (na >> 2); i += nt) a4[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int i = (na & ~3) + t; i < na; i += nt) acc[i] = 0.0f;
    for (int i = t; i < ncell; i += nt) cnt[i] = 0;
  }

  const int lpq = 1 << p.lpq_shift;
  const int j = t & (lpq - 1);
  const bool lane_on = j * VEC < D;
  const int c0 = lane_on ? j * VEC : 0;
  const int ngroups = nt >> p.lpq_shift;
  const int M = p.chunk_m;
  constexpr int kSQ = 8;  // queries per thread per scan round
  constexpr int kSP = 4;  // points per load batch in the scan

  for (int qs = 0; qs < Q; qs += p.scan_seg) {
    const int qe = min(Q, qs + p.scan_seg);
    if (t == 0) misc[0] = 0;
    __syncthreads();
    // ---- phase 1: scan [qs, qe)
    for (int qb = qs; qb < qe; qb += kSQ * nt) {
      bool relq[kSQ];
#pragma unroll
      for (int k = 0; k < kSQ; ++k) relq[k] = false;
      for (int pg = 0; pg < P; pg += kSP) {
        float ys[kSQ][kSP];
#pragma unroll
        for (int k = 0; k < kSQ; ++k) {
          const int q = qb + t + k * nt;
#pragma unroll
          for (int e = 0; e < kSP; ++e) {
            const int pt = pg + e;
            ys[k][e] = (q < qe && pt < P) ? p.loc[2 * (srow0 + static_cast<int64_t>(q) * qstride + pt) + 1] : -1.0e30f;
          }
        }
#pragma unroll
        for (int k = 0; k < kSQ; ++k) {
#pragma unroll
          for (int e = 0; e < kSP; ++e) {
            // rows [y0, y0+1] clipped into the level (NaN -> row 0) against the band
            const float y0f = floorf(pixel_coord(ys[k][e], fh));
            const float lo = fminf(fmaxf(y0f, 0.0f), fh - 1.0f);
            const float hi = fminf(fmaxf(y0f + 1.0f, 0.0f), fh - 1.0f);
            const bool valid = (qb + t + k * nt < qe) && (pg + e < P);
            relq[k] = relq[k] || (valid && hi >= static_cast<float>(r0) && lo < static_cast<float>(r1));
          }
        }
      }
#pragma unroll
      for (int k = 0; k < kSQ; ++k) {
        const uint64_t mask = __ballot(relq[k]);
        int base = 0;
        if (lane == 0 && mask) base = atomicAdd(&misc[0], __popcll(mask));
        base = __shfl(base, 0, 64);
        if (relq[k]) rel[base + __popcll(mask & ((uint64_t{1} << lane) - 1))] = static_cast<uint16_t>(qb + t + k * nt - qs);
      }
    }
    __syncthreads();
    const int nrel = misc[0];

    // ---- phase 2: chunks of listed queries
    for (int m0 = 0; m0 < nrel; m0 += M) {
      const int m = min(M, nrel - m0);
      const int ns = m * P;
      // a. stage grad_output rows (4 channels per item), locations and weights
      {
        const int gq = D >> 2;  // 4-channel items per row
        if (p.g_vec4) {
          for (int e = t; e < m * gq; e += nt) {
            const int i = e / gq, part = e - i * gq;
            const int q = qs + rel[m0 + i];
            const int64_t go = ((static_cast<int64_t>(b) * Q + q) * p.heads + h) * D + part * 4;
            float v[4];
            load_any<4>(p.gout, go, gbf, v);
            *reinterpret_cast<float4*>(cg + i * D + part * 4) = make_float4(v[0], v[1], v[2], v[3]);
          }
        } else {
          for (int e = t; e < m * D; e += nt) {
            const int i = e / D, ch = e - i * D;
            const int q = qs + rel[m0 + i];
            float v[1];
            load_any<1>(p.gout, ((static_cast<int64_t>(b) * Q + q) * p.heads + h) * D + ch, gbf, v);
            cg[e] = v[0];
          }
        }
        for (int e = t; e < ns; e += nt) {
          const int i = e / P, pt = e - i * P;
          const int64_t si = srow0 + static_cast<int64_t>(qs + rel[m0 + i]) * qstride + pt;
          cl[e] = loc2[si];
          ca[e] = p.attn[si];
        }
      }
      __syncthreads();
      // b. owner gradients and cell buckets, one lane group per sample
      for (int e = t >> p.lpq_shift; e < ns; e += ngroups) {
        const int i = e / P, pt = e - i * P;
        const float2 xy = cl[e];
        const float a = ca[e];
        const Bilinear c = bilinear(xy.x, xy.y, L.h, W);
        const int yo = static_cast<int>(fminf(fmaxf(c.y0f, 0.0f), fh - 1.0f));
        if (want_dl && yo >= r0 && yo < r1) {
          // D_c = <g, v_c>; dA = sum_c w_c D_c; d out/d ix = gy (m10 D10 - m00 D00) + fy (m11 D11 - m01 D01), ...
          float g[VEC], v[VEC];
          load_vec<float, VEC>(cg + i * D + c0, g);
          if (!lane_on) {
#pragma unroll
            for (int k = 0; k < VEC; ++k) g[k] = 0.0f;
          }
          const VT* base = sv + c0;
          const int bb = r0 * W;
          float d00 = 0.0f, d10 = 0.0f, d01 = 0.0f, d11 = 0.0f;
          load_vec<VT, VEC>(base + (c.i00 - bb) * D, v);
#pragma unroll
          for (int k = 0; k < VEC; ++k) d00 += g[k] * v[k];
          load_vec<VT, VEC>(base + (c.i10 - bb) * D, v);
#pragma unroll
          for (int k = 0; k < VEC; ++k) d10 += g[k] * v[k];
          load_vec<VT, VEC>(base + (c.i01 - bb) * D, v);
#pragma unroll
          for (int k = 0; k < VEC; ++k) d01 += g[k] * v[k];
          load_vec<VT, VEC>(base + (c.i11 - bb) * D, v);
#pragma unroll
          for (int k = 0; k < VEC; ++k) d11 += g[k] * v[k];
          d00 = group_sum(d00, lpq);
          d10 = group_sum(d10, lpq);
          d01 = group_sum(d01, lpq);
          d11 = group_sum(d11, lpq);
          if (j == 0) {
            const float da = c.w00 * d00 + c.w10 * d10 + c.w01 * d01 + c.w11 * d11;
            const float g00 = c.m00 * d00, g10 = c.m10 * d10, g01 = c.m01 * d01, g11 = c.m11 * d11;
            const float dx = (1.0f - c.fy) * (g10 - g00) + c.fy * (g11 - g01);
            const float dy = (1.0f - c.fx) * (g01 - g00) + c.fx * (g11 - g10);
            const int64_t si = srow0 + static_cast<int64_t>(qs + rel[m0 + i]) * qstride + pt;
            if (p.dattn) p.dattn[si] = da;
            if (p.dloc) *reinterpret_cast<float2*>(p.dloc + 2 * si) = make_float2(a * fw * dx, a * fh * dy);
          }
        }
        if (j == 0 && want_dv) {
          // The sample's cell: its floor corner (x0, y0), or for non-finite weights its clipped
          // first corner (the reference adds those weights at the clipped corner indices).
          int cx, cy;
          const bool finite = isfinite(c.w00) && isfinite(c.w10) && isfinite(c.w01) && isfinite(c.w11);
          if (finite) {
            cx = static_cast<int>(fminf(fmaxf(floorf(pixel_coord(xy.x, fw)), -2.0f), fw));
            cy = static_cast<int>(fminf(fmaxf(c.y0f, -2.0f), fh));
          } else {
            cx = c.i00 % W;
            cy = c.i00 / W;
          }
          const int kx = cx + 1, ky = cy - r0 + 1;  // cell coordinates inside the band's cell grid
          const bool in = kx >= 0 && kx <= W && ky >= 0 && ky <= rb &&
                          (c.w00 != 0.0f || c.w10 != 0.0f || c.w01 != 0.0f || c.w11 != 0.0f);
          int key = -1;
          if (in) {
            key = ky * (W + 1) + kx;
            srank[e] = atomicAdd(&cnt[key], 1);
            swt[e] = make_float4(a * c.w00, a * c.w10, a * c.w01, a * c.w11);
          }
          skey[e] = key;
        }
      }
      if (want_dv) {
        __syncthreads();
        // c. cell offsets (clears the counts for the next chunk)
        block_scan_counts(cnt, off, ncell, misc + 4);
        // d. samples into cell order (query slot and a * corner weights)
        for (int e = t; e < ns; e += nt) {
          const int key = skey[e];
          if (key >= 0) {
            const int pos = off[key] + srank[e];
            rslot[pos] = e / P;
            rw[pos] = swt[e];
          }
        }
        __syncthreads();
        // e. cell-major accumulation in four colour phases: one lane per (cell, 4 channels) sums
        //    a * w_k * g over the cell's samples for its four corners in registers, then adds them
        //    to the corner pixels. Cells of one colour (cell x and y parities) are at least two
        //    cells apart, so their 2x2 pixel footprints are disjoint and no two lanes write the
        //    same accumulator element.
        const int gpp = (D + 3) >> 2;  // channel groups per cell
        for (int color = 0; color < 4; ++color) {
          const int ox = color & 1, oy = color >> 1;
          const int nu = (W + 1 - ox + 1) >> 1;   // cells per row of this colour
          const int nv = (rb + 1 - oy + 1) >> 1;  // cell rows of this colour
          for (int task = t; task < nu * nv * gpp; task += nt) {
            const int cidx = task / gpp, grp = task - cidx * gpp;
            const int v = cidx / nu, u = cidx - v * nu;
            const int kx = 2 * u + ox, ky = 2 * v + oy;
            const int key = ky * (W + 1) + kx;
            const int ch0 = grp * 4;
            const int nch = min(4, D - ch0);
            float s[4][4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
              for (int e = 0; e < 4; ++e) s[k][e] = 0.0f;
            const int rbeg = off[key], rend = off[key + 1];
            for (int r = rbeg; r < rend; ++r) {
              const float4 w4 = rw[r];
              const float* gr = cg + rslot[r] * D + ch0;
              float g4[4];
              if (nch == 4) {
                const float4 gv = *reinterpret_cast<const float4*>(gr);
                g4[0] = gv.x; g4[1] = gv.y; g4[2] = gv.z; g4[3] = gv.w;
              } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) g4[e] = e < nch ? gr[e] : 0.0f;
              }
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                s[0][e] += w4.x * g4[e];
                s[1][e] += w4.y * g4[e];
                s[2][e] += w4.z * g4[e];
                s[3][e] += w4.w * g4[e];
              }
            }
            if (rend > rbeg) {
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                // corner k of cell (kx, ky) is pixel (kx - 1 + (k & 1), ky - 1 + (k >> 1)) of the band
                const int px = kx - 1 + (k & 1), py = ky - 1 + (k >> 1);
                if (px >= 0 && px < W && py >= 0 && py < rb) {
                  float* ap = acc + (py * W + px) * D + ch0;
                  for (int e = 0; e < nch; ++e) ap[e] += s[k][e];
                }
              }
            }
          }
          __syncthreads();
        }
      }
      __syncthreads();
    }
  }

  // ---- phase 3
  __syncthreads();
  if (want_dv) {
    VT* dst = static_cast<VT*>(p.dvalue) + band_off;
    for (int i = t; i < rb * W * D; i += nt) {
      if constexpr (std::is_same<VT, float>::value) dst[i] = acc[i];
      else dst[i] = f32_to_bf16(acc[i]);
    }
  }
}

}  // namespace msda

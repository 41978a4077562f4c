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
constexpr int kRing = 128;  // records per wave in the backward ring (two waves' worth)

using bf16_t = uint16_t;
typedef __attribute__((address_space(3))) volatile int lds_vint;
typedef __attribute__((address_space(3))) int lds_int;

// An integer the compiler cannot see through. Reading a tag back through an opaque copy of its
// address keeps the compiler from forwarding the value this lane just stored (the read must see
// what *any* lane stored), without the per-access waits a volatile pointer costs.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

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
  int lpq_shift;
  int nwork;    // (level, band) items per slice
  int vec16;
  int chunk_q;  // queries whose locations / weights are staged in LDS at a time
  int loc_lds;  // byte offset of that staging area in LDS
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

// acc[pix[k]] += aw[k] * g for the corners k with `pending[k]`, for every lane group of the wave.
// Same-pixel collisions between lane groups are resolved with write-tag / read-back rounds (see
// the header comment); all four corners of a sample share each round. Corners of one sample with
// nonzero weight are distinct pixels; a repeated pixel (possible only for NaN weights, whose
// clipped corners coincide) is deferred to a later round so no read-modify-write is lost.
template <int VEC>
__device__ __forceinline__ void accumulate_corners(float* acc, int dim, int c0, bool lane_on, const int (&pix)[4],
                                                   bool (&pending)[4], const float (&aw)[4], const float (&g)[VEC],
                                                   lds_int* tags, int gid) {
  while (__any(pending[0] || pending[1] || pending[2] || pending[3])) {
    bool att[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      att[k] = pending[k];
#pragma unroll
      for (int m = 0; m < k; ++m) att[k] = att[k] && !(att[m] && pix[m] == pix[k]);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (att[k]) tags[pix[k]] = gid;
    // Reads are issued for every lane (from pixel 0 when not needed) so they share one wait.
    bool win[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int t = tags[opaque(att[k] ? pix[k] : 0)];
      win[k] = att[k] && t == gid;
    }
    float cur[4][VEC];
#pragma unroll
    for (int k = 0; k < 4; ++k) load_vec<float, VEC>(acc + (win[k] ? pix[k] : 0) * dim + c0, cur[k]);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (win[k] && lane_on) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) cur[k][e] += aw[k] * g[e];
        store_vec<float, VEC>(acc + pix[k] * dim + c0, cur[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) pending[k] = pending[k] && !win[k];
  }
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
  const int r0 = (wk - L.band_first) * L.band_rows;  // band rows [r0, r1); staged rows [r0, rs1)
  const int r1 = min(L.h, r0 + L.band_rows);
  const int rs1 = min(L.h, r1 + 1);
  const int rowlen = L.w * p.dim;
  const int64_t n = static_cast<int64_t>(b) * p.heads + h;
  const int64_t band_off = (n * p.len_value + L.start + static_cast<int64_t>(r0) * L.w) * p.dim;

  // LDS: staged rows | per-wave f32 accumulators | per-wave pixel tags | per-wave record rings |
  //      staged locations (float2) and weights of `chunk_q` queries x `points` samples
  const int nwaves = blockDim.x >> 6;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int band_px = (r1 - r0) * L.w;
  const int nacc = band_px * p.dim;
  const int nacc_pad = (nacc + 3) & ~3;
  VT* sv = reinterpret_cast<VT*>(lds_raw);
  const int nstage = (rs1 - r0) * rowlen;
  const int stage_bytes = ((nstage * static_cast<int>(sizeof(VT))) + 15) & ~15;
  float* acc_all = reinterpret_cast<float*>(lds_raw + stage_bytes);
  int* tags_all = reinterpret_cast<int*>(acc_all + nwaves * nacc_pad);
  lds_vint* ring_all = (lds_vint*)(tags_all + ((nwaves * band_px + 3) & ~3));
  float* acc = acc_all + wave * nacc_pad;
  lds_int* tags = (lds_int*)(tags_all + wave * band_px);
  lds_vint* ring = ring_all + wave * kRing;
  float2* cl = reinterpret_cast<float2*>(lds_raw + p.loc_lds);  // [chunk_q][points]
  float* ca = reinterpret_cast<float*>(cl + p.chunk_q * p.points);
  const bool want_dv = p.dvalue != nullptr;
  const bool want_dl = p.dloc != nullptr || p.dattn != nullptr;

  stage_copy(sv, static_cast<const VT*>(p.value) + band_off, nstage, p.vec16);
  if (want_dv) {
    float4* a4 = reinterpret_cast<float4*>(acc_all);
    const int n4 = (nwaves * nacc_pad) >> 2;
    for (int i = threadIdx.x; i < n4; i += blockDim.x) a4[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  __syncthreads();

  const int lpq = 1 << p.lpq_shift;
  const int j = lane & (lpq - 1);
  const int gid = lane >> p.lpq_shift;  // record slot inside the wave (also the tag value)
  const int per_pass = 64 >> p.lpq_shift;
  const bool lane_on = j * VEC < p.dim;
  const int c0 = lane_on ? j * VEC : 0;
  const int LP = p.levels * p.points;
  const int P = p.points;
  const int band_base = r0 * L.w;  // flat index of the band's first pixel inside the level
  const float fw = static_cast<float>(L.w), fh = static_cast<float>(L.h);
  const bool gbf = p.gout_bf16 != 0;
  const int64_t qstride = static_cast<int64_t>(p.heads) * LP;  // samples between consecutive queries
  const int64_t srow0 = (static_cast<int64_t>(b) * p.queries * p.heads + h) * LP + l * P;  // sample (q=0, pt=0)
  const float2* lsrc = reinterpret_cast<const float2*>(p.loc);

  // Process `cnt` (<= per_pass) queued queries starting at ring position `head`, one per lane
  // group; `c_lo` is the first query of the staged chunk.
  auto process = [&](int head, int cnt, int c_lo) {
    const bool has = gid < cnt;
    const int q = has ? ring[(head + gid) & (kRing - 1)] : c_lo;
    const int64_t bqh = (static_cast<int64_t>(b) * p.queries + q) * p.heads + h;
    const int64_t s0 = srow0 + static_cast<int64_t>(q) * qstride;
    float g[VEC];
    if (has) load_any<VEC>(p.gout, bqh * p.dim + c0, gbf, g);
    if (!has || !lane_on) {
#pragma unroll
      for (int k = 0; k < VEC; ++k) g[k] = 0.0f;
    }
    for (int pt = 0; pt < P; ++pt) {
      const float2 xy = cl[(q - c_lo) * P + pt];
      const float a = ca[(q - c_lo) * P + pt];
      const Bilinear c = bilinear(xy.x, xy.y, L.h, L.w);
      // Owner band: the one holding the floor row clamped into the level (NaN -> row 0); both
      // clipped corner rows of an owned sample are among the staged rows.
      const int yo = static_cast<int>(fminf(fmaxf(c.y0f, 0.0f), fh - 1.0f));
      const bool own = has && want_dl && yo >= r0 && yo < r1;
      const bool in0 = has && c.y0c >= r0 && c.y0c < r1;
      const bool in1 = has && c.y1c >= r0 && c.y1c < r1;
      if (own) {
        // D_c = <g, v_c> per corner; every gradient term is a combination of these.
        float v[VEC];
        float d00 = 0.0f, d10 = 0.0f, d01 = 0.0f, d11 = 0.0f;
        const VT* base = sv + c0;
        load_vec<VT, VEC>(base + (c.i00 - band_base) * p.dim, v);
#pragma unroll
        for (int k = 0; k < VEC; ++k) d00 += g[k] * v[k];
        load_vec<VT, VEC>(base + (c.i10 - band_base) * p.dim, v);
#pragma unroll
        for (int k = 0; k < VEC; ++k) d10 += g[k] * v[k];
        load_vec<VT, VEC>(base + (c.i01 - band_base) * p.dim, v);
#pragma unroll
        for (int k = 0; k < VEC; ++k) d01 += g[k] * v[k];
        load_vec<VT, VEC>(base + (c.i11 - band_base) * p.dim, v);
#pragma unroll
        for (int k = 0; k < VEC; ++k) d11 += g[k] * v[k];
        d00 = group_sum(d00, lpq);
        d10 = group_sum(d10, lpq);
        d01 = group_sum(d01, lpq);
        d11 = group_sum(d11, lpq);
        if (j == 0) {
          // dA = sum_c w_c D_c; d out/d ix = gy (m10 D10 - m00 D00) + fy (m11 D11 - m01 D01), etc.
          const float da = c.w00 * d00 + c.w10 * d10 + c.w01 * d01 + c.w11 * d11;
          const float g00 = c.m00 * d00, g10 = c.m10 * d10, g01 = c.m01 * d01, g11 = c.m11 * d11;
          const float dx = (1.0f - c.fy) * (g10 - g00) + c.fy * (g11 - g01);
          const float dy = (1.0f - c.fx) * (g01 - g00) + c.fx * (g11 - g10);
          const int64_t si = s0 + pt;
          if (p.dattn) p.dattn[si] = da;
          if (p.dloc) *reinterpret_cast<float2*>(p.dloc + 2 * si) = make_float2(a * fw * dx, a * fh * dy);
        }
      }
      if (want_dv) {
        const int pix[4] = {c.i00 - band_base, c.i10 - band_base, c.i01 - band_base, c.i11 - band_base};
        bool pend[4] = {in0 && c.w00 != 0.0f, in0 && c.w10 != 0.0f, in1 && c.w01 != 0.0f, in1 && c.w11 != 0.0f};
        const float aw[4] = {a * c.w00, a * c.w10, a * c.w01, a * c.w11};
        accumulate_corners<VEC>(acc, p.dim, c0, lane_on, pix, pend, aw, g, tags, gid);
      }
    }
  };

  int head = 0, tail = 0;  // wave-uniform ring positions
  constexpr int UL = 4;
  const int nt = blockDim.x;
  for (int c_lo = 0; c_lo < p.queries; c_lo += p.chunk_q) {
    const int nq = min(p.chunk_q, p.queries - c_lo);
    const int E = nq * P;
    // Stage this chunk's locations / weights (all loads of a batch in flight before the stores).
    for (int base = threadIdx.x; base < E; base += UL * nt) {
      float2 rl[UL];
      float ra[UL];
#pragma unroll
      for (int u = 0; u < UL; ++u) {
        const int i = base + u * nt;
        if (i < E) {
          const int qq = i / P, pt = i - qq * P;
          const int64_t si = srow0 + static_cast<int64_t>(c_lo + qq) * qstride + pt;
          rl[u] = lsrc[si];
          ra[u] = p.attn[si];
        }
      }
#pragma unroll
      for (int u = 0; u < UL; ++u) {
        const int i = base + u * nt;
        if (i < E) {
          cl[i] = rl[u];
          ca[i] = ra[u];
        }
      }
    }
    __syncthreads();
    // Scan, one lane per query: the query is relevant if one of its samples on this level has its
    // floor row (clamped into the level) in the band, or a clipped corner row in the band. Rows
    // [y0, y0+1] clipped to [0, H-1]: y0 <= -1 gives row 0 only, y0 >= H-1 gives row H-1 only.
    for (int qb = wave * 64; qb < nq; qb += nwaves * 64) {
      const int qq = qb + lane;
      bool rel = false;
      if (qq < nq) {
        for (int pt = 0; pt < P; ++pt) {
          const float y0f = floorf(pixel_coord(cl[qq * P + pt].y, fh));
          const float lo = fminf(fmaxf(y0f, 0.0f), fh - 1.0f);        // clipped first row (NaN -> 0)
          const float hi = fminf(fmaxf(y0f + 1.0f, 0.0f), fh - 1.0f);  // clipped second row
          rel = rel || (hi >= static_cast<float>(r0) && lo < static_cast<float>(r1));
        }
      }
      const uint64_t mask = __ballot(rel);
      if (rel) ring[(tail + __popcll(mask & ((uint64_t{1} << lane) - 1))) & (kRing - 1)] = c_lo + qq;
      tail += __popcll(mask);
      while (tail - head >= per_pass) {
        process(head, per_pass, c_lo);
        head += per_pass;
      }
    }
    while (head < tail) {  // drain before the staged chunk is replaced
      process(head, min(per_pass, tail - head), c_lo);
      head += min(per_pass, tail - head);
    }
    __syncthreads();
  }

  if (want_dv) {
    VT* dst = static_cast<VT*>(p.dvalue) + band_off;
    for (int i = threadIdx.x; i < nacc; i += blockDim.x) {
      float s = 0.0f;
      for (int w = 0; w < nwaves; ++w) s += acc_all[w * nacc_pad + i];
      if constexpr (std::is_same<VT, float>::value) dst[i] = s;
      else dst[i] = f32_to_bf16(s);
    }
  }
}

}  // namespace msda

// msda_kernels.h — gfx950 device code for multi-scale deformable attention: the forward kernel
// and the device helpers the backward kernels share (msda_band_kernels.h, msda_gather_kernels.h,
// msda_fused_bwd_kernels.h).
//
// Semantics follow RF-DETR-JAX's gather sampler, src/rfdetr_jax/models/ops.py:64-134 and
// ops.py:208-292: grid_sample(bilinear, zeros, align_corners=False) of each (batch, head) value
// slice at 2*loc-1, corner order (x0,y0),(x1,y0),(x0,y1),(x1,y1), masked weights multiplied onto
// values read at clipped indices, level-major point sum.
//
// fwd_kernel — one workgroup per (batch b, group of hg heads, block of queries). The group's value
// slices (the levels that fit) are staged into LDS with one batched copy; levels that do not fit
// are gathered through L2. Lanes are laid out channel group, then head, then query, so the lanes of
// one query read locations / weights and write output rows as contiguous runs of the
// [B, Q, H, ...] tensors. Each lane group computes a sample's coordinates once.
//
// Generic (flat) pointers to LDS cost vector-memory issue slots, so LDS reads go through
// address_space(3) pointers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace msda {

constexpr int kMaxLevels = 16;
constexpr int kXcds = 8;               // MI355X: 8 accelerator complex dies, workgroups dispatched round-robin
constexpr int kSampleMaxThreads = 1024;  // forward workgroups
constexpr int kPassBatch = 4;           // samples whose location / weight loads are issued together

using bf16_t = uint16_t;

struct LevelDesc {
  int h, w;        // level height and width
  float fh, fw;    // the same, as floats
  int small;       // h * w * dim < 2^24: corner offsets fit 24-bit multiplies
  int start;       // first position of the level in the value slice
  int lds;         // per-sample kernels: element offset of the staged level inside a head's LDS region, -1 = L2
  int band_rows;   // backward band kernel: image rows per band
  int band_first;  // backward band kernel: index of the level's first band among a slice's (level, band) items
  // The reference sampler the level reproduces (msda_fwd_sampler / msda_bwd_sampler):
  int rmode;      // forward rounding of a bf16 value map: kRoundNone, kRoundGather, kRoundGatherF32, kRoundMatmul
  int pallas_xy;  // pixel coordinates as the Pallas sampler forms them, loc * size - 0.5
};

// Forward rounding points of the reference's samplers on a bf16 value map (ops.py:64-186):
//   kRoundNone       f32 interpolation of the bf16 values, the weighted sum over points in f32;
//   kRoundGather     "gather": fractions, 1 - fraction, the corner-weight products, each corner
//                    product and the four-corner sum rounded to bf16 (ops.py:88-91, :123, :134);
//   kRoundGatherF32  "gather-f32": f32 interpolation, the sample rounded to bf16 (ops.py:137-144);
//   kRoundMatmul     "matmul": the axis kernels and their outer product rounded to bf16, the
//                    contraction with the values in f32, its result rounded to bf16 (ops.py:163-186).
enum RoundMode { kRoundNone = 0, kRoundGather = 1, kRoundGatherF32 = 2, kRoundMatmul = 3 };

// Forward kernels.
struct SampleParams {
  const void* value;
  const float* loc;
  const float* attn;
  void* out;         // forward: output [B, Q, H*D]
  int out_bf16;
  int pair_share;    // forward: one level, two points, two lanes per (query, head) (fwd_pair)
  int heads, dim, queries, levels, points;
  int64_t len_value;
  int lpq_shift;   // log2(lanes per (query, head)); each lane owns VEC channels
  int hg;          // heads per workgroup (divides heads)
  int qblock;      // queries per workgroup
  int nqb;         // query blocks per (batch, head group)
  int head_lds;    // LDS elements of one head's staged levels
  int all_staged;  // every level is staged, so a head group's value rows are one contiguous copy
  int vec16;       // value staging may use 16-byte vectors
  // Channel split (cs_shift > 0, forward only): 2^cs_shift workgroups share each head, one run of
  // its channels each, so that a value slice too large for the LDS at head_dim channels is staged
  // at head_dim / 2^cs_shift. `heads` and `dim` then count the split heads and their channels,
  // while the tensors hold `rheads` heads of `vstride` channels (rheads == heads and vstride == dim
  // without a split). The outputs of the parts are disjoint: no reduction.
  int rheads, vstride, cs_shift;
  // MSDeformAttn prologue fused in (kFused kernels, ops.py:388-404): `loc` then holds the raw
  // sampling offsets and `attn` the attention logits.
  const float* ref;  // reference points [B, Q, L, ref_dim]
  int ref_dim;       // 2 (points) or 4 (boxes: centre, width, height)
  float fpoints;     // n_points as a float: the box form divides the offsets by it
  float inv_points;  // 1 / n_points when n_points is a power of two (x / P == x * (1 / P) exactly), else 0
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

// The pixel coordinate of a location along one axis of level L: ops.py's formula, or the Pallas
// sampler's (LevelDesc::pallas_xy). Every kernel that decides a sample's cell goes through it, so
// a band's scan and the sample's corners agree on the floor.
// Written without a branch: ops.py's ((grid + 1) * size - 1) * 0.5 and the Pallas kernel's
// (loc * size - 0.5) * 1 share the multiply by size and differ in its operand and in two constants,
// so both cost the same six operations (a branch here stalled the backward's item loop).
__device__ __forceinline__ float level_coord(float loc, float size, const LevelDesc& L) {
#pragma clang fp contract(off)
  const bool pallas = L.pallas_xy != 0;
  const float grid1 = (2.0f * loc - 1.0f) + 1.0f;  // ops.py:270 then + 1 (2 * loc is exact)
  const float x = pallas ? loc : grid1;
  const float c = pallas ? 0.5f : 1.0f, half = pallas ? 1.0f : 0.5f;
  return (x * size - c) * half;  // ops.py:83-84 (dividing by two is exact) / deform_pallas.py:223-224
}

struct Bilinear {
  int o00, o10, o01, o11;      // element offsets (clipped pixel index * dim) of the corners in the level
  float w00, w10, w01, w11;    // masked corner weights
  float m00, m10, m01, m11;    // in-bounds masks
  float fx, fy;                // fractional parts
  int x0, y0;                  // floor corner, clamped to [-2, size] (outside means all-masked)
  int cx0, cy0;                // clipped floor corner
};

// ops.py:85-128 for one sample position. Offsets use 24-bit multiplies (full rate), valid while
// a level's H*W*dim < 2^24 elements; larger levels take the 32-bit path.
__device__ __forceinline__ Bilinear bilinear(float lx, float ly, const LevelDesc& L, int dim) {
  Bilinear c;
  const int h = L.h, w = L.w;
  const float ix = level_coord(lx, L.fw, L);
  const float iy = level_coord(ly, L.fh, L);
  const float x0f = floorf(ix), y0f = floorf(iy);
  c.fx = ix - x0f;  // rounded in f32 like ops.py:88-89 (inexact only for ix in (-1, 0))
  c.fy = iy - y0f;
  const float gx = 1.0f - c.fx, gy = 1.0f - c.fy;
  // Clamp before the integer conversion so huge or NaN coordinates stay defined; the clamp does
  // not change any in-bounds decision (values below -1 or above size-1 are out of bounds anyway).
  const int x0 = static_cast<int>(fminf(fmaxf(x0f, -2.0f), L.fw));
  const int y0 = static_cast<int>(fminf(fmaxf(y0f, -2.0f), L.fh));
  const int x1 = x0 + 1, y1 = y0 + 1;
  const bool mx0 = static_cast<unsigned>(x0) < static_cast<unsigned>(w);
  const bool mx1 = static_cast<unsigned>(x1) < static_cast<unsigned>(w);
  const bool my0 = static_cast<unsigned>(y0) < static_cast<unsigned>(h);
  const bool my1 = static_cast<unsigned>(y1) < static_cast<unsigned>(h);
  const int cx0 = min(max(x0, 0), w - 1), cx1 = min(max(x1, 0), w - 1);
  const int cy0 = min(max(y0, 0), h - 1), cy1 = min(max(y1, 0), h - 1);
  if (L.small) {
    const int r0 = __umul24(cy0, w), r1 = __umul24(cy1, w);
    c.o00 = __umul24(r0 + cx0, dim);
    c.o10 = __umul24(r0 + cx1, dim);
    c.o01 = __umul24(r1 + cx0, dim);
    c.o11 = __umul24(r1 + cx1, dim);
  } else {
    c.o00 = (cy0 * w + cx0) * dim;
    c.o10 = (cy0 * w + cx1) * dim;
    c.o01 = (cy1 * w + cx0) * dim;
    c.o11 = (cy1 * w + cx1) * dim;
  }
  c.m00 = (mx0 && my0) ? 1.0f : 0.0f;
  c.m10 = (mx1 && my0) ? 1.0f : 0.0f;
  c.m01 = (mx0 && my1) ? 1.0f : 0.0f;
  c.m11 = (mx1 && my1) ? 1.0f : 0.0f;
  // weight = (wx * wy) * inside, ops.py:123-128 (NaN coordinates give NaN weights, as there)
  c.w00 = (gx * gy) * c.m00;
  c.w10 = (c.fx * gy) * c.m10;
  c.w01 = (gx * c.fy) * c.m01;
  c.w11 = (c.fx * c.fy) * c.m11;
  c.x0 = x0;
  c.y0 = y0;
  c.cx0 = cx0;
  c.cy0 = cy0;
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

// LDS-qualified loads: a generic pointer that may point at LDS or global memory compiles to
// flat loads, and the optimizer merges identical LDS / global branches back into one, so LDS
// reads go through an address_space(3) pointer.
#define MSDA_LDS __attribute__((address_space(3)))

template <typename VT, int VEC>
__device__ __forceinline__ void load_vec_lds(const VT* p_generic, float (&o)[VEC]) {
  const MSDA_LDS VT* p = (const MSDA_LDS VT*)(p_generic);
  if constexpr (VEC == 1) {
    if constexpr (std::is_same<VT, float>::value) o[0] = *p;
    else o[0] = bf16_to_f32(*p);
  } else if constexpr (std::is_same<VT, float>::value) {
    const typename VecT<float, VEC>::type v = *(const MSDA_LDS typename VecT<float, VEC>::type*)(p);
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = v[k];
  } else {
    const typename VecT<bf16_t, VEC>::type v = *(const MSDA_LDS typename VecT<bf16_t, VEC>::type*)(p);
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
    // bf16 rows (outputs, grad_value) are written once and not read back by the writing kernel:
    // non-temporal stores (measured on MI355X: the two_level_fwdbwd_b8_bf16 backward 3.5 % faster;
    // f32 rows stay ordinary stores, whose rotated 16-byte chunks were slower non-temporal)
    typename VecT<bf16_t, VEC>::type v;
#pragma unroll
    for (int k = 0; k < VEC; ++k) v[k] = f32_to_bf16(a[k]);
    __builtin_nontemporal_store(v, reinterpret_cast<typename VecT<bf16_t, VEC>::type*>(p));
  }
}

template <int VEC>
__device__ __forceinline__ void store_any(void* base, int64_t off, bool is_bf16, const float (&a)[VEC]) {
  if (is_bf16) store_vec<bf16_t, VEC>(static_cast<bf16_t*>(base) + off, a);
  else store_vec<float, VEC>(static_cast<float*>(base) + off, a);
}

// Rotated chunk order. A lane's VEC channels span N = VEC * sizeof(VT) / 16 chunks of 16 bytes
// (N = 1 when the run is a single chunk, shorter, or not a multiple of 16 bytes). Register slot k
// of a lane holds channel chunk (k + rot) mod N, where rot steps with the lane's (query, head)
// index. An LDS row of 64 bytes spans four of the 16 four-bank groups a 16-lane access cycle
// uses, so lanes reading the same chunk of random rows pile into four groups; rotating the chunk
// by lane spreads them over all 16 (measured: same-chunk reads of random rows spend about two
// thirds of LDS cycles in bank conflicts).
template <typename VT, int VEC>
constexpr int rot_chunks() {
  return (VEC * static_cast<int>(sizeof(VT))) % 16 == 0 && VEC * static_cast<int>(sizeof(VT)) >= 32
             ? VEC * static_cast<int>(sizeof(VT)) / 16
             : 1;
}

template <typename VT, int VEC, bool kLds>
__device__ __forceinline__ void load_rot(const VT* p, int rot, float (&o)[VEC]) {
  constexpr int N = rot_chunks<VT, VEC>();
  if constexpr (N == 1) {
    if constexpr (kLds) load_vec_lds<VT, VEC>(p, o);
    else load_vec<VT, VEC>(p, o);
  } else {
    constexpr int E = VEC / N;
#pragma unroll
    for (int k = 0; k < N; ++k) {
      const int c = (k + rot) & (N - 1);
      float t[E];
      if constexpr (kLds) load_vec_lds<VT, E>(p + c * E, t);
      else load_vec<VT, E>(p + c * E, t);
#pragma unroll
      for (int i = 0; i < E; ++i) o[k * E + i] = t[i];
    }
  }
}

// The same order for a tensor in either dtype (grad_output), chunks counted in VT elements.
template <typename VT, int VEC>
__device__ __forceinline__ void load_any_rot(const void* base, int64_t off, bool is_bf16, int rot, float (&o)[VEC]) {
  constexpr int N = rot_chunks<VT, VEC>();
  if constexpr (N == 1) {
    load_any<VEC>(base, off, is_bf16, o);
  } else {
    constexpr int E = VEC / N;
#pragma unroll
    for (int k = 0; k < N; ++k) {
      float t[E];
      load_any<E>(base, off + ((k + rot) & (N - 1)) * E, is_bf16, t);
#pragma unroll
      for (int i = 0; i < E; ++i) o[k * E + i] = t[i];
    }
  }
}

template <typename VT, int VEC>
__device__ __forceinline__ void store_any_rot(void* base, int64_t off, bool is_bf16, int rot, const float (&a)[VEC]) {
  constexpr int N = rot_chunks<VT, VEC>();
  if constexpr (N == 1) {
    store_any<VEC>(base, off, is_bf16, a);
  } else {
    constexpr int E = VEC / N;
#pragma unroll
    for (int k = 0; k < N; ++k) {
      float t[E];
#pragma unroll
      for (int i = 0; i < E; ++i) t[i] = a[k * E + i];
      store_any<E>(base, off + ((k + rot) & (N - 1)) * E, is_bf16, t);
    }
  }
}

// Waits until every vector-memory operation this wave issued has completed (gfx9 s_waitcnt
// encoding: vmcnt 0, expcnt and lgkmcnt left at their maxima). Placed where a group of loads is
// about to be consumed and before the group's stores: vmcnt counts loads and stores in issue order,
// so once the wait is explicit the compiler needs no later vmcnt waits, which would otherwise also
// wait for the acknowledgement of every store issued before them.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Cooperative copy global -> LDS of `count` elements. With 16-byte rows the copy goes straight
// from global memory into LDS (global_load_lds_dwordx4: lane i of a wave writes 16 bytes at the
// wave's LDS base + 16 i, no registers involved), each wave streaming whole 1 KB blocks, so every
// block is in flight at once; the wave waits for its own transfers before returning (the caller's
// barrier then publishes them). Otherwise each thread issues a batch of loads before any store.
// kWait = false leaves the 16-byte path's transfers outstanding (the caller waits before its barrier).
// wave0, nw: only waves [wave0, wave0 + nw) copy (default: all of the workgroup's waves).
template <typename VT, bool kWait = true>
__device__ __forceinline__ void stage_copy(VT* dst, const VT* __restrict__ src, int count, bool vec16, int wave0 = 0, int nw = 0) {
  constexpr int U = 8;
  if (nw <= 0) nw = static_cast<int>(blockDim.x >> 6);  // waves [wave0, wave0 + nw) copy; others return
  const int wave = static_cast<int>(threadIdx.x >> 6) - wave0;
  if (wave < 0 || wave >= nw) return;
  const int nt = nw * 64, t = static_cast<int>(threadIdx.x) - wave0 * 64;
  if (vec16) {
    const int n16 = static_cast<int>((static_cast<int64_t>(count) * sizeof(VT)) / 16);
    const uint4* s = reinterpret_cast<const uint4*>(src);
    uint4* d = reinterpret_cast<uint4*>(dst);
    const int lane = threadIdx.x & 63;
    const int nblk = n16 >> 6;  // whole 1 KB blocks
    for (int blk = wave; blk < nblk; blk += nw)
      __builtin_amdgcn_global_load_lds(s + blk * 64 + lane, (MSDA_LDS void*)(d + blk * 64), 16, 0, 0);
    for (int i = (nblk << 6) + t; i < n16; i += nt) d[i] = s[i];
    if constexpr (kWait) wait_vmem();
  } else {
    int i = t;
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

// Staging of one part of a split head: `cells` cells of `dim` elements each, `stride` elements apart
// in memory, packed in LDS. dim and stride are whole 16-byte chunks and src is 16-byte aligned, so
// every chunk goes straight to LDS, 64 consecutive LDS chunks per wave instruction.
template <typename VT>
__device__ __forceinline__ void stage_cells(VT* dst, const VT* __restrict__ src, int cells, int dim, int stride) {
  constexpr int E = 16 / static_cast<int>(sizeof(VT));  // elements per chunk
  const int cpc = dim / E;                               // chunks per cell
  const int n16 = cells * cpc;
  const int t = static_cast<int>(threadIdx.x), nt = static_cast<int>(blockDim.x);
  const int lane = t & 63, wave = t >> 6, nw = nt >> 6;
  uint4* d = reinterpret_cast<uint4*>(dst);
  auto chunk = [&](int i) {
    const int cell = i / cpc;
    return reinterpret_cast<const uint4*>(src + static_cast<int64_t>(cell) * stride) + (i - cell * cpc);
  };
  const int nblk = n16 >> 6;
  for (int blk = wave; blk < nblk; blk += nw)
    __builtin_amdgcn_global_load_lds(chunk(blk * 64 + lane), (MSDA_LDS void*)(d + blk * 64), 16, 0, 0);
  for (int i = (nblk << 6) + t; i < n16; i += nt) d[i] = *chunk(i);
  wait_vmem();
}

// ---------------------------------------------------------------------------------------------
// per-sample kernels: shared work-item decomposition and staging

struct SampleItem {
  int b, h0, qb;
};

// Work item = (batch b, head group, query block); the blocks of one (b, group) are adjacent in
// logical order, so they run on one XCD and share its L2 copy of the group's value rows.
__device__ __forceinline__ SampleItem sample_item(const SampleParams& p) {
  const int ngroups = p.heads / p.hg;
  const int lid = xcd_logical(blockIdx.x, gridDim.x);
  SampleItem it;
  it.qb = lid % p.nqb;
  const int rest = lid / p.nqb;
  it.h0 = (rest % ngroups) * p.hg;
  it.b = rest / ngroups;
  return it;
}

// The group's slices are consecutive rows of value [B*H, S, D]: when every level is staged they
// are one contiguous copy (a split head, always alone in its group: one run of each cell).
template <typename VT>
__device__ __forceinline__ void stage_group(const SampleParams& p, VT* lds, const VT* __restrict__ vg) {
  const int64_t slice_elems = p.len_value * p.dim;
  if (p.all_staged) {
    if (p.cs_shift > 0) stage_cells(lds, vg, static_cast<int>(p.len_value), p.dim, p.vstride);
    else stage_copy(lds, vg, static_cast<int>(p.hg * slice_elems), p.vec16);
    return;
  }
  for (int hh = 0; hh < p.hg; ++hh)
    for (int l = 0; l < p.levels; ++l) {
      const LevelDesc L = p.lv[l];
      if (L.lds >= 0)
        stage_copy(lds + hh * p.head_lds + L.lds, vg + hh * slice_elems + static_cast<int64_t>(L.start) * p.dim,
                   L.h * L.w * p.dim, p.vec16);
    }
}

// Lane layout: channel groups of one (query, head) are adjacent, then the group's heads, then
// queries; so the lanes of one query touch contiguous runs of its [H, ...] rows.
struct SampleLane {
  int j, hl, qs, qpp, c0;
  int rot;  // chunk rotation of this lane's channel run (rot_chunks)
  bool active, lane_on;
};

template <typename VT, int VEC>
__device__ __forceinline__ SampleLane sample_lane(const SampleParams& p) {
  SampleLane s;
  const int lpq = 1 << p.lpq_shift;
  const int t = threadIdx.x;
  s.j = t & (lpq - 1);
  const int hq = t >> p.lpq_shift;
  s.hl = hq % p.hg;
  s.qs = hq / p.hg;
  s.qpp = (static_cast<int>(blockDim.x) >> p.lpq_shift) / p.hg;  // queries per pass
  s.active = s.qs < s.qpp;
  s.lane_on = s.j * VEC < p.dim;
  s.c0 = s.lane_on ? s.j * VEC : 0;
  s.rot = hq & (rot_chunks<VT, VEC>() - 1);  // consecutive (query, head) lanes rotate by one chunk
  return s;
}

// A lane's inputs for up to N samples of one (query, head), loaded together.
template <int N>
struct SampleIn {
  float2 xy[N];
  float a[N];
};

template <int N>
__device__ __forceinline__ void load_in(SampleIn<N>& f, const float2* __restrict__ lq, const float* __restrict__ aq, int s0,
                                        int LP) {
#pragma unroll
  for (int u = 0; u < N; ++u) {
    if (s0 + u < LP) {
      f.xy[u] = lq[s0 + u];
      f.a[u] = aq[s0 + u];
    }
  }
}

// Queries per lane whose inputs are loaded together when a query's samples fit NS (NS = 0: one
// query at a time, its samples in chunks of kPassBatch). The loads of a group are all in flight
// before the first is used, so a lane waits one memory latency per group rather than per query
// (sized so that no instantiation spills registers at four waves per SIMD).
constexpr int query_group(int ns, int vec, bool fused = false) {
  if (ns == 0) return 1;
  // + a reference point and a box offset per sample
  if (fused) return vec >= 8 ? (ns <= 2 ? 2 : 1) : (ns <= 2 ? 4 : 2);
  return ns <= 2 ? 4 : 2;
}

// Samples per chunk of the per-query loop (NS = 0); the fused prologue's per-sample reference
// points and box offsets make the chunk half as long, within the same register budget.
constexpr int pass_batch(bool fused) { return fused ? 2 : kPassBatch; }

// own >= 0 (fwd_pair): only sample `own` of each query is loaded, into slot 0 (the lane computes
// that sample's coordinates and receives the other's from its partner lane).
template <int NS, int QU>
__device__ __forceinline__ void load_group(SampleIn<NS> (&in)[QU], const float2* __restrict__ loc2, const float* __restrict__ attn,
                                           int64_t row0, int64_t row_step, int q0, int q_step, int q_hi, int LP, int own = -1) {
#pragma unroll
  for (int i = 0; i < QU; ++i) {
    if (q0 + i * q_step < q_hi) {
      const int64_t row = row0 + i * row_step;
      if (own >= 0) {
        in[i].xy[0] = loc2[row * LP + own];
        in[i].a[0] = attn[row * LP + own];
      } else {
        load_in<NS>(in[i], loc2 + row * LP, attn + row * LP, 0, LP);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// MSDeformAttn prologue fused into the forward kernel (ops.py:388-404): sample locations from
// reference points and raw offsets, attention weights from a softmax over each (query, head)'s
// L*P logits; fused_offset_grad is the transpose the fused backward's epilogue applies.

// What the prologue adds per sample: the reference point of the sample's level (x, y, and for
// boxes w, h), and the offset the box form scales (off / n_points; the raw offset for points).
template <int N, bool kFused>
struct FusedIn {};
template <int N>
struct FusedIn<N, true> {
  float4 r[N];
  float2 t[N];
};

// Reference point of level l for query row bq = b * Q + q.
__device__ __forceinline__ float4 load_ref(const SampleParams& p, int64_t bq, int l) {
  const int64_t i = bq * p.levels + l;
  if (p.ref_dim == 4) return *reinterpret_cast<const float4*>(p.ref + i * 4);
  const float2 v = *reinterpret_cast<const float2*>(p.ref + i * 2);
  return make_float4(v.x, v.y, 0.0f, 0.0f);
}

// Reference points of samples s0 .. s0 + N - 1, the first at level l, point pt.
template <int N>
__device__ __forceinline__ void load_refs(FusedIn<N, true>& x, const SampleParams& p, int64_t bq, int s0, int LP, int l, int pt) {
#pragma unroll
  for (int u = 0; u < N; ++u) {
    if (s0 + u < LP) {
      x.r[u] = load_ref(p, bq, l);
      if (++pt == p.points) {
        pt = 0;
        ++l;
      }
    }
  }
}

// jax.nn.softmax as ops.py:403-404 calls it, in f32: weight = exp(x - max) / sum(exp(x - max)).
// The statistics are formed in sample order, from memory or from registers, with the same
// operations, so both give the same weights.
struct SoftmaxStats {
  float m, s;
};

__device__ __forceinline__ float softmax_weight(float x, SoftmaxStats st) { return expf(x - st.m) / st.s; }

__device__ __forceinline__ SoftmaxStats softmax_stats(const float* __restrict__ x, int LP) {
  SoftmaxStats st{-__builtin_inff(), 0.0f};
  for (int k = 0; k < LP; ++k) st.m = fmaxf(st.m, x[k]);
  for (int k = 0; k < LP; ++k) st.s += expf(x[k] - st.m);
  return st;
}

// From registers, when every sample of the row is loaded: the logits become the weights in place,
// each exponential computed once.
template <int N>
__device__ __forceinline__ void softmax_regs(SampleIn<N>& f, int LP) {
  float m = -__builtin_inff(), s = 0.0f;
#pragma unroll
  for (int u = 0; u < N; ++u)
    if (u < LP) m = fmaxf(m, f.a[u]);
#pragma unroll
  for (int u = 0; u < N; ++u)
    if (u < LP) {
      f.a[u] = expf(f.a[u] - m);
      s += f.a[u];
    }
#pragma unroll
  for (int u = 0; u < N; ++u)
    if (u < LP) f.a[u] = f.a[u] / s;
}

// ops.py:388-399 for one sample. Points: ref + off / (W_l, H_l). Boxes: ref_xy + off / n_points *
// ref_wh * 0.5, evaluated left to right. Each division is one IEEE rounding (precise_divide,
// ops.py:46-62; hipcc's f32 division is correctly rounded) and nothing is contracted.
// t: the offset term that multiplies ref_wh (boxes), kept for the reference-point gradient.
__device__ __forceinline__ float2 fused_location_at(float2 off, float4 r, float2& t, float fw, float fh, int ref_dim,
                                                    float inv_points, float fpoints) {
#pragma clang fp contract(off)
  if (ref_dim == 2) {
    t = off;
    return make_float2(r.x + off.x / fw, r.y + off.y / fh);
  }
  t = inv_points != 0.0f ? make_float2(off.x * inv_points, off.y * inv_points) : make_float2(off.x / fpoints, off.y / fpoints);
  return make_float2(r.x + (t.x * r.z) * 0.5f, r.y + (t.y * r.w) * 0.5f);
}

__device__ __forceinline__ float2 fused_location(float2 off, float4 r, float2& t, const LevelDesc& L, const SampleParams& p) {
  return fused_location_at(off, r, t, L.fw, L.fh, p.ref_dim, p.inv_points, p.fpoints);
}

// Turns loaded offsets of samples s0 .. s0 + N - 1 into locations.
template <int N>
__device__ __forceinline__ void fused_locations(SampleIn<N>& f, FusedIn<N, true>& x, const SampleParams& p, int s0, int LP, int l,
                                                int pt) {
#pragma unroll
  for (int u = 0; u < N; ++u) {
    if (s0 + u < LP) {
      f.xy[u] = fused_location(f.xy[u], x.r[u], x.t[u], p.lv[l], p);
      if (++pt == p.points) {
        pt = 0;
        ++l;
      }
    }
  }
}

// Turns loaded (offset, logit) pairs of samples s0 .. s0 + N - 1 into (location, weight), with the
// row's softmax statistics.
template <int N>
__device__ __forceinline__ void fused_prologue(SampleIn<N>& f, FusedIn<N, true>& x, SoftmaxStats st, const SampleParams& p,
                                               int s0, int LP, int l, int pt) {
#pragma unroll
  for (int u = 0; u < N; ++u)
    if (s0 + u < LP) f.a[u] = softmax_weight(f.a[u], st);
  fused_locations<N>(f, x, p, s0, LP, l, pt);
}

// The same when the row's samples are all in registers (s0 = 0, N >= LP).
template <int N>
__device__ __forceinline__ void fused_prologue_row(SampleIn<N>& f, FusedIn<N, true>& x, const SampleParams& p, int LP) {
  softmax_regs<N>(f, LP);
  fused_locations<N>(f, x, p, 0, LP, 0, 0);
}

// The transpose of fused_location_at for one sample: the offset gradient, and the sample's share of
// the reference-point gradient added into r (x, y, and w, h for boxes). Nothing is contracted: each
// product is rounded before it is added, so a sum over points comes out the same whether it is kept
// in r across the points or formed from the shares afterwards.
__device__ __forceinline__ float2 fused_offset_grad(float2 gl, float4 ref, float2 t, float fw, float fh, int ref_dim,
                                                    float inv_points, float fpoints, float (&r)[4]) {
#pragma clang fp contract(off)
  r[0] += gl.x;
  r[1] += gl.y;
  if (ref_dim == 2) return make_float2(gl.x / fw, gl.y / fh);
  const float hx = gl.x * 0.5f, hy = gl.y * 0.5f;
  r[2] += hx * t.x;
  r[3] += hy * t.y;
  if (inv_points != 0.0f) return make_float2((hx * ref.z) * inv_points, (hy * ref.w) * inv_points);
  return make_float2((hx * ref.z) / fpoints, (hy * ref.w) / fpoints);
}

// ---------------------------------------------------------------------------------------------
// forward

template <typename VT, int VEC, bool kLds>
__device__ __forceinline__ void fwd_corners(float (&acc)[VEC], const VT* base, const Bilinear& c, float a, int rot) {
  const float a00 = a * c.w00, a10 = a * c.w10, a01 = a * c.w01, a11 = a * c.w11;
  // Two corners in flight at a time keeps 16-channel lanes within the register budget; one fused
  // multiply-add per channel and corner.
  float u0[VEC], u1[VEC];
  load_rot<VT, VEC, kLds>(base + c.o00, rot, u0);
  load_rot<VT, VEC, kLds>(base + c.o10, rot, u1);
#pragma unroll
  for (int k = 0; k < VEC; ++k) acc[k] = fmaf(u1[k], a10, fmaf(u0[k], a00, acc[k]));
  load_rot<VT, VEC, kLds>(base + c.o01, rot, u0);
  load_rot<VT, VEC, kLds>(base + c.o11, rot, u1);
#pragma unroll
  for (int k = 0; k < VEC; ++k) acc[k] = fmaf(u1[k], a11, fmaf(u0[k], a01, acc[k]));
}

// The corners of one sample at a level with a reference sampler's bf16 rounding points (RoundMode),
// added into acc as a * sample. Values are read in the lane's rotated chunk order; the rounding is
// per channel, so the order does not matter. Products and sums are not contracted.
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

template <typename VT, int VEC, bool kLds>
__device__ __forceinline__ void fwd_corners_rounded(float (&acc)[VEC], const VT* base, const Bilinear& c, float a, int rot, int mode) {
#pragma clang fp contract(off)
  float w00, w10, w01, w11;
  if (mode == kRoundGather) {
    const float wx1 = round_bf16(c.fx), wy1 = round_bf16(c.fy);
    const float wx0 = round_bf16(1.0f - wx1), wy0 = round_bf16(1.0f - wy1);
    w00 = round_bf16(wx0 * wy0) * c.m00;
    w10 = round_bf16(wx1 * wy0) * c.m10;
    w01 = round_bf16(wx0 * wy1) * c.m01;
    w11 = round_bf16(wx1 * wy1) * c.m11;
  } else if (mode == kRoundMatmul) {
    const float kx0 = round_bf16(1.0f - c.fx), kx1 = round_bf16(c.fx);
    const float ky0 = round_bf16(1.0f - c.fy), ky1 = round_bf16(c.fy);
    w00 = round_bf16(ky0 * kx0) * c.m00;
    w10 = round_bf16(ky0 * kx1) * c.m10;
    w01 = round_bf16(ky1 * kx0) * c.m01;
    w11 = round_bf16(ky1 * kx1) * c.m11;
  } else {  // kRoundGatherF32: the f32 weights of ops.py:123-128
    w00 = c.w00;
    w10 = c.w10;
    w01 = c.w01;
    w11 = c.w11;
  }
  float u00[VEC], u10[VEC], u01[VEC], u11[VEC];
  load_rot<VT, VEC, kLds>(base + c.o00, rot, u00);
  load_rot<VT, VEC, kLds>(base + c.o10, rot, u10);
  load_rot<VT, VEC, kLds>(base + c.o01, rot, u01);
  load_rot<VT, VEC, kLds>(base + c.o11, rot, u11);
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    float p00 = u00[k] * w00, p10 = u10[k] * w10, p01 = u01[k] * w01, p11 = u11[k] * w11;
    if (mode == kRoundGather) {
      p00 = round_bf16(p00);
      p10 = round_bf16(p10);
      p01 = round_bf16(p01);
      p11 = round_bf16(p11);
    }
    const float sample = round_bf16(((p00 + p10) + p01) + p11);
    acc[k] = fmaf(a, sample, acc[k]);
  }
}

// kStaged: every level is staged in LDS (no L2 gather path is compiled).
template <typename VT, int VEC, int N, bool kStaged>
__device__ __forceinline__ void fwd_pass(float (&acc)[VEC], const SampleIn<N>& f, int s0, int LP, int& l, int& pt,
                                         const SampleParams& p, const VT* hlds, const VT* __restrict__ vs, int rot) {
  const int D = p.dim;
#pragma unroll
  for (int u = 0; u < N; ++u) {
    if (s0 + u < LP) {
      const LevelDesc L = p.lv[l];
      const Bilinear c = bilinear(f.xy[u].x, f.xy[u].y, L, D);
      // Separate LDS and global paths: a pointer that may be either compiles to flat loads.
      if (L.rmode != kRoundNone) {
        if (kStaged || L.lds >= 0) fwd_corners_rounded<VT, VEC, true>(acc, hlds + L.lds, c, f.a[u], rot, L.rmode);
        else fwd_corners_rounded<VT, VEC, false>(acc, vs + static_cast<int64_t>(L.start) * D, c, f.a[u], rot, L.rmode);
      } else if (kStaged || L.lds >= 0) {
        fwd_corners<VT, VEC, true>(acc, hlds + L.lds, c, f.a[u], rot);
      } else {
        fwd_corners<VT, VEC, false>(acc, vs + static_cast<int64_t>(L.start) * D, c, f.a[u], rot);
      }
      if (++pt == p.points) {
        pt = 0;
        ++l;
      }
    }
  }
}

// One level, two points, two lanes per (query, head) (pair_share): lane j computes the corner
// offsets and weights of sample j only (in slot `slot` of f: 0 when the lane loaded its own sample
// only, j when both are in registers, as after the fused prologue's softmax) and the two lanes
// exchange them, so each sample's coordinates are computed once; each lane then adds its own
// sample first (the order of the two f32 additions per channel is the only difference from
// fwd_pass).
template <typename VT, int VEC>
__device__ __forceinline__ void fwd_pair(float (&acc)[VEC], const SampleIn<2>& f, const SampleParams& p, const VT* hlds,
                                         int rot, int slot) {
  const LevelDesc L = p.lv[0];
  const float2 xy = slot ? f.xy[1] : f.xy[0];
  const float a = slot ? f.a[1] : f.a[0];
  const Bilinear c = bilinear(xy.x, xy.y, L, p.dim);
  // lane swap with the neighbour: DPP quad_perm [1, 0, 3, 2] (a register move, no LDS traffic)
  auto swap_i = [](int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); };
  auto swap_f = [&](float v) { return __int_as_float(swap_i(__float_as_int(v))); };
  Bilinear o;  // the partner's sample: offsets and attention-weighted corner weights
  o.o00 = swap_i(c.o00);
  o.o10 = swap_i(c.o10);
  o.o01 = swap_i(c.o01);
  o.o11 = swap_i(c.o11);
  Bilinear m = c;
  m.w00 = a * c.w00;
  m.w10 = a * c.w10;
  m.w01 = a * c.w01;
  m.w11 = a * c.w11;
  o.w00 = swap_f(m.w00);
  o.w10 = swap_f(m.w10);
  o.w01 = swap_f(m.w01);
  o.w11 = swap_f(m.w11);
  fwd_corners<VT, VEC, true>(acc, hlds + L.lds, m, 1.0f, rot);
  fwd_corners<VT, VEC, true>(acc, hlds + L.lds, o, 1.0f, rot);
}

// Four waves per SIMD (<= 128 VGPRs): latency is hidden by other waves rather than by
// registers holding the next query's inputs (measured faster on MI355X).
// kFused: `loc` / `attn` are raw offsets and logits, turned into locations and weights first.
template <typename VT, int VEC, int NS, bool kStaged, bool kFused>
__global__ void __launch_bounds__(kSampleMaxThreads) __attribute__((amdgpu_waves_per_eu(4)))
fwd_kernel(const SampleParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  VT* lds = reinterpret_cast<VT*>(lds_raw);
  const SampleItem it = sample_item(p);
  const SampleLane ln = sample_lane<VT, VEC>(p);
  const int rot = ln.rot;
  const int D = p.dim;
  const int64_t slice_elems = p.len_value * D;
  // split heads: head h is run h & csm of the channels of head h >> cs_shift in memory
  const int csm = (1 << p.cs_shift) - 1;
  const VT* __restrict__ vg = static_cast<const VT*>(p.value) +
                              (static_cast<int64_t>(it.b) * p.rheads + (it.h0 >> p.cs_shift)) * (p.len_value * p.vstride) +
                              (it.h0 & csm) * D;
  const int h = it.h0 + ln.hl;
  const int rh = h >> p.cs_shift, sub = h & csm;
  // (b, q, rh) rows of the locations and weights; output row (row << cs_shift) + sub of [B, Q, H, D]
  auto out_off = [&](int64_t row) { return ((row << p.cs_shift) + sub) * D + ln.c0; };
  const int LP = p.levels * p.points;
  const int q_lo = it.qb * p.qblock;
  const int q_hi = min(p.queries, q_lo + p.qblock);
  const float2* __restrict__ loc2 = reinterpret_cast<const float2*>(p.loc);
  constexpr int QU = query_group(NS, VEC, kFused);
  constexpr int NI = NS == 0 ? 1 : NS;
  const int q_first = q_lo + ln.qs;
  const int64_t row_first = (static_cast<int64_t>(it.b) * p.queries + q_first) * p.rheads + rh;  // (b, q, h)
  const int64_t row_step = static_cast<int64_t>(ln.qpp) * p.rheads;
  const int64_t bq0 = static_cast<int64_t>(it.b) * p.queries;  // query row b * Q of the reference points
  SampleIn<NI> in[QU];
  FusedIn<NI, kFused> fin[QU];
  auto load_refs_group = [&](int q0) {
    if constexpr (kFused) {
#pragma unroll
      for (int i = 0; i < QU; ++i)
        if (q0 + i * ln.qpp < q_hi) load_refs<NI>(fin[i], p, bq0 + q0 + i * ln.qpp, 0, LP, 0, 0);
    }
  };
  // The first group's inputs are requested before the staging copy, so their latency overlaps it.
  // fwd_pair lanes load their own sample only
  const int own = (NS == 2 && kStaged && !kFused && p.pair_share) ? ln.j : -1;
  if constexpr (NS > 0)
    if (ln.active) {
      load_group<NS, QU>(in, loc2, p.attn, row_first, row_step, q_first, ln.qpp, q_hi, LP, own);
      load_refs_group(q_first);
    }
  stage_group(p, lds, vg);
  __syncthreads();
  if (!ln.active) return;  // no barrier follows

  const VT* __restrict__ vs = vg + ln.hl * slice_elems + ln.c0;  // this head's slice in global memory
  const VT* hlds = lds + ln.hl * p.head_lds + ln.c0;
  if constexpr (NS > 0) {
    for (int qg = q_first; qg < q_hi; qg += QU * ln.qpp) {
      const int64_t row0 = row_first + static_cast<int64_t>((qg - q_first) / ln.qpp) * row_step;
      if (qg != q_first) {
        load_group<NS, QU>(in, loc2, p.attn, row0, row_step, qg, ln.qpp, q_hi, LP, own);
        load_refs_group(qg);
      }
      wait_vmem();
      if constexpr (kFused) {
#pragma unroll
        for (int i = 0; i < QU; ++i)
          if (qg + i * ln.qpp < q_hi) fused_prologue_row<NS>(in[i], fin[i], p, LP);
      }
#pragma unroll
      for (int i = 0; i < QU; ++i) {
        if (qg + i * ln.qpp < q_hi) {
          const int64_t row = row0 + i * row_step;
          float acc[VEC];
#pragma unroll
          for (int k = 0; k < VEC; ++k) acc[k] = 0.0f;
          if constexpr (NS == 2 && kStaged) {
            if (p.pair_share) {
              fwd_pair<VT, VEC>(acc, in[i], p, hlds, rot, kFused ? ln.j : 0);
              if (ln.lane_on) store_any_rot<VT, VEC>(p.out, out_off(row), p.out_bf16 != 0, rot, acc);
              continue;
            }
          }
          int l = 0, pt = 0;  // level and point of the next sample (level-major order, ops.py:285)
          fwd_pass<VT, VEC, NS, kStaged>(acc, in[i], 0, LP, l, pt, p, hlds, vs, rot);
          if (ln.lane_on) store_any_rot<VT, VEC>(p.out, out_off(row), p.out_bf16 != 0, rot, acc);
        }
      }
    }
  } else {
    for (int q = q_first; q < q_hi; q += ln.qpp) {
      const int64_t row = (static_cast<int64_t>(it.b) * p.queries + q) * p.rheads + rh;
      float acc[VEC];
#pragma unroll
      for (int k = 0; k < VEC; ++k) acc[k] = 0.0f;
      int l = 0, pt = 0;
      SoftmaxStats st{};
      if constexpr (kFused) st = softmax_stats(p.attn + row * LP, LP);
      constexpr int PB = pass_batch(kFused);
      for (int s0 = 0; s0 < LP; s0 += PB) {
        SampleIn<PB> f;
        load_in<PB>(f, loc2 + row * LP, p.attn + row * LP, s0, LP);
        if constexpr (kFused) {
          FusedIn<PB, true> x;
          load_refs<PB>(x, p, bq0 + q, s0, LP, l, pt);
          fused_prologue<PB>(f, x, st, p, s0, LP, l, pt);
        }
        fwd_pass<VT, VEC, PB, kStaged>(acc, f, s0, LP, l, pt, p, hlds, vs, rot);
      }
      if (ln.lane_on) store_any_rot<VT, VEC>(p.out, out_off(row), p.out_bf16 != 0, rot, acc);
    }
  }
}

// base[idx] with the byte offset formed in 32 bits (the caller guarantees idx * sizeof(T) < 2^32):
// a uniform base plus a 32-bit lane offset compiles to one address operand per access.
template <typename T>
__device__ __forceinline__ T* at(T* base, uint32_t idx) {
  using C = typename std::conditional<std::is_const<T>::value, const char, char>::type;
  return reinterpret_cast<T*>(reinterpret_cast<C*>(base) + idx * static_cast<uint32_t>(sizeof(T)));
}

}  // namespace msda

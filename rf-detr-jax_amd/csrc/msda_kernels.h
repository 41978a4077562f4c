// msda_kernels.h — gfx950 device code for multi-scale deformable attention (forward and VJP).
//
// Semantics follow RF-DETR-JAX's gather sampler, src/rfdetr_jax/models/ops.py:64-134 and
// ops.py:208-292: grid_sample(bilinear, zeros, align_corners=False) of each (batch, head) value
// slice at 2*loc-1, corner order (x0,y0),(x1,y0),(x0,y1),(x1,y1), masked weights multiplied onto
// values read at clipped indices, level-major point sum. Gradients are the VJP of those lines.
//
// Kernels:
//  * fwd_kernel — one workgroup per (batch b, group of hg heads, block of queries). The group's
//    value slices (the levels that fit) are staged into LDS with one batched copy; levels that do
//    not fit are gathered through L2. Lanes are laid out channel group, then head, then query, so
//    the lanes of one query read locations / weights and write output rows as contiguous runs of
//    the [B, Q, H, ...] tensors. Each lane group computes a sample's coordinates once.
//  * bwd_sample_kernel — the same decomposition for the backward pass: per sample, the dot
//    products D_c = <g, v_c> with the four corners give grad_attention_weights and
//    grad_sampling_locations, and a 16-byte record (floor cell, a*(1-fx), a*fx, fy) is written to
//    a workspace in slice-major order [b*H+h][l][q][p], which grad_value reads contiguously.
//  * bwd_value_kernel — one workgroup per (slice, level, band of rows). It reads its slice's
//    records, counting-sorts those whose cell touches the band by cell into LDS (integer LDS
//    atomics count and rank them), and has one lane per (cell, 4 channels) sum
//    a * w_k * g over the cell's records in registers, grad_output rows being gathered from global
//    memory. Corner k's sum goes to the k-th of four f32 band accumulators: for a fixed corner,
//    distinct cells hit distinct pixels, so no two lanes ever update one element and no atomics on
//    floats are needed; each grad_value element is written once, as the sum of the four, in the
//    value dtype.
//
// Measured on MI355X (per CU): LDS float atomics (ds_add_f32) cost ~195 cycles per wave
// instruction against ~6 for integer ones, and device-wide f32 atomics reach ~1.3 TB/s at best;
// hence no float atomics anywhere. Generic (flat) pointers to LDS cost vector-memory issue slots,
// so LDS reads go through address_space(3) pointers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace msda {

constexpr int kMaxLevels = 16;
constexpr int kXcds = 8;               // MI355X: 8 accelerator complex dies, workgroups dispatched round-robin
constexpr int kSampleMaxThreads = 1024;  // forward and per-sample backward workgroups
constexpr int kValueMaxThreads = 1024;  // grad_value workgroups
constexpr int kPassBatch = 4;           // samples whose location / weight loads are issued together

using bf16_t = uint16_t;

struct LevelDesc {
  int h, w;        // level height and width
  float fh, fw;    // the same, as floats
  int small;       // h * w * dim < 2^24: corner offsets fit 24-bit multiplies
  int start;       // first position of the level in the value slice
  int lds;         // per-sample kernels: element offset of the staged level inside a head's LDS region, -1 = L2
  int band_rows;   // grad_value kernel: image rows per band
  int band_first;  // grad_value kernel: index of the level's first band among a slice's (level, band) items
  uint32_t band_magic;  // ceil(2^32 / band_rows) (0 when band_rows == 1): row / band_rows = umulhi(row, magic)
};

// row / band_rows for 0 <= row < 2^16 and band_rows < 2^16: with magic = ceil(2^32 / band_rows),
// row * magic / 2^32 exceeds row / band_rows by less than 2^-16 < 1 / band_rows, so the floor is exact.
__device__ __forceinline__ int band_of(int row, const LevelDesc& L) {
  return L.band_rows == 1 ? row : static_cast<int>(__umulhi(static_cast<uint32_t>(row), L.band_magic));
}

// Forward and per-sample backward kernels.
struct SampleParams {
  const void* value;
  const float* loc;
  const float* attn;
  void* out;         // forward: output [B, Q, H*D]
  int out_bf16;
  const void* gout;  // backward: grad_output [B, Q, H*D]
  int gout_bf16;
  float* dloc;       // backward: grad_sampling_locations, or null
  float* dattn;      // backward: grad_attention_weights, or null
  uint4* bins;       // backward: grad_value records, binned by (slice, level band), or null
  int small_bins;    // a workgroup's bin region holds < 2^24 records (24-bit index arithmetic)
  int pair_share;    // forward: one level, two points, two lanes per (query, head) (fwd_pair)
  int* bin_counts;   // backward: records per (slice, level band, query block)
  int nwork;         // backward: (level, band) items per slice
  int heads, dim, queries, levels, points;
  int64_t len_value;
  int lpq_shift;   // log2(lanes per (query, head)); each lane owns VEC channels
  int hg;          // heads per workgroup (divides heads)
  int qblock;      // queries per workgroup
  int nqb;         // query blocks per (batch, head group)
  int head_lds;    // LDS elements of one head's staged levels
  int all_staged;  // every level is staged, so a head group's value rows are one contiguous copy
  int vec16;       // value staging may use 16-byte vectors
  // MSDeformAttn prologue fused in (kFused kernels, ops.py:388-404): `loc` then holds the raw
  // sampling offsets and `attn` the attention logits, and `dloc` / `dattn` receive their gradients.
  const float* ref;  // reference points [B, Q, L, ref_dim]
  int ref_dim;       // 2 (points) or 4 (boxes: centre, width, height)
  float fpoints;     // n_points as a float: the box form divides the offsets by it
  float inv_points;  // 1 / n_points when n_points is a power of two (x / P == x * (1 / P) exactly), else 0
  float* dref;       // backward: reference-point gradient per head group [H / hg, B * Q, L, ref_dim], or null
  int64_t bq_total;  // B * Q (rows per head group of `dref`)
  LevelDesc lv[kMaxLevels];
};

// A sample's record for grad_value, one per (sample, band its bilinear cell touches), in the bin of
// (slice, level band) and query block that produced it: `key` is the cell's index in the band's
// cell grid ((ky * (W + 1) + kx) with kx = x0 + 1, ky = y0 - r0 + 1; for non-finite weights the
// clipped first corner's cell), packed with the query's offset inside its query block; then
// u = a * (1 - fx), v = a * fx and fy, so that the corner weights are u*(1-fy), v*(1-fy), u*fy, v*fy.
struct __align__(16) SampleRec {
  uint32_t key_q;  // key | (query offset in block) << 16
  float u, v, fy;
};

struct ValueParams {
  const SampleRec* bins;   // [slice][item][query block][qblock * points]
  const int* bin_counts;   // [slice][item][query block]
  int nqb, qblock;         // query blocks of the per-sample pass, and their size
  const void* gout;
  int gout_bf16;
  void* dvalue;
  int heads, dim, queries, levels, points;
  int64_t len_value;
  int nwork;   // (level, band) items per slice
  int cap;     // records listed per segment (LDS list capacity)
  int g_vec4;  // grad_output rows may be read 4 channels at a time
  int vec16;   // grad_value rows may be written 16 bytes at a time
  // fused prologue: the reference-point gradient's sum over head groups, done by this kernel's
  // threads before their own work (ref_grad_sum), or ref_n = 0
  const float* ref_part;
  float* dref;
  int64_t ref_n;
  int ref_groups;
  LevelDesc lv[kMaxLevels];
};

// grad_reference_points [B, Q, L, ref_dim] (n elements) = the sum over head groups of the
// per-group partials [groups][n], added in group order, four groups' loads in flight at once.
// Thread `tid` of `nthreads` handles elements tid, tid + nthreads, ...
__device__ __forceinline__ void ref_grad_sum(const float* __restrict__ part, float* __restrict__ dref, int64_t n, int groups,
                                             int64_t tid, int64_t nthreads) {
  for (int64_t i = tid; i < n; i += nthreads) {
    const float* s = part + i;
    float acc = 0.0f;
    int g = 0;
    for (; g + 4 <= groups; g += 4) {
      const float a0 = s[(g + 0) * n], a1 = s[(g + 1) * n], a2 = s[(g + 2) * n], a3 = s[(g + 3) * n];
      acc = (((acc + a0) + a1) + a2) + a3;
    }
    for (; g < groups; ++g) acc += s[g * n];
    dref[i] = acc;
  }
}

// LDS carve-up of one grad_value workgroup; shared by the host planner and the kernel. Every
// region starts on a 16-byte boundary.
struct ValueLayout {
  int acc, cnt, off, misc, nonempty, binpre, list, total;
};

__host__ __device__ inline int align16i(int x) { return (x + 15) & ~15; }

__host__ __device__ inline ValueLayout value_layout(int band_rows, int w, int dim, int cap, int nqb, int nacc) {
  ValueLayout L;
  const int ncell = (band_rows + 1) * (w + 1);
  int o = 0;
  L.acc = o;      o += nacc * align16i(band_rows * w * dim * 4);  // one per bilinear corner, or one in all
  L.cnt = o;      o += align16i((ncell + 1) * 4);
  L.off = o;      o += align16i((ncell + 1) * 4);
  L.misc = o;     o += 128;  // 4 counters + one scan slot per wave (<= 16 waves) + spare
  L.nonempty = o; o += align16i(ncell * 2);
  L.binpre = o;   o += align16i((nqb + 1) * 4);
  L.list = o;     o += cap * 16;
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
  const float ix = pixel_coord(lx, L.fw);
  const float iy = pixel_coord(ly, L.fh);
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

// load_any_rot with a 32-bit element offset from a byte base (byte offset formed in 32 bits)
template <typename VT, int VEC>
__device__ __forceinline__ void load_any_rot32(const char* base, uint32_t off, bool is_bf16, int rot, float (&o)[VEC]) {
  constexpr int N = rot_chunks<VT, VEC>();
  constexpr int E = VEC / N;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const uint32_t e = off + static_cast<uint32_t>(((k + rot) & (N - 1)) * E);
    float t[E];
    if (is_bf16) load_vec<bf16_t, E>(reinterpret_cast<const bf16_t*>(base + e * 2u), t);
    else load_vec<float, E>(reinterpret_cast<const float*>(base + e * 4u), t);
#pragma unroll
    for (int i = 0; i < E; ++i) o[k * E + i] = t[i];
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
template <typename VT, bool kWait = true>
__device__ __forceinline__ void stage_copy(VT* dst, const VT* __restrict__ src, int count, bool vec16) {
  constexpr int U = 8;
  const int nt = blockDim.x;
  if (vec16) {
    const int n16 = static_cast<int>((static_cast<int64_t>(count) * sizeof(VT)) / 16);
    const uint4* s = reinterpret_cast<const uint4*>(src);
    uint4* d = reinterpret_cast<uint4*>(dst);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = nt >> 6;
    const int nblk = n16 >> 6;  // whole 1 KB blocks
    for (int blk = wave; blk < nblk; blk += nwaves)
      __builtin_amdgcn_global_load_lds(s + blk * 64 + lane, (MSDA_LDS void*)(d + blk * 64), 16, 0, 0);
    for (int i = (nblk << 6) + static_cast<int>(threadIdx.x); i < n16; i += nt) d[i] = s[i];
    if constexpr (kWait) wait_vmem();
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
// are one contiguous copy.
template <typename VT>
__device__ __forceinline__ void stage_group(const SampleParams& p, VT* lds, const VT* __restrict__ vg) {
  const int64_t slice_elems = p.len_value * p.dim;
  if (p.all_staged) {
    stage_copy(lds, vg, static_cast<int>(p.hg * slice_elems), p.vec16);
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
// before the first is used, so a lane waits one memory latency per group rather than per query;
// the backward also holds each query's grad_output row (VEC floats), so it groups fewer (sized so
// that no instantiation spills registers at four waves per SIMD).
constexpr int query_group(int ns, int vec, bool backward, bool fused = false) {
  if (ns == 0) return 1;
  // + a reference point and a box offset per sample, and the backward's dA per sample
  if (fused) return backward ? 1 : vec >= 8 ? (ns <= 2 ? 2 : 1) : (ns <= 2 ? 4 : 2);
  if (!backward) return ns <= 2 ? 4 : 2;
  if (vec >= 16) return ns <= 2 ? 2 : 1;
  if (vec == 8) return 2;
  return ns <= 2 ? 4 : 2;
}

// Samples per chunk of the per-query loop (NS = 0); the fused prologue's per-sample reference
// points and box offsets make the chunk half as long, within the same register budget.
constexpr int pass_batch(bool fused) { return fused ? 2 : kPassBatch; }

template <int NS, int QU>
__device__ __forceinline__ void load_group(SampleIn<NS> (&in)[QU], const float2* __restrict__ loc2, const float* __restrict__ attn,
                                           int64_t row0, int64_t row_step, int q0, int q_step, int q_hi, int LP) {
#pragma unroll
  for (int i = 0; i < QU; ++i) {
    if (q0 + i * q_step < q_hi) {
      const int64_t row = row0 + i * row_step;
      load_in<NS>(in[i], loc2 + row * LP, attn + row * LP, 0, LP);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// MSDeformAttn prologue fused into the per-sample kernels (ops.py:388-404): sample locations from
// reference points and raw offsets, attention weights from a softmax over each (query, head)'s
// L*P logits; and, in the backward, the gradients of offsets, logits and reference points.

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
__device__ __forceinline__ float2 fused_location(float2 off, float4 r, float2& t, const LevelDesc& L, const SampleParams& p) {
#pragma clang fp contract(off)
  if (p.ref_dim == 2) {
    t = off;
    return make_float2(r.x + off.x / L.fw, r.y + off.y / L.fh);
  }
  t = p.inv_points != 0.0f ? make_float2(off.x * p.inv_points, off.y * p.inv_points)
                           : make_float2(off.x / p.fpoints, off.y / p.fpoints);
  return make_float2(r.x + (t.x * r.z) * 0.5f, r.y + (t.y * r.w) * 0.5f);
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

// Backward state of one (query, head) row: sum_k a_k dA_k for the softmax VJP, and the running
// reference-point gradient of the current level (x, y, and w, h for boxes).
struct FusedAcc {
  float S;
  float r[4];
};

// Gradients of one sample from the core's (grad_loc, dA): the offset gradient (the transpose of
// fused_location: grad_loc / (W_l, H_l), or ((grad_loc * 0.5) * ref_wh) / n_points) and the
// sample's share of the reference-point gradient (grad_loc, and (grad_loc * 0.5) * t for w, h).
__device__ __forceinline__ float2 fused_sample_grads(float2 gl, float a, float dA, float4 r, float2 t, const LevelDesc& L,
                                                     const SampleParams& p, FusedAcc& fa) {
  fa.S += a * dA;
  fa.r[0] += gl.x;
  fa.r[1] += gl.y;
  if (p.ref_dim == 2) return make_float2(gl.x / L.fw, gl.y / L.fh);
  const float hx = gl.x * 0.5f, hy = gl.y * 0.5f;
  fa.r[2] += hx * t.x;
  fa.r[3] += hy * t.y;
  if (p.inv_points != 0.0f) return make_float2((hx * r.z) * p.inv_points, (hy * r.w) * p.inv_points);
  return make_float2((hx * r.z) / p.fpoints, (hy * r.w) / p.fpoints);
}

// End of a level: sums the reference-point gradient over the head group's lanes (hg * lanes per
// (query, head) <= 64, a power of two, so the group is aligned inside one wave) and writes it for
// (head group, b, q, level); the sum over groups is ref_grad_kernel's.
__device__ __forceinline__ void flush_ref_grad(FusedAcc& fa, const SampleParams& p, int hl, int j, int64_t bq, int group,
                                               int l) {
  const int lpq = 1 << p.lpq_shift;
  for (int o = lpq; o < (lpq * p.hg); o <<= 1) {
#pragma unroll
    for (int k = 0; k < 4; ++k) fa.r[k] += __shfl_xor(fa.r[k], o, 64);
  }
  if (p.dref != nullptr && hl == 0 && j == 0) {
    // group-major [H / hg][B * Q][L][ref_dim], so the reduction reads each group's rows contiguously
    float* d = p.dref + ((static_cast<int64_t>(group) * p.bq_total + bq) * p.levels + l) * p.ref_dim;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < p.ref_dim) d[k] = fa.r[k];  // constant indices keep fa.r in registers
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) fa.r[k] = 0.0f;
}

// Softmax VJP of one row, after every sample's dA is in grad_logits:
// grad_logit_k = a_k * (dA_k - sum_j a_j dA_j) (the transpose of jax.nn.softmax's JVP).
__device__ __forceinline__ void fused_logit_grads(const float* __restrict__ logits, float* glog, int LP, SoftmaxStats st,
                                                  float S) {
  for (int k = 0; k < LP; ++k) glog[k] = softmax_weight(logits[k], st) * (glog[k] - S);
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
      if (kStaged || L.lds >= 0) fwd_corners<VT, VEC, true>(acc, hlds + L.lds, c, f.a[u], rot);
      else fwd_corners<VT, VEC, false>(acc, vs + static_cast<int64_t>(L.start) * D, c, f.a[u], rot);
      if (++pt == p.points) {
        pt = 0;
        ++l;
      }
    }
  }
}

// One level, two points, two lanes per (query, head) (pair_share): lane j computes the corner
// offsets and weights of sample j only and the two lanes exchange them, so each sample's
// coordinates are computed once; each lane then adds its own sample first (the order of the two
// f32 additions per channel is the only difference from fwd_pass).
template <typename VT, int VEC>
__device__ __forceinline__ void fwd_pair(float (&acc)[VEC], const SampleIn<2>& f, const SampleParams& p, const VT* hlds,
                                         int rot, int j) {
  const LevelDesc L = p.lv[0];
  const float2 xy = j ? f.xy[1] : f.xy[0];
  const float a = j ? f.a[1] : f.a[0];
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
  const VT* __restrict__ vg = static_cast<const VT*>(p.value) + (static_cast<int64_t>(it.b) * p.heads + it.h0) * slice_elems;
  const int h = it.h0 + ln.hl;
  const int LP = p.levels * p.points;
  const int q_lo = it.qb * p.qblock;
  const int q_hi = min(p.queries, q_lo + p.qblock);
  const float2* __restrict__ loc2 = reinterpret_cast<const float2*>(p.loc);
  constexpr int QU = query_group(NS, VEC, false, kFused);
  constexpr int NI = NS == 0 ? 1 : NS;
  const int q_first = q_lo + ln.qs;
  const int64_t row_first = (static_cast<int64_t>(it.b) * p.queries + q_first) * p.heads + h;  // (b, q, h)
  const int64_t row_step = static_cast<int64_t>(ln.qpp) * p.heads;
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
  if constexpr (NS > 0)
    if (ln.active) {
      load_group<NS, QU>(in, loc2, p.attn, row_first, row_step, q_first, ln.qpp, q_hi, LP);
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
        load_group<NS, QU>(in, loc2, p.attn, row0, row_step, qg, ln.qpp, q_hi, LP);
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
              fwd_pair<VT, VEC>(acc, in[i], p, hlds, rot, ln.j);
              if (ln.lane_on) store_any_rot<VT, VEC>(p.out, row * D + ln.c0, p.out_bf16 != 0, rot, acc);
              continue;
            }
          }
          int l = 0, pt = 0;  // level and point of the next sample (level-major order, ops.py:285)
          fwd_pass<VT, VEC, NS, kStaged>(acc, in[i], 0, LP, l, pt, p, hlds, vs, rot);
          if (ln.lane_on) store_any_rot<VT, VEC>(p.out, row * D + ln.c0, p.out_bf16 != 0, rot, acc);
        }
      }
    }
  } else {
    for (int q = q_first; q < q_hi; q += ln.qpp) {
      const int64_t row = (static_cast<int64_t>(it.b) * p.queries + q) * p.heads + h;
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
      if (ln.lane_on) store_any_rot<VT, VEC>(p.out, row * D + ln.c0, p.out_bf16 != 0, rot, acc);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// backward, per sample: grad_attention_weights, grad_sampling_locations, grad_value records

template <typename VT, int VEC, bool kLds>
__device__ __forceinline__ void corner_dots(const VT* base, const Bilinear& c, const float (&g)[VEC], float& d00,
                                            float& d10, float& d01, float& d11, int rot) {
  float u0[VEC], u1[VEC];
  load_rot<VT, VEC, kLds>(base + c.o00, rot, u0);
  load_rot<VT, VEC, kLds>(base + c.o10, rot, u1);
  d00 = 0.0f;
  d10 = 0.0f;
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    d00 = fmaf(g[k], u0[k], d00);
    d10 = fmaf(g[k], u1[k], d10);
  }
  load_rot<VT, VEC, kLds>(base + c.o01, rot, u0);
  load_rot<VT, VEC, kLds>(base + c.o11, rot, u1);
  d01 = 0.0f;
  d11 = 0.0f;
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    d01 = fmaf(g[k], u0[k], d01);
    d11 = fmaf(g[k], u1[k], d11);
  }
}

// Appends a record to the bin of (slice n, item) for this workgroup's query block; the rank comes
// from the workgroup's LDS counter of that (head, item).
// base[idx] with the byte offset formed in 32 bits (the caller guarantees idx * sizeof(T) < 2^32):
// a uniform base plus a 32-bit lane offset compiles to one address operand per access.
template <typename T>
__device__ __forceinline__ T* at(T* base, uint32_t idx) {
  using C = typename std::conditional<std::is_const<T>::value, const char, char>::type;
  return reinterpret_cast<T*>(reinterpret_cast<C*>(base) + idx * static_cast<uint32_t>(sizeof(T)));
}

// Per-workgroup bases of the per-sample pass: row (b, q_lo, h0) of the [B, Q, H, ...] tensors and
// the record bins of slice (b, h0). Lanes index them with 32-bit offsets.
struct SampleBases {
  const float2* loc;
  const float* attn;
  const char* gout;  // bytes
  float* dattn;
  float2* dloc;
  uint4* bins;
};

__device__ __forceinline__ void emit_record(const SampleParams& p, const SampleBases& sb, int* lcnt, int hl, int item, int key,
                                            int qoff, int qb, uint4 payload) {
  const int pos = atomicAdd(&lcnt[hl * p.nwork + item], 1);
  payload.x = static_cast<uint32_t>(key) | (static_cast<uint32_t>(qoff) << 16);
  // bins of the workgroup's slices: [hg][nwork][nqb][qblock * points]; below 2^24 records in all
  // (small_bins) every factor fits a 24-bit multiply, and the region stays below 2^28 records
  // (16-byte offsets in 32 bits) in any case (both checked on the host)
  const uint32_t subcap = static_cast<uint32_t>(p.qblock) * static_cast<uint32_t>(p.points);
  uint32_t idx;
  if (p.small_bins) {
    const uint32_t bin = __umul24(__umul24(static_cast<uint32_t>(hl), static_cast<uint32_t>(p.nwork)) + static_cast<uint32_t>(item),
                                  static_cast<uint32_t>(p.nqb)) + static_cast<uint32_t>(qb);
    idx = __umul24(bin, subcap) + static_cast<uint32_t>(pos);
  } else {
    idx = ((static_cast<uint32_t>(hl) * p.nwork + item) * p.nqb + qb) * subcap + static_cast<uint32_t>(pos);
  }
  *at(sb.bins, idx) = payload;
}

// kKeepDA (fused, grouped path): each sample's dA stays in dA_out for the softmax VJP, instead
// of passing through grad_logits in memory.
template <typename VT, int VEC, int N, bool kStaged, bool kFused, bool kKeepDA = false>
__device__ __forceinline__ void bwd_pass(const SampleIn<N>& f, const FusedIn<N, kFused>& x, FusedAcc& fa, const float (&g)[VEC],
                                         int s0, int LP, int& l, int& pt, const SampleParams& p, const SampleLane& ln,
                                         const VT* hlds, const VT* __restrict__ vs, const SampleBases& sb, uint32_t lrow, int* lcnt,
                                         int qoff, int qb, int64_t bq, int group, float (&dA_out)[N]) {
  const int D = p.dim;
  const int lpq = 1 << p.lpq_shift;
#pragma unroll
  for (int u = 0; u < N; ++u) {
    if (s0 + u < LP) {
      const LevelDesc L = p.lv[l];
      const Bilinear c = bilinear(f.xy[u].x, f.xy[u].y, L, D);
      const float a = f.a[u];
      float d00, d10, d01, d11;
      if (kStaged || L.lds >= 0) corner_dots<VT, VEC, true>(hlds + L.lds, c, g, d00, d10, d01, d11, ln.rot);
      else corner_dots<VT, VEC, false>(vs + static_cast<int64_t>(L.start) * D, c, g, d00, d10, d01, d11, ln.rot);
      d00 = group_sum(d00, lpq);
      d10 = group_sum(d10, lpq);
      d01 = group_sum(d01, lpq);
      d11 = group_sum(d11, lpq);
      const uint32_t si = lrow * static_cast<uint32_t>(LP) + static_cast<uint32_t>(s0 + u);  // sample, from the workgroup's row
      if constexpr (kFused) {
        // every lane of the head group forms the sample's gradients (their sums over heads are
        // shuffled between lanes at the end of the level); lane 0 of the (query, head) writes
        const float dA = c.w00 * d00 + c.w10 * d10 + c.w01 * d01 + c.w11 * d11;
        const float g00 = c.m00 * d00, g10 = c.m10 * d10, g01 = c.m01 * d01, g11 = c.m11 * d11;
        const float dx = (1.0f - c.fy) * (g10 - g00) + c.fy * (g11 - g01);
        const float dy = (1.0f - c.fx) * (g01 - g00) + c.fx * (g11 - g10);
        const float2 gl = make_float2(a * L.fw * dx, a * L.fh * dy);
        const float2 goff = fused_sample_grads(gl, a, dA, x.r[u], x.t[u], L, p, fa);
        if constexpr (kKeepDA) dA_out[u] = dA;
        if (ln.j == 0) {
          if (!kKeepDA && sb.dattn) *at(sb.dattn, si) = dA;  // grad_logits holds dA until fused_logit_grads
          if (sb.dloc) *at(sb.dloc, si) = goff;
        }
        if (p.dref != nullptr && pt + 1 == p.points) flush_ref_grad(fa, p, ln.hl, ln.j, bq, group, l);
      }
      if (ln.j == 0) {
        if constexpr (!kFused) {
          // dA = sum_c w_c D_c (the sample itself); d out / d ix = gy (m10 D10 - m00 D00) + fy (m11 D11 - m01 D01)
          if (sb.dattn) *at(sb.dattn, si) = c.w00 * d00 + c.w10 * d10 + c.w01 * d01 + c.w11 * d11;
          if (sb.dloc) {
            const float g00 = c.m00 * d00, g10 = c.m10 * d10, g01 = c.m01 * d01, g11 = c.m11 * d11;
            const float dx = (1.0f - c.fy) * (g10 - g00) + c.fy * (g11 - g01);
            const float dy = (1.0f - c.fx) * (g01 - g00) + c.fx * (g11 - g10);
            // d ix / d loc = W (ops.py:270, :83): grid = 2 loc - 1, ix = ((grid + 1) W - 1) / 2
            *at(sb.dloc, si) = make_float2(a * L.fw * dx, a * L.fh * dy);
          }
        }
        if (p.bins) {
          // Non-finite weights (NaN or infinite coordinates) go to the clipped first corner's cell,
          // where the reference's scatter-add puts them.
          const bool finite = isfinite(c.w00) && isfinite(c.w10) && isfinite(c.w01) && isfinite(c.w11);
          const int x0 = finite ? c.x0 : c.cx0, y0 = finite ? c.y0 : c.cy0;
          const uint4 payload = make_uint4(0u, __float_as_uint(a * (1.0f - c.fx)), __float_as_uint(a * c.fx), __float_as_uint(c.fy));
          // the cell's rows y0, y0 + 1 that lie in the level, and the band of each
          if (x0 >= -1 && x0 <= L.w - 1) {
            const int ya = y0 >= 0 && y0 < L.h ? y0 : -1;
            const int yb = y0 + 1 >= 0 && y0 + 1 < L.h ? y0 + 1 : -1;
            const int ba = ya >= 0 ? band_of(ya, L) : -1;
            const int bb = yb >= 0 ? band_of(yb, L) : -1;
            // key: the cell's (row within the band + 1, x0 + 1), row-major over (band_rows + 1) x (w + 1)
            auto key = [&](int band) {
              const uint32_t r = static_cast<uint32_t>(y0 + 1) - __umul24(static_cast<uint32_t>(band), static_cast<uint32_t>(L.band_rows));
              return static_cast<int>(__umul24(r, static_cast<uint32_t>(L.w + 1)) + static_cast<uint32_t>(x0 + 1));
            };
            if (ba >= 0) emit_record(p, sb, lcnt, ln.hl, L.band_first + ba, key(ba), qoff, qb, payload);
            if (bb >= 0 && bb != ba) emit_record(p, sb, lcnt, ln.hl, L.band_first + bb, key(bb), qoff, qb, payload);
          }
        }
      }
      if (++pt == p.points) {
        pt = 0;
        ++l;
      }
    }
  }
}

// kFused: `loc` / `attn` are raw offsets and logits; `dloc` / `dattn` receive grad_offsets /
// grad_logits and `dref` the per-head-group reference-point gradients.
template <typename VT, int VEC, int NS, bool kStaged, bool kFused>
__global__ void __launch_bounds__(kSampleMaxThreads) __attribute__((amdgpu_waves_per_eu(4)))
bwd_sample_kernel(const SampleParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  VT* lds = reinterpret_cast<VT*>(lds_raw);
  const SampleItem it = sample_item(p);
  const SampleLane ln = sample_lane<VT, VEC>(p);
  const int D = p.dim;
  const int64_t slice_elems = p.len_value * D;
  const VT* __restrict__ vg = static_cast<const VT*>(p.value) + (static_cast<int64_t>(it.b) * p.heads + it.h0) * slice_elems;
  const int LP = p.levels * p.points;
  const int q_lo = it.qb * p.qblock;
  const int q_hi = min(p.queries, q_lo + p.qblock);
  const bool gbf = p.gout_bf16 != 0;
  // the workgroup's row (b, q_lo, h0) of the [B, Q, H, ...] tensors and its slices' record bins;
  // lane row r = (q - q_lo) * H + hl indexes them with 32-bit offsets
  const int64_t wrow = (static_cast<int64_t>(it.b) * p.queries + q_lo) * p.heads + it.h0;
  SampleBases sb;
  sb.loc = reinterpret_cast<const float2*>(p.loc) + wrow * LP;
  sb.attn = p.attn + wrow * LP;
  sb.gout = static_cast<const char*>(p.gout) + wrow * D * (gbf ? 2 : 4);
  sb.dattn = p.dattn ? p.dattn + wrow * LP : nullptr;
  sb.dloc = p.dloc ? reinterpret_cast<float2*>(p.dloc) + wrow * LP : nullptr;
  sb.bins = p.bins ? p.bins + (static_cast<int64_t>(it.b) * p.heads + it.h0) * p.nwork * p.nqb * static_cast<int64_t>(p.qblock) * p.points
                   : nullptr;
  auto lrow_of = [&](int q) { return __umul24(static_cast<uint32_t>(q - q_lo), static_cast<uint32_t>(p.heads)) + static_cast<uint32_t>(ln.hl); };
  // per (head, item) record counters of this workgroup, after the staged value rows
  int* lcnt = reinterpret_cast<int*>(lds_raw + align16i(p.hg * p.head_lds * static_cast<int>(sizeof(VT))));
  const int ncnt = p.bins ? p.hg * p.nwork : 0;
  for (int i = threadIdx.x; i < ncnt; i += blockDim.x) lcnt[i] = 0;
  constexpr int QU = query_group(NS, VEC, true, kFused);
  constexpr int NI = NS == 0 ? 1 : NS;
  const int q_first = q_lo + ln.qs;
  const uint32_t lrow_first = lrow_of(q_first);
  const uint32_t lrow_step = __umul24(static_cast<uint32_t>(ln.qpp), static_cast<uint32_t>(p.heads));
  const int64_t bq0 = static_cast<int64_t>(it.b) * p.queries;
  const int group = it.h0 / p.hg;
  SampleIn<NI> in[QU];
  float g[QU][VEC];
  // grad_output rows and sample inputs of a group of queries are requested together; the first
  // group's before the staging copy, so their latency overlaps it.
  auto load_gout = [&](uint32_t lrow0, int q0) {
#pragma unroll
    for (int i = 0; i < QU; ++i) {
      if (q0 + i * ln.qpp < q_hi) {
        if (ln.lane_on) {
          load_any_rot32<VT, VEC>(sb.gout, (lrow0 + i * lrow_step) * static_cast<uint32_t>(D) + static_cast<uint32_t>(ln.c0), gbf,
                                  ln.rot, g[i]);
        } else {
#pragma unroll
          for (int k = 0; k < VEC; ++k) g[i][k] = 0.0f;
        }
      }
    }
  };
  FusedIn<NI, kFused> fin[QU];
  auto load_inputs = [&](uint32_t lrow0, int q0) {
#pragma unroll
    for (int i = 0; i < QU; ++i)
      if (q0 + i * ln.qpp < q_hi) {
        const uint32_t r = (lrow0 + i * lrow_step) * static_cast<uint32_t>(LP);
        load_in<NI>(in[i], at(sb.loc, r), at(sb.attn, r), 0, LP);
        if constexpr (kFused) load_refs<NI>(fin[i], p, bq0 + q0 + i * ln.qpp, 0, LP, 0, 0);
      }
  };
  if constexpr (NS > 0) {
    if (ln.active) {
      load_gout(lrow_first, q_first);
      load_inputs(lrow_first, q_first);
    }
  }
  stage_group(p, lds, vg);
  __syncthreads();

  const VT* __restrict__ vs = vg + ln.hl * slice_elems + ln.c0;
  const VT* hlds = lds + ln.hl * p.head_lds + ln.c0;
  if constexpr (NS > 0) {
    uint32_t lrow0 = lrow_first;
    for (int qg = q_first; ln.active && qg < q_hi; qg += QU * ln.qpp, lrow0 += QU * lrow_step) {
      if (qg != q_first) {
        load_gout(lrow0, qg);
        load_inputs(lrow0, qg);
      }
      wait_vmem();
#pragma unroll
      for (int i = 0; i < QU; ++i) {
        const int q = qg + i * ln.qpp;
        if (q < q_hi) {
          int l = 0, pt = 0;
          FusedAcc fa{};
          float dA[NI];
          if constexpr (kFused) fused_prologue_row<NI>(in[i], fin[i], p, LP);
          const uint32_t lrow = lrow0 + i * lrow_step;
          bwd_pass<VT, VEC, NS, kStaged, kFused, kFused>(in[i], fin[i], fa, g[i], 0, LP, l, pt, p, ln, hlds, vs, sb, lrow, lcnt,
                                                         q - q_lo, it.qb, bq0 + q, group, dA);
          if constexpr (kFused) {
            // softmax VJP from registers: grad_logit_u = a_u (dA_u - sum_k a_k dA_k)
            if (sb.dattn && ln.j == 0) {
#pragma unroll
              for (int u = 0; u < NI; ++u)
                if (u < LP) *at(sb.dattn, lrow * static_cast<uint32_t>(LP) + u) = in[i].a[u] * (dA[u] - fa.S);
            }
          }
        }
      }
    }
  } else {
    uint32_t lrow = lrow_first;
    for (int q = q_first; ln.active && q < q_hi; q += ln.qpp, lrow += lrow_step) {
      load_gout(lrow, q);
      int l = 0, pt = 0;
      const uint32_t r = lrow * static_cast<uint32_t>(LP);
      SoftmaxStats st{};
      FusedAcc fa{};
      if constexpr (kFused) st = softmax_stats(at(sb.attn, r), LP);
      constexpr int PB = pass_batch(kFused);
      for (int s0 = 0; s0 < LP; s0 += PB) {
        SampleIn<PB> f;
        FusedIn<PB, kFused> x;
        load_in<PB>(f, at(sb.loc, r), at(sb.attn, r), s0, LP);
        if constexpr (kFused) {
          load_refs<PB>(x, p, bq0 + q, s0, LP, l, pt);
          fused_prologue<PB>(f, x, st, p, s0, LP, l, pt);
        }
        float unused[PB];
        bwd_pass<VT, VEC, PB, kStaged, kFused>(f, x, fa, g[0], s0, LP, l, pt, p, ln, hlds, vs, sb, lrow, lcnt, q - q_lo, it.qb,
                                               bq0 + q, group, unused);
      }
      if constexpr (kFused)
        if (sb.dattn && ln.j == 0) fused_logit_grads(at(sb.attn, r), at(sb.dattn, r), LP, st, fa.S);
    }
  }
  if (!p.bins) return;
  // records per (slice, item) of this query block, for the grad_value pass
  __syncthreads();
  for (int i = threadIdx.x; i < ncnt; i += blockDim.x) {
    const int hh = i / p.nwork, item = i - hh * p.nwork;
    const int64_t nn = static_cast<int64_t>(it.b) * p.heads + it.h0 + hh;
    p.bin_counts[(nn * p.nwork + item) * p.nqb + it.qb] = lcnt[i];
  }
}

// ---------------------------------------------------------------------------------------------
// backward, grad_value: one workgroup per (slice, level, band of rows [r0, r1))

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

// CG channels of a grad_output row: `base` is the (b, q=0, h) row of this workgroup's slice and
// `off` a 32-bit element offset from it (nch channels valid; the rest read as 0).
template <int CG>
__device__ __forceinline__ void load_gc(const void* __restrict__ base, bool bf16, bool vec4, int off, int nch, float (&o)[CG]) {
  if (nch == CG && vec4) {
#pragma unroll
    for (int k = 0; k < CG; k += 4) {
      if (bf16) {
        const uint2 r = *reinterpret_cast<const uint2*>(static_cast<const bf16_t*>(base) + off + k);
        o[k] = __uint_as_float(r.x << 16);
        o[k + 1] = __uint_as_float(r.x & 0xffff0000u);
        o[k + 2] = __uint_as_float(r.y << 16);
        o[k + 3] = __uint_as_float(r.y & 0xffff0000u);
      } else {
        const float4 r = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + off + k);
        o[k] = r.x;
        o[k + 1] = r.y;
        o[k + 2] = r.z;
        o[k + 3] = r.w;
      }
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < CG; ++e) {
    float x[1] = {0.0f};
    if (e < nch) load_any<1>(base, off + e, bf16, x);
    o[e] = x[0];
  }
}

// One grad_value task: s[k][e] += w_k * g[q][ch0 + e] over the records [ebeg, eend) of one cell,
// w_k the record's corner weights (ops.py:123-128 with the attention weight folded in, corner order
// 00, 10, 01, 11). MODE 0 / 1: f32 / bf16 rows of CG channels at 16-byte-aligned offsets, addressed
// by a 32-bit byte offset from the slice's first row (one address operation per row); MODE 2:
// any dtype, alignment and partial channel group.
template <int CG, int MODE>
__device__ __forceinline__ void cell_sums(const float4* list, int ebeg, int eend, const void* gbase, bool gbf, bool gv4,
                                          int ch0, int nch, int Q, int gqstride, float (&s)[4][CG]);

// grad_output rows a grad_value lane fetches together (with their weights): as many as the register
// budget holds next to the lane's 4 * CG corner sums.
constexpr int gather_batch(int cg) { return cg >= 8 ? 4 : 8; }

template <int CG, int MODE>
__device__ __forceinline__ void cell_sums(const float4* list, int ebeg, int eend, const void* gbase, bool gbf, bool gv4,
                                          int ch0, int nch, int Q, int gqstride, float (&s)[4][CG]) {
  constexpr int kGatherBatch = gather_batch(CG);
  const char* gb = static_cast<const char*>(gbase);
  for (int e0 = ebeg; e0 < eend; e0 += kGatherBatch) {
    float u[kGatherBatch], v[kGatherBatch], fy[kGatherBatch];
    float g[kGatherBatch][CG];
#pragma unroll
    for (int i = 0; i < kGatherBatch; ++i) {
      if (e0 + i < eend) {
        const float4 w = list[e0 + i];
        u[i] = w.x;
        v[i] = w.y;
        fy[i] = w.z;
        // the record's grad_output row offset (q * H * D, q clamped to Q - 1 when placed; < 2^30,
        // host-checked) plus this lane's channel group
        const unsigned el = static_cast<unsigned>(__float_as_int(w.w)) + static_cast<unsigned>(ch0);
        if constexpr (MODE == 0) {
          const float4* r = reinterpret_cast<const float4*>(gb + el * 4u);
#pragma unroll
          for (int k = 0; k < CG; k += 4) {
            const float4 x = r[k / 4];
            g[i][k] = x.x;
            g[i][k + 1] = x.y;
            g[i][k + 2] = x.z;
            g[i][k + 3] = x.w;
          }
        } else if constexpr (MODE == 1) {
          const uint2* r = reinterpret_cast<const uint2*>(gb + el * 2u);
#pragma unroll
          for (int k = 0; k < CG; k += 4) {
            const uint2 x = r[k / 4];
            g[i][k] = __uint_as_float(x.x << 16);
            g[i][k + 1] = __uint_as_float(x.x & 0xffff0000u);
            g[i][k + 2] = __uint_as_float(x.y << 16);
            g[i][k + 3] = __uint_as_float(x.y & 0xffff0000u);
          }
        } else {
          load_gc<CG>(gbase, gbf, gv4, static_cast<int>(el), nch, g[i]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kGatherBatch; ++i) {
      if (e0 + i < eend) {
        const float w00 = u[i] * (1.0f - fy[i]), w10 = v[i] * (1.0f - fy[i]);
        const float w01 = u[i] * fy[i], w11 = v[i] * fy[i];
#pragma unroll
        for (int e = 0; e < CG; ++e) {
          s[0][e] = fmaf(w00, g[i][e], s[0][e]);
          s[1][e] = fmaf(w10, g[i][e], s[1][e]);
          s[2][e] = fmaf(w01, g[i][e], s[2][e]);
          s[3][e] = fmaf(w11, g[i][e], s[3][e]);
        }
      }
    }
  }
}

// CG: channels per gather lane (4 or 8). NACC: 4 = one accumulator per bilinear corner (conflict-free,
// no colour passes); 1 = a single accumulator updated in four colour passes per round of tasks
// (cells of one x/y parity never share a pixel), for bands where four accumulators do not fit.
// Four waves per SIMD (<= 128 VGPRs) let two 512-thread workgroups share a CU.
template <typename VT, int CG, int NACC>
__global__ void __launch_bounds__(kValueMaxThreads) __attribute__((amdgpu_waves_per_eu(4)))
bwd_value_kernel(const ValueParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  if (p.ref_n > 0)
    ref_grad_sum(p.ref_part, p.dref, p.ref_n, p.ref_groups, static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x,
                 static_cast<int64_t>(gridDim.x) * blockDim.x);

  const int lid = xcd_logical(blockIdx.x, gridDim.x);
  const int h = lid % p.heads;
  const int rest = lid / p.heads;
  // Items in reverse order: the bands of the coarsest level start first. A level's samples are
  // split over its bands, so a coarse level's few bands hold the most records each; started last
  // (behind a fine level's many light bands), they would set the kernel's tail.
  const int wk = p.nwork - 1 - rest % p.nwork;
  const int b = rest / p.nwork;
  int l = 0;
  while (l + 1 < p.levels && wk >= p.lv[l + 1].band_first) ++l;
  const LevelDesc L = p.lv[l];
  const int W = L.w;
  const int r0 = (wk - L.band_first) * L.band_rows;
  const int r1 = min(L.h, r0 + L.band_rows);
  const int rb = r1 - r0;
  const int D = p.dim;
  const int P = p.points;
  const int Q = p.queries;
  const int ncell = (rb + 1) * (W + 1);
  const int64_t n = static_cast<int64_t>(b) * p.heads + h;
  const int nt = blockDim.x, t = threadIdx.x, lane = t & 63;

  const ValueLayout lay = value_layout(L.band_rows, W, D, p.cap, p.nqb, NACC);
  float* acc = reinterpret_cast<float*>(lds_raw + lay.acc);
  int* cnt = reinterpret_cast<int*>(lds_raw + lay.cnt);
  int* off = reinterpret_cast<int*>(lds_raw + lay.off);
  int* misc = reinterpret_cast<int*>(lds_raw + lay.misc);  // [2] non-empty cells, [4..] scan scratch
  uint16_t* nonempty = reinterpret_cast<uint16_t*>(lds_raw + lay.nonempty);
  int* binpre = reinterpret_cast<int*>(lds_raw + lay.binpre);
  float4* list = reinterpret_cast<float4*>(lds_raw + lay.list);  // segment's records, in cell order

  // With four accumulators, one per bilinear corner k, a cell adds its corner-k sum to accumulator
  // k, and distinct cells hit distinct pixels for a fixed k, so no two lanes ever update one element.
  const int acc_stride = align16i(L.band_rows * W * D * 4) / 4;  // floats between accumulators
  {
    const int na = (NACC - 1) * acc_stride + rb * W * D;
    float4* a4 = reinterpret_cast<float4*>(acc);
    for (int i = t; i < (na >> 2); i += nt) a4[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int i = (na & ~3) + t; i < na; i += nt) acc[i] = 0.0f;
    for (int i = t; i < ncell; i += nt) cnt[i] = 0;
    if (t < 4) misc[t] = 0;
  }

  // This workgroup's records: the bins of (slice n, item wk), one per query block of the
  // per-sample pass, with their counts; prefix sums of the counts in LDS.
  const int64_t subcap = static_cast<int64_t>(p.qblock) * P;
  const SampleRec* __restrict__ R = p.bins ? p.bins + (n * p.nwork + wk) * p.nqb * subcap : nullptr;
  const int* __restrict__ C = p.bin_counts ? p.bin_counts + (n * p.nwork + wk) * p.nqb : nullptr;
  // counts loaded in parallel, then an exclusive scan by the first wave (no bins without queries)
  for (int i = t; i < p.nqb; i += nt) binpre[i + 1] = C ? C[i] : 0;
  if (t == 0) binpre[0] = 0;
  __syncthreads();
  if (t < 64) {
    int carry = 0;
    for (int i0 = 0; i0 < p.nqb; i0 += 64) {
      const int i = i0 + lane;
      int v = i < p.nqb ? binpre[i + 1] : 0;
      for (int o = 1; o < 64; o <<= 1) {
        const int x = __shfl_up(v, o, 64);
        if (lane >= o) v += x;
      }
      if (i < p.nqb) binpre[i + 1] = carry + v;
      carry += __shfl(v, 63, 64);
    }
  }
  constexpr int U = 8;  // records loaded per thread before use
  // grad_output row (b, q=0, h); row q is q * H * D elements further (fits 32 bits: checked on the host)
  const int64_t grow0 = (static_cast<int64_t>(b) * Q * p.heads + h) * D;
  const void* gbase = p.gout_bf16 ? static_cast<const void*>(static_cast<const bf16_t*>(p.gout) + grow0)
                                  : static_cast<const void*>(static_cast<const float*>(p.gout) + grow0);
  const bool gbf = p.gout_bf16 != 0, gv4 = p.g_vec4 != 0;
  const int gqstride = p.heads * D;
  const int gpp = (D + CG - 1) / CG;  // channel groups per cell
  __syncthreads();  // counters cleared, prefix ready
  const int NR = binpre[p.nqb];
  // Record f of the workgroup lives in bin `qb` with binpre[qb] <= f < binpre[qb + 1]; a thread's f
  // only grows, so its bin index only moves forward.
  auto record = [&](int f, int& qb) {
    while (binpre[qb + 1] <= f) ++qb;
    return *reinterpret_cast<const uint4*>(R + qb * subcap + (f - binpre[qb]));
  };
  const int ncell_max = ncell;

  // Segments of at most `cap` records (a segment's records all fit the list).
  for (int s_lo = 0; s_lo < NR;) {
    const int s_hi = min(NR, s_lo + p.cap);
    // When the segment is at most U records per thread, pass A also copies each record into the
    // (not yet used) list LDS at its load position, and pass B reads it from there instead of
    // loading it from global memory again.
    const bool one_pass = s_hi - s_lo <= U * nt;
    uint4* stage = reinterpret_cast<uint4*>(list);
    // ---- pass A: per-cell counts
    {
      int qb = 0;
      for (int f = s_lo + t; f < s_hi; f += U * nt) {
        uint4 rr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) rr[u] = (f + u * nt < s_hi) ? record(f + u * nt, qb) : make_uint4(0xffffu, 0, 0, 0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const uint32_t key = rr[u].x & 0xffffu;
          if (static_cast<int>(key) < ncell_max) atomicAdd(&cnt[key], 1);
          if (one_pass && f + u * nt < s_hi) stage[f + u * nt - s_lo] = rr[u];
        }
      }
    }
    __syncthreads();
    // ---- cell offsets (counts cleared: they become the placement cursors) and non-empty cells
    block_scan_counts(cnt, off, ncell, misc + 4);
    for (int k0 = 0; k0 < ncell; k0 += nt) {
      const int key = k0 + t;
      const bool busy = key < ncell && off[key + 1] > off[key];
      const uint64_t mask = __ballot(busy);
      int base = 0;
      if (lane == 0 && mask) base = atomicAdd(&misc[2], __popcll(mask));
      base = __shfl(base, 0, 64);
      if (busy) nonempty[base + __popcll(mask & ((uint64_t{1} << lane) - 1))] = static_cast<uint16_t>(key);
    }
    // ---- pass B: each record goes to its place in cell order
    auto entry = [&](const uint4& r, int qb) {
      return make_float4(__uint_as_float(r.y), __uint_as_float(r.z), __uint_as_float(r.w),
                         __int_as_float(min(qb * p.qblock + static_cast<int>(r.x >> 16), Q - 1) * gqstride));
    };
    if (one_pass) {
      // records from the staging copy; every thread reads its records before any is placed
      uint4 rr[U];
      int qbs[U], pos[U];
      int qb = 0;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int f = s_lo + t + u * nt;
        if (f < s_hi) {
          while (binpre[qb + 1] <= f) ++qb;
          rr[u] = stage[f - s_lo];
        } else {
          rr[u] = make_uint4(0xffffu, 0, 0, 0);
        }
        qbs[u] = qb;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int key = static_cast<int>(rr[u].x & 0xffffu);
        pos[u] = key < ncell_max ? off[key] + atomicAdd(&cnt[key], 1) : -1;
      }
      __syncthreads();
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (pos[u] >= 0 && pos[u] < p.cap) list[pos[u]] = entry(rr[u], qbs[u]);
    } else {
      int qb = 0;
      for (int f = s_lo + t; f < s_hi; f += U * nt) {
        uint4 rr[U];
        int qbs[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          rr[u] = (f + u * nt < s_hi) ? record(f + u * nt, qb) : make_uint4(0xffffu, 0, 0, 0);
          qbs[u] = qb;
        }
        int pos[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int key = static_cast<int>(rr[u].x & 0xffffu);
          pos[u] = key < ncell_max ? off[key] + atomicAdd(&cnt[key], 1) : -1;
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (pos[u] >= 0 && pos[u] < p.cap) list[pos[u]] = entry(rr[u], qbs[u]);
      }
    }
    __syncthreads();
    const int ntask = misc[2] * gpp;
    // ---- one lane per (non-empty cell, CG channels) task: sum a * w_k * g over the cell's records
    //      in registers, kGatherBatch grad_output rows in flight, then add corner k's sum to
    //      accumulator k (conflict-free, so tasks need no barriers between them).
    for (int t0 = 0; t0 < ntask; t0 += nt) {
      const int task = t0 + t;
      int kx = 0, ky = 0, ch0 = 0, nch = 0, ebeg = 0, eend = 0;
      if (task < ntask) {
        const int ci = task / gpp, grp = task - ci * gpp;
        const int key = nonempty[ci];
        ky = key / (W + 1);
        kx = key - ky * (W + 1);
        ch0 = grp * CG;
        nch = min(CG, D - ch0);
        ebeg = off[key];
        eend = off[key + 1];
      }
      float s[4][CG];
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < CG; ++e) s[k][e] = 0.0f;
      // row loads specialised outside the record loop: f32 or bf16 rows of full 16-byte-aligned
      // channel groups, or the general path
      const int mode = (nch == CG && gv4) ? (gbf ? 1 : 0) : 2;
      if (mode == 0) cell_sums<CG, 0>(list, ebeg, eend, gbase, gbf, gv4, ch0, nch, Q, gqstride, s);
      else if (mode == 1) cell_sums<CG, 1>(list, ebeg, eend, gbase, gbf, gv4, ch0, nch, Q, gqstride, s);
      else cell_sums<CG, 2>(list, ebeg, eend, gbase, gbf, gv4, ch0, nch, Q, gqstride, s);
      // With one accumulator, cells of one colour (x and y parity) are updated per pass.
      const int color = (kx & 1) | ((ky & 1) << 1);
      for (int c = 0; c < (NACC == 4 ? 1 : 4); ++c) {
        if (task < ntask && (NACC == 4 || color == c)) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            // corner k of cell (kx, ky) is pixel (kx - 1 + (k & 1), ky - 1 + (k >> 1)) of the band
            const int px = kx - 1 + (k & 1), py = ky - 1 + (k >> 1);
            if (px >= 0 && px < W && py >= 0 && py < rb) {
              float* ap = acc + (NACC == 4 ? k * acc_stride : 0) + (py * W + px) * D + ch0;
              if (nch == CG && (D & 3) == 0) {
#pragma unroll
                for (int e = 0; e < CG; e += 4) {
                  float4 o = *reinterpret_cast<float4*>(ap + e);
                  o.x += s[k][e];
                  o.y += s[k][e + 1];
                  o.z += s[k][e + 2];
                  o.w += s[k][e + 3];
                  *reinterpret_cast<float4*>(ap + e) = o;
                }
              } else {
#pragma unroll
                for (int e = 0; e < CG; ++e)
                  if (e < nch) ap[e] += s[k][e];
              }
            }
          }
        }
        if (NACC == 1) __syncthreads();
      }
    }
    __syncthreads();  // every task done before the cell tables are reused
    // the placement cursors start the next segment at zero
    for (int i = t; i < ncell; i += nt) cnt[i] = 0;
    if (t == 0) misc[2] = 0;
    __syncthreads();
    s_lo = s_hi;
  }

  // ---- the band's grad_value rows, once, in the value dtype (the sum of the accumulators)
  VT* dst = static_cast<VT*>(p.dvalue) + (n * p.len_value + L.start + static_cast<int64_t>(r0) * W) * D;
  const int na = rb * W * D;
  if (p.vec16 && (na & 3) == 0) {
    for (int i = t; i < (na >> 2); i += nt) {
      float4 a = reinterpret_cast<const float4*>(acc)[i];
#pragma unroll
      for (int k = 1; k < NACC; ++k) {
        const float4 b = reinterpret_cast<const float4*>(acc + k * acc_stride)[i];
        a.x += b.x;
        a.y += b.y;
        a.z += b.z;
        a.w += b.w;
      }
      const float o[4] = {a.x, a.y, a.z, a.w};
      store_vec<VT, 4>(dst + 4 * i, o);
    }
  } else {
    for (int i = t; i < na; i += nt) {
      float o[1] = {acc[i]};
#pragma unroll
      for (int k = 1; k < NACC; ++k) o[0] += acc[i + k * acc_stride];
      store_vec<VT, 1>(dst + i, o);
    }
  }
}

}  // namespace msda

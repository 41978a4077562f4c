// msda_band_kernels.h — gfx950 backward of the deformable-attention core in one kernel.
//
// The VJP of RF-DETR-JAX's gather sampler (src/rfdetr_jax/models/ops.py:64-134, :208-292; the
// hand-written form of the same transpose is deform_pallas.py:97-120): for every sample
// (b, q, h, l, p) with corner weights w_c and attention weight a,
//   grad_value[cell_c] += w_c * a * g          (g = grad_output[b, q, h*D:(h+1)*D])
//   D_c = <g, value[cell_c]>,  grad_attn = sum_c w_c D_c,
//   grad_loc = a * (W, H) * (d/dix, d/diy) sum_c w_c D_c   (masks and floor have zero gradient).
//
// bwd_band_kernel: one workgroup per (slice n = b*H + h, item = (level l, band of image rows
// [r0, r1)), query block). With one query block the workgroup owns grad_value rows [r0, r1) of
// level l of slice n: every element has exactly one writer and nothing needs zeroing. When a
// level fits the LDS whole but the slices are too few to fill the CUs, the queries are split into
// blocks; each block writes an f32 partial sum of the rows, and bwd_part_sum_kernel adds the
// partials in block order.
//  1. Stage the band's value rows plus one halo row below into LDS (the rows a corner dot of a
//     sample whose floor row lies in the band can touch), zero an f64 accumulator for the band.
//  2. Banded levels only: scan. The threads read the locations of all queries at level l (a pass
//     holds as many queries as the list can hold points of; one pass at the usual shapes), several
//     loads in flight per thread, and append every point whose clipped corner rows meet the band to
//     an LDS list (wave ballot compaction), so the third phase runs on full waves.
//  3. Work items: a whole level's queries (all of a query's points), or the listed points; lps
//     lanes per item, CH channels each (lps = head_dim / CH). Waves take chunks of items from an
//     LDS counter, and a lane loads its next item's inputs before working on the current one. Per
//     point, the band that holds its clipped floor row computes the corner dots from the staged rows
//     and writes grad_attention_weights and grad_sampling_locations; every band its corner rows meet
//     adds a*w_c*g for its corners into the accumulator with ds_add_f64 (a*w_c is exact in f64;
//     its product with g is rounded to f64, and the sum is kept in f64).
//  4. Round the accumulator once to the value dtype and write the band's grad_value rows (or the
//     block's f32 partial rows).
//
// Measured on MI355X (per CU, 64-lane wave instructions, each written as the instruction): ds_add_f64
// 9.1 cycles with the 64 lanes on 64 consecutive doubles and 9.4 on random 16-double cells with
// rotated channels (17.1 on 8-double cells); ds_add_u64 7.0, ds_add_u32 5.0; but ds_add_f32,
// ds_add_rtn_f32 and ds_pk_add_bf16 193 cycles whatever the addresses, consecutive ones included
// (also with f32 denormals flushed). The accumulator is therefore f64 with 16-channel cells. Lane i
// of a sample-lane layout adds channel (t + r_i) mod 16 in instruction t, r_i = i mod 16: the lanes
// of one instruction then cover all 32 bank pairs of a 256-byte bank row twice (the same channel
// for every lane costs 63.5 cycles, a rotation by 16-byte chunks only 32.8).
#pragma once

#include "msda_kernels.h"

namespace msda {

constexpr int kBandMaxThreads = 1024;

struct BandParams {
  const void* value;  // [B*H, S, D]
  const float* loc;   // [B, Q, H, L, P, 2]
  const float* attn;  // [B, Q, H, L*P]
  const void* gout;   // [B, Q, H*D]
  int gout_bf16;
  void* dvalue;       // [B*H, S, D] in the value dtype, or null
  float* dloc;        // as loc, or null
  float* dattn;       // as attn, or null
  int heads, dim, queries, levels, points;
  int64_t len_value;
  int nwork;       // (level, band) items per slice
  int nqb;         // query blocks per (slice, item); with part, each block writes a partial sum
  int qblock;      // queries per block
  float* part;     // nqb > 1 and grad_value requested: partial grad_value sums [nqb][B*H][S][D] (f32),
                   // summed by bwd_part_sum_kernel; else null
  int64_t part_stride;  // B * H * S * D
  int qpass;       // queries scanned per pass (the list holds one entry per point of a pass)
  int lps_shift;   // log2(lanes per sample)
  int vec16;       // value rows and grad_value rows allow 16-byte accesses
  int lds_acc;     // byte offset of the f64 accumulator's first cell in LDS (one guard cell precedes
                   // it; the staged value rows start at 0)
  int lds_list;    // byte offset of the point list (entries: query offset << 16 | point)
  int lds_cnt;     // byte offset of the list counter
  LevelDesc lv[kMaxLevels];  // band_rows, band_first per level
  // The MSDeformAttn prologue in the kernel (FZ instantiations; one level, whole): `loc` holds the
  // sampling offsets and `attn` the attention logits, `dloc` receives grad_sampling_offsets and
  // `dattn` grad_attention_logits; locations and softmax weights are formed per (query, head) row
  // as the forward forms them (fused_location_at, softmax_regs), and the row's softmax VJP and
  // offset gradient follow its points. dref_part: [H][B * Q][ref_dim] per-head partial gradients
  // of the reference points (summed over the row's points in order), or null.
  const float* ref;  // [B, Q, 1, ref_dim]
  int ref_dim;
  float inv_points, fpoints;
  float* dref_part;
  int64_t bq_total;  // B * Q
  // whole levels: one work item per point rather than per query (fewer queries than the
  // workgroup's lanes can take two at a time; core op only)
  int point_items;
};

// Item k of a slice: level l (the last whose first item <= k) and band k - band_first.
struct BandItem {
  int l, r0, r1;
};

__device__ __forceinline__ BandItem band_item(const BandParams& p, int k) {
  int l = 0;
  while (l + 1 < p.levels && p.lv[l + 1].band_first <= k) ++l;
  BandItem it;
  it.l = l;
  it.r0 = (k - p.lv[l].band_first) * p.lv[l].band_rows;
  it.r1 = min(it.r0 + p.lv[l].band_rows, p.lv[l].h);
  return it;
}

// The clipped rows of a sample's two corner rows (ops.py:103-118 clip y0 and y0 + 1 into the
// level); a non-finite coordinate clamps to -2, i.e. both rows clip to 0, where bilinear() puts it.
__device__ __forceinline__ int2 clipped_rows(float ly, const LevelDesc& L) {
  const float iy = level_coord(ly, L.fh, L);
  const int y0 = static_cast<int>(fminf(fmaxf(floorf(iy), -2.0f), L.fh));
  return make_int2(min(max(y0, 0), L.h - 1), min(max(y0 + 1, 0), L.h - 1));
}

// Appends `entry` for the lanes with `flag` to an LDS list of 32-bit entries: one counter atomic
// per wave.
__device__ __forceinline__ void list_append32(bool flag, uint32_t entry, uint32_t* list, int* cnt) {
  const uint64_t m = __ballot(flag);
  if (m == 0) return;
  const int lane = threadIdx.x & 63;
  const int leader = __ffsll(static_cast<long long>(m)) - 1;
  int base = 0;
  if (lane == leader) base = atomicAdd(cnt, __popcll(m));
  base = __shfl(base, leader, 64);
  const uint32_t lo = static_cast<uint32_t>(m), hi = static_cast<uint32_t>(m >> 32);
  const int rank = static_cast<int>(__builtin_amdgcn_mbcnt_hi(hi, __builtin_amdgcn_mbcnt_lo(lo, 0u)));
  if (flag) list[base + rank] = entry;
}

// dst = (bit `lane` of mask) ? a : b. Written as the instruction itself: a C++ select between two
// array elements is folded by the compiler into a load at a selected index, which after unrolling
// becomes a dynamic register index (a 16-way select chain per element).
__device__ __forceinline__ float lane_select(float a, float b, uint64_t mask) {
  float r;
  asm("v_cndmask_b32_e64 %0, %2, %1, %3" : "=v"(r) : "v"(a), "v"(b), "s"(mask));
  return r;
}

// x rotated down by b places (x[t] <- x[(t + b) mod N]), b < 2^STEPS: stage s rotates by 2^s in
// the lanes whose bit s of b is set.
template <int N, int STEPS>
__device__ __forceinline__ void rotate_regs(float (&x)[N], int b) {
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int k = 1 << s;
    const uint64_t on = __ballot((b >> s) & 1);
    float y[N];
#pragma unroll
    for (int t = 0; t < N; ++t) y[t] = lane_select(x[(t + k) % N], x[t], on);
#pragma unroll
    for (int t = 0; t < N; ++t) x[t] = y[t];
  }
}

__device__ __forceinline__ void lds_add_f64(uint32_t byte_addr, double v) {
  __hip_atomic_fetch_add(reinterpret_cast<MSDA_LDS double*>(static_cast<uintptr_t>(byte_addr)), v, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_WORKGROUP);
}

// One lane's CH channels of one sample: D_c = <g, v_c> for the four corners, from the staged rows
// (element offsets relative to the first staged row), summed in channel order (the same order on
// every lane, so the result does not depend on which lane a sample lands on). Two corner rows in
// flight at a time, one for 16-channel lanes (register budget).
template <typename VT, int CH>
__device__ __forceinline__ float row_dot(const VT* row, const float (&g)[CH]) {
  float u[CH];
  load_vec_lds<VT, CH>(row, u);
  float d = 0.0f;
#pragma unroll
  for (int k = 0; k < CH; ++k) d = fmaf(g[k], u[k], d);
  return d;
}

template <typename VT, int CH>
__device__ __forceinline__ void band_dots(const VT* rows, const Bilinear& c, int rel, const float (&g)[CH], float& d00, float& d10,
                                          float& d01, float& d11) {
  d00 = row_dot<VT, CH>(rows + (c.o00 - rel), g);
  d10 = row_dot<VT, CH>(rows + (c.o10 - rel), g);
  d01 = row_dot<VT, CH>(rows + (c.o01 - rel), g);
  d11 = row_dot<VT, CH>(rows + (c.o11 - rel), g);
}

// The sample's grad_value contributions of the corners in rows [r0, r1): (a * w_c) * g in f64
// (a * w_c of two f32 values is exact, 48 significant bits; its product with g, up to 72, is
// rounded to f64's 53) and added in f64, one atomic per channel.
// `gr` holds the lane's channels rotated by `rr` places (gr[t] = channel (t + rr) mod CH), so
// instruction t of the lanes of a wave adds distinct channel slots. KD: head_dim when known at
// compile time (the accumulator cell size is then an immediate offset), else 0.
// Fast path (finite weights and grad_output): a row with both weights zero is skipped; otherwise
// both of its corners are added, at cells x0 and x0 + 1 of the accumulator row (a masked corner's
// weight is exactly 0, so it adds +0.0; the accumulator has one guard cell before its first and
// after its last cell, for x0 = -1 on the first row and x0 + 1 = W on the last). Otherwise every
// corner is added at its clipped cell, as the reference's scatter-add of w * (a * g) does (a NaN
// location gives NaN weights; an infinite grad_output times a masked weight gives NaN).
template <int CH, int KD>
__device__ __forceinline__ void band_scatter(uint32_t acc, int W, int H, int D, int r0, int r1, const Bilinear& c, float a,
                                             const float (&gr)[CH], int rr, int j, bool fast) {
  const uint32_t cell = static_cast<uint32_t>(KD > 0 ? KD : D) * 8u;  // bytes per accumulator cell
  const uint32_t lane_ch = static_cast<uint32_t>(j * CH) * 8u;          // this lane's channel group
  const double ad = static_cast<double>(a);
  const double aw[4] = {ad * c.w00, ad * c.w10, ad * c.w01, ad * c.w11};
  if (fast) {
#pragma unroll
    for (int dy = 0; dy < 2; ++dy) {
      const int y = c.y0 + dy;
      const double wl = aw[2 * dy], wr = aw[2 * dy + 1];
      if (y < r0 || y >= r1 || (wl == 0.0 && wr == 0.0)) continue;
      // -1 <= x0 <= W - 1 here (an unmasked corner); the base is formed modulo 2^32
      const uint32_t base = acc + static_cast<uint32_t>((y - r0) * W + c.x0) * cell + lane_ch;
#pragma unroll
      for (int t = 0; t < CH; ++t) {
        const uint32_t o = base + static_cast<uint32_t>((t + rr) & (CH - 1)) * 8u;
        const double gt = static_cast<double>(gr[t]);
        lds_add_f64(o, wl * gt);
        lds_add_f64(o + cell, wr * gt);
      }
    }
    return;
  }
  const int ry[2] = {c.cy0, min(max(c.y0 + 1, 0), H - 1)};
  const int rx[2] = {c.cx0, min(max(c.x0 + 1, 0), W - 1)};
#pragma unroll 1
  for (int k = 0; k < 4; ++k) {
    const int y = ry[k >> 1];
    if (y < r0 || y >= r1) continue;
    const uint32_t base = acc + static_cast<uint32_t>((y - r0) * W + rx[k & 1]) * cell + lane_ch;
#pragma unroll
    for (int t = 0; t < CH; ++t)
      lds_add_f64(base + static_cast<uint32_t>((t + rr) & (CH - 1)) * 8u, aw[k] * static_cast<double>(gr[t]));
  }
}

// Per-workgroup views of the [B, Q, H, ...] tensors at (b, q = 0, h) and level l: sample (q, pt)
// of the workgroup is element q * qstride + pt, addressed with 32-bit offsets (the host bounds
// Q * H * L * P and Q * H * D).
template <typename GT>
struct BandViews {
  const float2* loc;
  const float* attn;
  float2* dloc;
  float* dattn;
  const GT* gout;    // this lane's first channel of row (b, 0, h)
  uint32_t qstride;  // H * L * P
  uint32_t gstride;  // H * D (grad_output elements between queries)
};

// Value rows in LDS (VT) and grad_output rows in global memory (GT), CH channels, channel order.
template <typename GT, int CH>
__device__ __forceinline__ void load_g(const GT* row, float (&g)[CH]) {
  load_vec<GT, CH>(row, g);
}

// A query's P points at level l: locations (P * 8 bytes) and weights (P * 4 bytes) are contiguous,
// so two or four points load as one vector each when aligned.
template <int PB>
__device__ __forceinline__ void load_points(const float2* loc, const float* attn, uint32_t si0, int p0, int P, uint32_t pmask,
                                            float2 (&xy)[PB], float (&a)[PB]) {
  if constexpr (PB == 2) {
    if (P == 2 && (si0 & 1u) == 0 && p0 == 0) {
      const float4 l4 = *reinterpret_cast<const float4*>(at(loc, si0));
      const float2 a2 = *reinterpret_cast<const float2*>(at(attn, si0));
      xy[0] = make_float2(l4.x, l4.y);
      xy[1] = make_float2(l4.z, l4.w);
      a[0] = a2.x;
      a[1] = a2.y;
      return;
    }
  } else if constexpr (PB == 4) {
    if (P == 4 && (si0 & 3u) == 0 && p0 == 0) {
      const float4 l0 = *reinterpret_cast<const float4*>(at(loc, si0));
      const float4 l1 = *reinterpret_cast<const float4*>(at(loc, si0 + 2));
      const float4 a4 = *reinterpret_cast<const float4*>(at(attn, si0));
      xy[0] = make_float2(l0.x, l0.y);
      xy[1] = make_float2(l0.z, l0.w);
      xy[2] = make_float2(l1.x, l1.y);
      xy[3] = make_float2(l1.z, l1.w);
      a[0] = a4.x;
      a[1] = a4.y;
      a[2] = a4.z;
      a[3] = a4.w;
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < PB; ++i) {
    if (p0 + i < P && ((pmask >> ((p0 + i) & 31)) & 1)) {
      xy[i] = *at(loc, si0 + p0 + i);
      a[i] = *at(attn, si0 + p0 + i);
    }
  }
}

// VT: value dtype, GT: grad_output dtype, CH: channels per lane, KD: head_dim when it is 16 or 32
// and a multiple of CH (every lane then has channels), else 0.
// Work item: (batch b, level-band item, query block, head h), batch-major. A band that is a whole
// level takes every sample of its query block directly (lanes walk the queries in order); a level
// cut into bands is scanned first, and the queries with a point in the band are listed.
template <typename VT, typename GT, int CH, int KD, bool FZ = false>
__global__ void __launch_bounds__(kBandMaxThreads) bwd_band_kernel(const BandParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const int nt = blockDim.x, tid = threadIdx.x;
  const int lid = xcd_logical(blockIdx.x, gridDim.x);
  // batch-major logical order: the workgroups of one batch entry (which share its location,
  // weight and grad_output rows) run on one XCD
  const int per_b = p.heads * p.nwork * p.nqb;
  const int b = lid / per_b;
  int rest = lid - b * per_b;
  const int item = rest / (p.heads * p.nqb);
  rest -= item * p.heads * p.nqb;
  const int qb = rest / p.heads;
  const int h = rest - qb * p.heads;
  const BandItem bi = band_item(p, item);
  const LevelDesc L = p.lv[bi.l];
  const int W = L.w, D = KD > 0 ? KD : p.dim, Q = p.queries, P = p.points, LP = p.levels * p.points;
  const int r0 = bi.r0, r1 = bi.r1, rv1 = min(r1 + 1, L.h);  // owned rows, staged rows
  const bool whole = r0 == 0 && r1 == L.h;                    // the band is the whole level
  const int q_lo = qb * p.qblock, q_hi = min(Q, q_lo + p.qblock);
  const int64_t n = static_cast<int64_t>(b) * p.heads + h;
  const int64_t slice = p.len_value * D;
  VT* vrows = reinterpret_cast<VT*>(lds_raw);
  // LDS byte address of the accumulator (an address-space cast, not the generic pointer's bits)
  const uint32_t acc = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((MSDA_LDS unsigned char*)(lds_raw + p.lds_acc)));
  double* accp = reinterpret_cast<double*>(lds_raw + p.lds_acc);
  uint32_t* list = reinterpret_cast<uint32_t*>(lds_raw + p.lds_list);
  int* cnt = reinterpret_cast<int*>(lds_raw + p.lds_cnt);
  const bool want_dv = p.dvalue != nullptr;
  const bool want_dots = p.dloc != nullptr || p.dattn != nullptr || (FZ && p.dref_part != nullptr);
  const int owned_elems = (r1 - r0) * W * D;

  // 1. staging (issued here, waited for before the barrier that precedes its use) and accumulator
  //    zeroing. A band's staging goes to the upper half of the waves, so that the lower half's scan
  //    loads (phase 2) do not queue behind the transfers (loads complete in issue order).
  if (tid == 0) cnt[0] = 0;
  if (!whole) __syncthreads();  // the counter, before any append
  const int nwaves_all = nt >> 6;
  const int stage_w0 = (!whole && nwaves_all >= 2) ? nwaves_all / 2 : 0;
  if (want_dots)
    stage_copy<VT, false>(vrows, static_cast<const VT*>(p.value) + n * slice + static_cast<int64_t>(L.start + r0 * W) * D,
                          (rv1 - r0) * W * D, p.vec16 != 0, stage_w0, nwaves_all - stage_w0);
  if (want_dv)  // the band's cells and the guard cell on each side
    for (int i = tid; i < owned_elems + 2 * D; i += nt) accp[i - D] = 0.0;

  // lane layout of the query phase
  const int lps = KD > 0 ? KD / CH : 1 << p.lps_shift;
  const int j = tid & (lps - 1);  // channel group of the lane
  const int sl = tid / lps;       // query slot
  const bool lane_on = KD > 0 || j * CH < D;
  const int c0 = lane_on ? j * CH : 0;
  const int rr = sl & (CH - 1);   // channel rotation of the lane's f64 adds
  const int rel = r0 * W * D;     // level element offset of the first staged row

  BandViews<GT> vw;
  {
    const int64_t row0 = static_cast<int64_t>(b) * Q * p.heads + h;  // row (b, 0, h)
    const int64_t s0 = row0 * LP + bi.l * P;
    vw.loc = reinterpret_cast<const float2*>(p.loc) + s0;
    vw.attn = p.attn + s0;
    vw.dloc = p.dloc ? reinterpret_cast<float2*>(p.dloc) + s0 : nullptr;
    vw.dattn = p.dattn ? p.dattn + s0 : nullptr;
    vw.gout = static_cast<const GT*>(p.gout) + row0 * D + c0;
    vw.qstride = static_cast<uint32_t>(p.heads * LP);
    vw.gstride = static_cast<uint32_t>(p.heads * D);
  }

  // One query: its grad_output row (one read) and its locations and weights at level l serve all of
  // its points in `pmask`; the band holding a point's clipped floor row writes its gradients of the
  // location and weight, every band its rows meet adds its grad_value terms.
  // Points whose inputs are loaded together (fewer for 16-channel lanes: register budget).
  constexpr int PB = CH >= 16 ? 2 : 4;
  auto load_grad = [&](uint32_t q, float (&g)[CH]) {
    if (lane_on) {
      load_g<GT, CH>(vw.gout + __umul24(q, vw.gstride), g);
    } else {
#pragma unroll
      for (int t = 0; t < CH; ++t) g[t] = 0.0f;
    }
  };
  // grad_output rotated for the grad_value adds (gr[t] = channel (t + rr) mod CH); false when a
  // channel is infinite or NaN
  auto rotate_grad = [&](const float (&g)[CH], float (&gr)[CH]) {
    float z = 0.0f;  // any infinite or NaN channel makes z NaN (inf * 0)
#pragma unroll
    for (int t = 0; t < CH; ++t) {
      gr[t] = g[t];
      z = fmaf(g[t], 0.0f, z);
    }
    rotate_regs<CH, (CH >= 16 ? 4 : CH >= 8 ? 3 : CH >= 4 ? 2 : CH >= 2 ? 1 : 0)>(gr, rr);
    return z == 0.0f;
  };
  // the points p0 + i, i < NB, of a query whose inputs are in xy and a (`every`: all NB of them are
  // points of the query and in pmask)
  // The point's weight and location gradients go to `sink(i, si, da, dl)` in lane j = 0 (the
  // default writes them; the fused epilogue keeps da and turns dl into the offset gradient).
  auto write_grads = [&](int, uint32_t si, float da, float2 dl) {
    if (vw.dattn) *at(vw.dattn, si) = da;
    if (vw.dloc) *at(vw.dloc, si) = dl;
  };
  auto do_points = [&](uint32_t si0, int p0, uint32_t pmask, const float (&g)[CH], const float (&gr)[CH], bool gfin,
                       const auto& xy, const auto& a, bool every, auto&& sink) {
    constexpr int NB = sizeof(a) / sizeof(float);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      if (!every && !(p0 + i < P && ((pmask >> ((p0 + i) & 31)) & 1))) continue;
      const uint32_t si = si0 + p0 + i;
      const Bilinear c = bilinear(xy[i].x, xy[i].y, L, D);
      if (want_dots && c.cy0 >= r0 && c.cy0 < r1) {
        float d00, d10, d01, d11;
        band_dots<VT, CH>(vrows + c0, c, rel, g, d00, d10, d01, d11);
        for (int o = 1; o < lps; o <<= 1) {
          d00 += __shfl_xor(d00, o, 64);
          d10 += __shfl_xor(d10, o, 64);
          d01 += __shfl_xor(d01, o, 64);
          d11 += __shfl_xor(d11, o, 64);
        }
        if (j == 0) {
          const float da = c.w00 * d00 + c.w10 * d10 + c.w01 * d01 + c.w11 * d11;
          const float g00 = c.m00 * d00, g10 = c.m10 * d10, g01 = c.m01 * d01, g11 = c.m11 * d11;
          const float dx = (1.0f - c.fy) * (g10 - g00) + c.fy * (g11 - g01);
          const float dy = (1.0f - c.fx) * (g01 - g00) + c.fx * (g11 - g10);
          // d ix / d loc = W (ops.py:270, :83): grid = 2 loc - 1, ix = ((grid + 1) W - 1) / 2
          sink(i, si, da, make_float2(a[i] * L.fw * dx, a[i] * L.fh * dy));
        }
      }
      if (want_dv && lane_on) {
        const bool fast = gfin && isfinite(a[i]) && isfinite(c.fx) && isfinite(c.fy);
        band_scatter<CH, KD>(acc, W, L.h, D, r0, r1, c, a[i], gr, rr, j, fast);
      }
    }
  };
  auto do_query = [&](uint32_t q, uint32_t pmask) {
    const uint32_t si0 = __umul24(q, vw.qstride);
    float g[CH], gr[CH];
    load_grad(q, g);
    const bool gfin = want_dv ? rotate_grad(g, gr) : true;
    for (int p0 = 0; p0 < P; p0 += PB) {
      float2 xy[PB];
      float a[PB];
      load_points<PB>(vw.loc, vw.attn, si0, p0, P, pmask, xy, a);
      do_points(si0, p0, pmask, g, gr, gfin, xy, a, false, write_grads);
    }
  };

  // Work is handed out a wave at a time from an LDS counter (one atomic per wave and chunk of 64 /
  // lps queries), so waves that run ahead take more and the workgroup ends within one chunk.
  const int lane = tid & 63;
  const int qpw = 64 / lps;  // queries per wave chunk
  auto grab = [&](int* counter) {
    int base = 0;
    if (lane == 0) base = atomicAdd(counter, qpw);
    return __shfl(base, 0, 64) + lane / lps;
  };
  // Software-pipelined loop over `count` work items, NP points each: item e is the points
  // [p0, p0 + NP) of query q, (q, p0) = locate(e). Waves take chunks of qpw items, the first chunk
  // by wave index, the next ones from the counter cnt[1] (which the caller sets to nwaves * qpw
  // before a barrier). A lane issues the loads of its next item before it works on the current
  // one, so the memory latency overlaps the VALU and LDS work; the loads are unconditional (the
  // item index clamped into range), so no wait depends on a branch. `first_early`: the first
  // items' inputs load before the barrier that ends the staging (whole levels, where the items are
  // known before it). NP 2 and 4 use 16-byte loads (the caller checks the alignment).
  auto pipelined = [&](auto np_tag, int count, auto locate, bool first_early) {
    constexpr int NP = decltype(np_tag)::value;
    auto load_item = [&](int e, uint32_t& si, uint32_t& qi, float (&g)[CH], float2 (&xy)[NP], float (&a)[NP], float4& rf) {
      const uint2 qp = locate(min(e, count - 1));
      load_grad(qp.x, g);
      qi = qp.x;
      si = __umul24(qp.x, vw.qstride) + qp.y;
      if constexpr (FZ) {  // the reference point of row (b, q) at the (only) level
        const int64_t i = static_cast<int64_t>(b) * Q + qp.x;
        if (p.ref_dim == 4) {
          rf = *reinterpret_cast<const float4*>(p.ref + i * 4);
        } else {
          const float2 r2 = *reinterpret_cast<const float2*>(p.ref + i * 2);
          rf = make_float4(r2.x, r2.y, 0.0f, 0.0f);
        }
      }
      if constexpr (NP == 1) {
        xy[0] = *at(vw.loc, si);
        a[0] = *at(vw.attn, si);
      } else {
#pragma unroll
        for (int k = 0; k < NP / 2; ++k) {
          const float4 l4 = *reinterpret_cast<const float4*>(at(vw.loc, si + 2 * k));
          xy[2 * k] = make_float2(l4.x, l4.y);
          xy[2 * k + 1] = make_float2(l4.z, l4.w);
        }
        if constexpr (NP == 4) {
          const float4 a4 = *reinterpret_cast<const float4*>(at(vw.attn, si));
          a[0] = a4.x;
          a[1] = a4.y;
          a[2] = a4.z;
          a[3] = a4.w;
        } else {
          const float2 a2 = *reinterpret_cast<const float2*>(at(vw.attn, si));
          a[0] = a2.x;
          a[1] = a2.y;
        }
      }
    };
    int e = (tid >> 6) * qpw + lane / lps;
    uint32_t si, qi;
    float g[CH];
    float2 xy[NP];
    float a[NP];
    float4 rf = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (first_early) {
      if (count > 0) load_item(e, si, qi, g, xy, a, rf);
      wait_vmem();  // this wave's staging transfers, before the barrier publishes them
      __syncthreads();
    }
    if (count == 0) return;
    if (!first_early) load_item(e, si, qi, g, xy, a, rf);
    while (__shfl(e, 0, 64) < count) {
      const int en = grab(&cnt[1]);
      uint32_t sin, qin;
      float gn[CH];
      float2 xyn[NP];
      float an[NP];
      float4 rfn;
      load_item(en, sin, qin, gn, xyn, an, rfn);
      if (e < count) {
        float gr[CH];
        const bool gfin = want_dv ? rotate_grad(g, gr) : true;
        if constexpr (FZ) {
          // the row's softmax weights (softmax_regs' operations) and locations (fused_location_at)
          float m = -__builtin_inff(), sum = 0.0f;
#pragma unroll
          for (int i = 0; i < NP; ++i) m = fmaxf(m, a[i]);
#pragma unroll
          for (int i = 0; i < NP; ++i) {
            a[i] = expf(a[i] - m);
            sum += a[i];
          }
#pragma unroll
          for (int i = 0; i < NP; ++i) a[i] = a[i] / sum;
          float2 tt[NP];
#pragma unroll
          for (int i = 0; i < NP; ++i) xy[i] = fused_location_at(xy[i], rf, tt[i], L.fw, L.fh, p.ref_dim, p.inv_points, p.fpoints);
          // per point, in order: keep dA, turn the location gradient into the offset gradient and
          // the reference point's share (the transpose of fused_location_at)
          float dA[NP];
          float r4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
          auto fused_sink = [&](int i, uint32_t sp, float da, float2 dl) {
            dA[i] = da;
            const float2 go = fused_offset_grad(dl, rf, tt[i], L.fw, L.fh, p.ref_dim, p.inv_points, p.fpoints, r4);
            if (vw.dloc) *at(vw.dloc, sp) = go;
          };
          do_points(si, 0, 0xffffffffu, g, gr, gfin, xy, a, true, fused_sink);
          if (j == 0 && want_dots) {
            // softmax VJP in place: grad_logit_k = a_k (dA_k - sum_j a_j dA_j)
            float S = 0.0f;
#pragma unroll
            for (int i = 0; i < NP; ++i) S += a[i] * dA[i];
            if (vw.dattn) {
#pragma unroll
              for (int i = 0; i < NP; ++i) *at(vw.dattn, si + i) = a[i] * (dA[i] - S);
            }
            if (p.dref_part != nullptr) {
              const int64_t bq = static_cast<int64_t>(b) * Q + qi;
              float* d = p.dref_part + (static_cast<int64_t>(h) * p.bq_total + bq) * p.ref_dim;
#pragma unroll
              for (int c = 0; c < 4; ++c)
                if (c < p.ref_dim) d[c] = r4[c];
            }
          }
        } else {
          do_points(si, 0, 0xffffffffu, g, gr, gfin, xy, a, true, write_grads);
        }
      }
      e = en;
      si = sin;
      qi = qin;
      rf = rfn;
#pragma unroll
      for (int t = 0; t < CH; ++t) g[t] = gn[t];
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        xy[i] = xyn[i];
        a[i] = an[i];
      }
    }
  };
  const int nwaves = nt >> 6;
  // 16-byte alignment of the query rows' locations (and weights for four points): the row offsets
  // are multiples of P, so the base pointers decide
  const bool rows16 = (reinterpret_cast<uintptr_t>(vw.loc) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(vw.attn) & (P == 4 ? 15 : 7)) == 0;
  if (!FZ && whole && p.point_items) {
    // 2'. every sample of the block belongs to this workgroup, and its queries are few for the
    //     lanes: one item per point (a query's points are consecutive items), so that every wave
    //     has items and a lane's chain of items is short
    if (tid == 0) cnt[1] = nwaves * qpw;
    auto locate = [&](int e) {
      const uint32_t qo = static_cast<uint32_t>(e) / static_cast<uint32_t>(P);
      return make_uint2(static_cast<uint32_t>(q_lo) + qo, static_cast<uint32_t>(e) - qo * static_cast<uint32_t>(P));
    };
    pipelined(std::integral_constant<int, 1>{}, (q_hi - q_lo) * P, locate, true);
  } else if (whole && rows16 && (P == 2 || (P == 4 && CH < 16))) {
    // 2'. every sample of the block belongs to this workgroup: one item per query
    if (tid == 0) cnt[1] = nwaves * qpw;
    auto locate = [&](int e) { return make_uint2(static_cast<uint32_t>(q_lo + e), 0u); };
    if (P == 2)
      pipelined(std::integral_constant<int, 2>{}, q_hi - q_lo, locate, true);
    else
      pipelined(std::integral_constant<int, 4>{}, q_hi - q_lo, locate, true);
  } else if (!FZ && whole) {
    // every sample of the block belongs to this workgroup, points per query other than 2 or 4
    // (or unaligned rows): waves take chunks of its queries from the counter
    if (tid == 0) cnt[1] = 0;
    wait_vmem();  // this wave's staging transfers, before the barrier publishes them
    __syncthreads();
    const int qcount = q_hi - q_lo;
    for (int e = grab(&cnt[1]); __shfl(e, 0, 64) < qcount; e = grab(&cnt[1]))
      if (e < qcount) do_query(static_cast<uint32_t>(q_lo + e), 0xffffffffu);
  } else if (!FZ) {
    for (int q0 = q_lo; q0 < q_hi; q0 += p.qpass) {
      const int qn = min(p.qpass, q_hi - q0);
      if (q0 > q_lo) {
        __syncthreads();  // the previous pass's list is consumed
        if (tid == 0) cnt[0] = 0;
        __syncthreads();
      }
      // 2. scan: one query per thread, its P locations at level l four at a time; every point
      //    whose clipped corner rows meet the band is listed as (query offset << 16 | point). The
      //    first pass runs on the waves that do not stage (whole waves: the appends use ballots).
      const int sth = (q0 == q_lo && stage_w0 > 0) ? stage_w0 * 64 : nt;
      for (int qq = 0; qq < qn && tid < sth; qq += sth) {
        const int qo = qq + tid;
        const bool qv = qo < qn;
        const float2* lq = at(vw.loc, __umul24(static_cast<uint32_t>(q0 + (qv ? qo : 0)), vw.qstride));
        for (int p0 = 0; p0 < P; p0 += 4) {
          float ly[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (qv && p0 + i < P) ly[i] = lq[p0 + i].y;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (p0 + i >= P) break;  // uniform
            bool in = false;
            if (qv) {
              const int2 ry = clipped_rows(ly[i], L);
              in = (ry.x >= r0 && ry.x < r1) || (ry.y >= r0 && ry.y < r1);
            }
            list_append32(in, (static_cast<uint32_t>(qo) << 16) | static_cast<uint32_t>(p0 + i), list, cnt);
          }
        }
      }
      if (tid == 0) cnt[1] = nwaves * qpw;
      wait_vmem();  // this wave's staging transfers, before the barrier publishes them
      __syncthreads();
      // 3. one item per listed point (lps lanes for wide heads), no barrier: waves drift apart, so
      //    the VALU-heavy and the LDS-atomic-heavy parts of different waves overlap
      const int nlist = cnt[0];
      auto locate = [&](int e) {
        const uint32_t ent = list[e];
        return make_uint2(static_cast<uint32_t>(q0) + (ent >> 16), ent & 0xffffu);
      };
      pipelined(std::integral_constant<int, 1>{}, nlist, locate, false);
    }
  }
  if (!want_dv) return;
  __syncthreads();
  // 4. the band's grad_value rows, rounded once to the value dtype, or this query block's partial
  //    sums (f32) when the slice's queries are split over several workgroups. With aligned rows a
  //    lane takes two consecutive accumulator elements per pass: its 16-byte LDS read sits at a
  //    16-byte lane stride (no bank conflicts; wider runs per lane conflict), and a wave stores one
  //    contiguous run.
  const int64_t row_off = n * slice + static_cast<int64_t>(L.start + r0 * W) * D;
  auto write_rows = [&](auto* dst) {
    using OT = std::remove_pointer_t<decltype(dst)>;
    if (p.vec16) {
      const int pairs = owned_elems >> 1;
      for (int i = tid; i < pairs; i += nt) {
        float f[2] = {static_cast<float>(accp[2 * i]), static_cast<float>(accp[2 * i + 1])};
        store_vec<OT, 2>(dst + 2 * i, f);
      }
      if ((owned_elems & 1) && tid == 0) {
        float f[1] = {static_cast<float>(accp[owned_elems - 1])};
        store_vec<OT, 1>(dst + owned_elems - 1, f);
      }
    } else {
      for (int i = tid; i < owned_elems; i += nt) {
        float f[1] = {static_cast<float>(accp[i])};
        store_vec<OT, 1>(dst + i, f);
      }
    }
  };
  if (p.part != nullptr)
    write_rows(p.part + static_cast<int64_t>(qb) * p.part_stride + row_off);
  else
    write_rows(static_cast<VT*>(p.dvalue) + row_off);
}

// grad_reference_points of the fused backward at one level: the per-head partials part[H][n]
// (n = B * Q * ref_dim) added in head order, for elements i0, i0 + step, ...
__device__ __forceinline__ void ref_head_sum(const float* __restrict__ part, float* __restrict__ dref, int heads, int64_t n, int64_t i0,
                                             int64_t step) {
  constexpr int U = 8;  // heads' partials in flight per thread
  for (int64_t i = i0; i < n; i += step) {
    float sum = 0.0f;
    for (int h0 = 0; h0 < heads; h0 += U) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = h0 + u < heads ? part[(h0 + u) * n + i] : 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (h0 + u < heads) sum += v[u];
    }
    dref[i] = sum;
  }
}

// grad_value = the sum of the query blocks' partial sums, in block order (deterministic), rounded
// once to the value dtype. `n` elements; block k starts at k * stride (stride: n rounded up to a
// multiple of 4, so every block's quads are 16-byte aligned). Workgroup w (in XCD-contiguous
// logical order, as the band kernel's) sums one contiguous range of quads: with the band kernel's
// batch-major order, the partials an XCD reads are mostly those its own workgroups wrote. U quads
// per thread and pass, every block's loads issued before the sums. vec: dv allows 16-byte (f32)
// or 8-byte (bf16) stores of a quad. rpart (or null): the fused backward's per-head reference-point
// partials, added into dref by the same launch (ref_head_sum).
template <typename VT>
__global__ void __launch_bounds__(256) bwd_part_sum_kernel(const float* __restrict__ part, int nqb, int64_t n, int64_t stride,
                                                           VT* __restrict__ dv, int vec, const float* rpart, float* dref, int heads,
                                                           int64_t nref) {
  if (rpart != nullptr)
    ref_head_sum(rpart, dref, heads, nref, static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x, static_cast<int64_t>(gridDim.x) * 256);
  constexpr int U = 4;
  const int64_t nq = n / 4;
  const int64_t T = 256;
  const int64_t per = (nq + gridDim.x - 1) / gridDim.x;
  const int64_t lo = static_cast<int64_t>(xcd_logical(blockIdx.x, gridDim.x)) * per;
  const int64_t hi = min(nq, lo + per);
  const float4* __restrict__ p4 = reinterpret_cast<const float4*>(part);
  const int64_t bq = stride / 4;  // quads per block
  for (int64_t q0 = lo + threadIdx.x; q0 < hi; q0 += T * U) {
    float4 s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t q = q0 + u * T;
      s[u] = p4[q < hi ? q : lo];
    }
    for (int k = 1; k < nqb; ++k) {
      float4 t[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t q = q0 + u * T;
        t[u] = p4[k * bq + (q < hi ? q : lo)];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        s[u].x += t[u].x;
        s[u].y += t[u].y;
        s[u].z += t[u].z;
        s[u].w += t[u].w;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t q = q0 + u * T;
      if (q >= hi) continue;
      const float f[4] = {s[u].x, s[u].y, s[u].z, s[u].w};
      if (vec) {
        store_vec<VT, 4>(dv + q * 4, f);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) store_vec<VT, 1>(dv + q * 4 + e, {f[e]});
      }
    }
  }
  // the last n mod 4 elements
  if (blockIdx.x == 0 && threadIdx.x < n - nq * 4) {
    const int64_t e = nq * 4 + threadIdx.x;
    float x = part[e];
    for (int k = 1; k < nqb; ++k) x += part[k * stride + e];
    store_vec<VT, 1>(dv + e, {x});
  }
}

}  // namespace msda

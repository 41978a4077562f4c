// msda_gather_kernels.h — gfx950 backward of the deformable-attention core as a sorted gather.
//
// The VJP of RF-DETR-JAX's gather sampler (src/rfdetr_jax/models/ops.py:64-134, :208-292; the
// hand-written form of the same transpose is deform_pallas.py:97-120): for every sample
// (b, q, h, l, p) with corner weights w_c (masked) at clipped cells cell_c and attention weight a,
//   grad_value[cell_c] += (a * w_c) * g        (g = grad_output[b, q, h*D:(h+1)*D])
//   D_c = <g, value[cell_c]>,  grad_attn = sum_c w_c D_c,
//   grad_loc = a * (W, H) * (d/dix, d/diy) sum_c w_c D_c   (masks and floor have zero gradient).
//
// bwd_gather_kernel: one workgroup per (batch b, level l, block of queries, head h). Every sample
// of the block gives four entries (one per corner, at its clipped cell, also when the corner is
// masked: its weight is then 0, as in the reference's scatter-add), and the workgroup computes
// the block's grad_value rows of level l without atomics on the data:
//  0. Stage the block's grad_output rows (f32) and, when they fit, the level's value rows into LDS;
//     zero one counter per cell.
//  1. One thread per sample: a rank per corner from its cell's counter (ds_add_rtn_u32) and
//     a * w_c into a slot per (sample, corner); the corner dots from the staged g row and the value
//     rows (LDS or global memory), then grad_attn and grad_loc.
//  2. Exclusive scan of the counters: the offset of each cell's entries in cell order.
//  3. Place: the entry (sample, corner) goes to position offset[cell] + rank. Thread t later reads
//     positions [t R, t R + R), so position i is stored at slot (i mod R) * threads + i / R and the
//     threads of a wave read consecutive slots.
//  4. Gather: thread t takes positions [t R, t R + R) (R = ceil(entries / threads): every thread
//     the same share, whatever the cells' counts) in one flat loop, adding (a w_c) g into D
//     registers cell by cell (g from LDS). A cell whose first position is in [t R, t R + R) belongs
//     to thread t, which writes its grad_value row (zeros for a cell without entries). A cell that
//     runs on past t R + R is completed after a barrier from the partial sums of the threads it
//     runs into, added in thread order.
// With several query blocks per (slice, level) each block writes f32 partial rows, which
// bwd_part_sum_kernel adds in block order. grad_value's sums depend on the timing of the atomics
// only through the order of the entries inside a cell (the counter ranks), which can change the
// f32 rounding of a sum in its last bits; grad_attn and grad_loc do not depend on it.
#pragma once

#include "msda_band_kernels.h"

namespace msda {

constexpr int kGatherSpt = 4;          // samples per thread held from the sort to the placement
constexpr int kGatherCellBits = 15;    // cells per level
typedef float gfloat4 __attribute__((ext_vector_type(4)));  // LDS-qualified 16-byte accesses

// Row stride (floats) of the staged grad_output rows: head_dim + 4. With a 64-byte stride (16
// banks) random rows fall on 4 bank positions and a wave's 16-byte reads conflict 16 ways; with
// 80 bytes (or 144 for head_dim 32) the rows start on 16 distinct 4-bank groups.
template <int KD>
constexpr int gather_gstride() { return KD + 4; }

struct GatherParams {
  const void* value;  // [B*H, S, D]
  const float* loc;   // [B, Q, H, L, P, 2]
  const float* attn;  // [B, Q, H, L*P]
  const void* gout;   // [B, Q, H*D]
  void* dvalue;       // [B*H, S, D] in the value dtype, or null
  float* dloc;        // as loc, or null
  float* dattn;       // as attn, or null
  float* part;        // several query blocks and grad_value requested: [nqb][B*H][S][D] f32, else null
  int64_t part_stride;  // B * H * S * D
  int heads, queries, levels, points;
  int64_t len_value;
  int nqb, qblock;    // query blocks per (slice, level) and queries per block
  int p_shift;        // log2(points) if points is a power of two, else -1
  int lds_g;          // byte offsets in LDS: grad_output rows (f32) [max(qblock, threads)][D + 4]
  int lds_wt;         // weight slots [qblock * points * 4] f32
  int lds_key;        // sorted entries [qblock * points * 4 + threads] u16
  int lds_cnt;        // cell counters, then offsets [cells + 1] i32
  int lds_scan;       // one i32 per wave
  int lds_val;        // staged value rows of the level (VT) or -1: read from global memory
  LevelDesc lv[kMaxLevels];
};

template <typename VT, int KD>
__device__ __forceinline__ void gather_store_row(const GatherParams& p, int64_t row, int qb, const float (&acc)[KD]) {
  if (p.part != nullptr) store_vec<float, KD>(p.part + static_cast<int64_t>(qb) * p.part_stride + row * KD, acc);
  else store_vec<VT, KD>(static_cast<VT*>(p.dvalue) + row * KD, acc);
}

// Phase 1's corner dots and the per-sample gradients of grad_attn and grad_loc for a thread's
// samples (kStaged: value rows in LDS, else in global memory). The dots of all samples come before
// any store, so that waiting for a sample's loads never waits for an earlier store.
// The four corner dots of one sample. Not inlined: a call per sample keeps the compiler from
// issuing the row loads of all of a thread's samples at once (4 samples x 5 rows of head_dim
// floats would not fit the registers).
template <typename VT, int KD, bool kStaged>
__device__ __attribute__((noinline)) gfloat4 sample_dots(const VT* rows, const float* grow, int o00, int o10, int o01, int o11) {
  float g[KD];
  load_vec_lds<float, KD>(grow, g);
  const int cell[4] = {o00, o10, o01, o11};
  float dd[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float v[KD];
    if constexpr (kStaged) load_vec_lds<VT, KD>(rows + cell[k] * KD, v);
    else load_vec<VT, KD>(rows + static_cast<int64_t>(cell[k]) * KD, v);
    float d = 0.0f;
#pragma unroll
    for (int t = 0; t < KD; ++t) d = fmaf(g[t], v[t], d);
    dd[k] = d;
  }
  return gfloat4{dd[0], dd[1], dd[2], dd[3]};
}

template <typename VT, int KD, bool kStaged>
__device__ __forceinline__ void gather_dots(const GatherParams& p, const LevelDesc& L, const VT* rows, const float* gq,
                                            const float2 (&xy)[kGatherSpt], const float (&av)[kGatherSpt], int tid, int nt,
                                            int ns, int q_lo, uint32_t qstride, int64_t s_base) {
  constexpr int GS = gather_gstride<KD>();
  const int P = p.points;
  float dd[kGatherSpt][4];
#pragma unroll
  for (int i = 0; i < kGatherSpt; ++i) {
    const int s = tid + i * nt < ns ? tid + i * nt : 0;
    const Bilinear c = bilinear(xy[i].x, xy[i].y, L, 1);
    const int q = p.p_shift >= 0 ? s >> p.p_shift : s / P;
    const gfloat4 d = sample_dots<VT, KD, kStaged>(rows, gq + q * GS, c.o00, c.o10, c.o01, c.o11);
    dd[i][0] = d.x;
    dd[i][1] = d.y;
    dd[i][2] = d.z;
    dd[i][3] = d.w;
  }
  float2* dloc2 = p.dloc ? reinterpret_cast<float2*>(p.dloc) + s_base : nullptr;
  float* dattn = p.dattn ? p.dattn + s_base : nullptr;
#pragma unroll
  for (int i = 0; i < kGatherSpt; ++i) {
    const int s = tid + i * nt;
    if (s < ns) {
      const Bilinear c = bilinear(xy[i].x, xy[i].y, L, 1);
      const int q = p.p_shift >= 0 ? s >> p.p_shift : s / P;
      const uint32_t si = static_cast<uint32_t>(q_lo + q) * qstride + static_cast<uint32_t>(s - q * P);
      const float d00 = dd[i][0], d10 = dd[i][1], d01 = dd[i][2], d11 = dd[i][3];
      if (dattn) *at(dattn, si) = c.w00 * d00 + c.w10 * d10 + c.w01 * d01 + c.w11 * d11;
      if (dloc2) {
        const float g00 = c.m00 * d00, g10 = c.m10 * d10, g01 = c.m01 * d01, g11 = c.m11 * d11;
        const float dx = (1.0f - c.fy) * (g10 - g00) + c.fy * (g11 - g01);
        const float dy = (1.0f - c.fx) * (g01 - g00) + c.fx * (g11 - g10);
        // d ix / d loc = W (ops.py:270, :83): grid = 2 loc - 1, ix = ((grid + 1) W - 1) / 2
        *at(dloc2, si) = make_float2(av[i] * L.fw * dx, av[i] * L.fh * dy);
      }
    }
  }
}

// VT: value dtype, GT: grad_output dtype, KD: head_dim (16 or 32), NT: maximum threads.
template <typename VT, typename GT, int KD, int NT>
__global__ void __launch_bounds__(NT) bwd_gather_kernel(const GatherParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const int nt = blockDim.x, tid = threadIdx.x;
  const int lid = xcd_logical(blockIdx.x, gridDim.x);
  // batch-major logical order: the workgroups of one batch entry run on one XCD
  const int per_b = p.levels * p.nqb * p.heads;
  const int b = lid / per_b;
  int rest = lid - b * per_b;
  const int l = rest / (p.nqb * p.heads);
  rest -= l * p.nqb * p.heads;
  const int qb = rest / p.heads;
  const int h = rest - qb * p.heads;
  const LevelDesc L = p.lv[l];
  const int C = L.h * L.w, Q = p.queries, P = p.points, LP = p.levels * P;
  const int q_lo = qb * p.qblock, nq = min(Q - q_lo, p.qblock);
  const int ns = nq * P;
  // LDS through address-space-qualified pointers (a generic pointer compiles to flat accesses)
  MSDA_LDS unsigned char* lds = (MSDA_LDS unsigned char*)(lds_raw);
  float* gq = reinterpret_cast<float*>(lds_raw + p.lds_g);  // generic: load_vec_lds casts it
  MSDA_LDS float* wt = (MSDA_LDS float*)(lds + p.lds_wt);
  MSDA_LDS uint16_t* key = (MSDA_LDS uint16_t*)(lds + p.lds_key);
  MSDA_LDS int* cnt = (MSDA_LDS int*)(lds + p.lds_cnt);
  MSDA_LDS int* scan = (MSDA_LDS int*)(lds + p.lds_scan);
  const bool want_dv = p.dvalue != nullptr;
  const bool want_dots = p.dloc != nullptr || p.dattn != nullptr;
  const int64_t n = static_cast<int64_t>(b) * p.heads + h;
  const int64_t row0 = n * p.len_value + L.start;  // grad_value row of the level's first cell
  const VT* vrows = static_cast<const VT*>(p.value) + row0 * KD;
  const VT* vlds = p.lds_val >= 0 ? reinterpret_cast<const VT*>(lds_raw + p.lds_val) : nullptr;
  constexpr int GS = gather_gstride<KD>();

  // 0. counters, grad_output rows of the block (and the level's value rows when they are staged)
  for (int i = tid; i <= C; i += nt) cnt[i] = 0;
  if (want_dots && vlds != nullptr)
    stage_copy<VT, false>(const_cast<VT*>(vlds), vrows, C * KD, (reinterpret_cast<uintptr_t>(vrows) & 15) == 0);
  {
    constexpr int C4 = KD / 4;  // 4-channel chunks per row
    const GT* g0 = static_cast<const GT*>(p.gout) + ((static_cast<int64_t>(b) * Q + q_lo) * p.heads + h) * KD;
    const uint32_t gstride = static_cast<uint32_t>(p.heads * KD);
    constexpr int U = 4;
    for (int i0 = tid; i0 < nq * C4; i0 += U * nt) {
      float v[U][4];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        // unconditional (past the end: chunk 0 again): loads under a branch are each waited for
        // where the branches join
        const int i = i0 + u * nt < nq * C4 ? i0 + u * nt : 0;
        load_vec<GT, 4>(g0 + static_cast<uint32_t>(i / C4) * gstride + (i % C4) * 4, v[u]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * nt;
        if (i < nq * C4)
          *(MSDA_LDS gfloat4*)(lds + p.lds_g + static_cast<uint32_t>((i / C4) * GS + (i % C4) * 4) * 4) =
              gfloat4{v[u][0], v[u][1], v[u][2], v[u][3]};
      }
    }
  }

  // 1. the samples' locations and weights (loaded before the barrier, unconditionally: a thread
  //    past the block's samples reloads sample 0)
  const uint32_t qstride = static_cast<uint32_t>(p.heads * LP);
  const int64_t s_base = (static_cast<int64_t>(b) * Q * p.heads + h) * LP + l * P;  // sample (q = 0, p = 0)
  const float2* loc2 = reinterpret_cast<const float2*>(p.loc) + s_base;
  const float* attn = p.attn + s_base;
  auto sample_index = [&](int s) {
    const int q = p.p_shift >= 0 ? s >> p.p_shift : s / P;
    return static_cast<uint32_t>(q_lo + q) * qstride + static_cast<uint32_t>(s - q * P);
  };
  float2 xy[kGatherSpt];
  float av[kGatherSpt];
#pragma unroll
  for (int i = 0; i < kGatherSpt; ++i) {
    const uint32_t si = sample_index(tid + i * nt < ns ? tid + i * nt : 0);
    xy[i] = *at(loc2, si);
    av[i] = *at(attn, si);
  }
  wait_vmem();  // staged rows of this wave, before the barrier publishes them
  __syncthreads();
  // ranks (u16, in the entry area until the placement) and weight slots, only when grad_value is
  // requested: the sort serves it alone
#pragma unroll
  for (int i = 0; i < kGatherSpt; ++i) {
    const int s = tid + i * nt;
    if (want_dv && s < ns) {
      const Bilinear c = bilinear(xy[i].x, xy[i].y, L, 1);  // dim 1: offsets are cell indices
      const int cell[4] = {c.o00, c.o10, c.o01, c.o11};
      const float w[4] = {c.w00, c.w10, c.w01, c.w11};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = __hip_atomic_fetch_add(cnt + cell[k], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        key[4 * s + k] = static_cast<uint16_t>(r);
        wt[4 * s + k] = av[i] * w[k];
      }
    }
  }
  // corner dots D_c = <g, value[cell_c]> in channel order (g from LDS, value rows from LDS when
  // staged, else global memory), then grad_attn and grad_loc: every load before any store
  if (want_dots) {
    if (vlds != nullptr) gather_dots<VT, KD, true>(p, L, vlds, gq, xy, av, tid, nt, ns, q_lo, qstride, s_base);
    else gather_dots<VT, KD, false>(p, L, vrows, gq, xy, av, tid, nt, ns, q_lo, qstride, s_base);
  }
  if (!want_dv) return;
  __syncthreads();

  // 2. exclusive scan of the counters (each thread a run of cells, then the waves' totals)
  {
    const int per = (C + nt - 1) / nt;
    const int c0 = min(tid * per, C), c1 = min(c0 + per, C);
    int sum = 0;
    for (int c = c0; c < c1; ++c) sum += cnt[c];
    const int lane = tid & 63, wave = tid >> 6;
    int x = sum;
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) scan[wave] = x;
    __syncthreads();
    int run = x - sum;
    for (int w = 0; w < wave; ++w) run += scan[w];
    for (int c = c0; c < c1; ++c) {
      const int v = cnt[c];
      cnt[c] = run;
      run += v;
    }
    if (tid == nt - 1) cnt[C] = run;
  }
  __syncthreads();

  // 3. place the entries (slot of position i: (i mod R) * threads + i / R): every position is read
  //    into registers before the barrier after which the entry area is overwritten
  const int E = cnt[C];
  const int R = max(1, (E + nt - 1) / nt);
  const uint32_t rmagic = R > 1 ? 0xffffffffu / static_cast<uint32_t>(R) + 1u : 0u;  // i / R = umulhi(i, magic)
  uint32_t slot[kGatherSpt][4];
#pragma unroll
  for (int i = 0; i < kGatherSpt; ++i) {
    const int s = tid + i * nt;
    if (s < ns) {
      const Bilinear c = bilinear(xy[i].x, xy[i].y, L, 1);
      const int cell[4] = {c.o00, c.o10, c.o01, c.o11};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t pos = static_cast<uint32_t>(cnt[cell[k]]) + key[4 * s + k];
        const uint32_t hi = R > 1 ? __umulhi(pos, rmagic) : pos;
        slot[i][k] = (pos - hi * R) * nt + hi;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kGatherSpt; ++i) {
    const int s = tid + i * nt;
    if (s < ns) {
#pragma unroll
      for (int k = 0; k < 4; ++k) key[slot[i][k]] = static_cast<uint16_t>(4 * s + k);
    }
  }
  __syncthreads();

  // 4. gather over positions [s0, e0)
  const int s0 = tid * R, e0 = min(s0 + R, E);
  auto lower_bound = [&](int x) {  // first c in [0, C] with cnt[c] >= x (C + 1 if none)
    int lo = 0, hi = C + 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (cnt[mid] < x) lo = mid + 1;
      else hi = mid;
    }
    return lo;
  };
  auto entry = [&](int pos, float (&acc)[KD]) {
    const uint32_t kv = key[(pos - s0) * nt + tid];
    const int s = static_cast<int>(kv >> 2);
    const int q = p.p_shift >= 0 ? s >> p.p_shift : s / P;
    float g[KD];
    load_vec_lds<float, KD>(gq + q * GS, g);
    const float w = wt[kv];
#pragma unroll
    for (int t = 0; t < KD; ++t) acc[t] = fmaf(w, g[t], acc[t]);
  };
  // One flat loop over the run's positions (the same trip count on every lane of a wave). `c` is
  // the cell of the current position and `bend` its end; the first cell is a head when it began
  // before s0 (its sum is then a partial for the cell's owner).
  float acc[KD], head[KD], span_acc[KD];
#pragma unroll
  for (int t = 0; t < KD; ++t) {
    acc[t] = 0.0f;
    head[t] = 0.0f;
    span_acc[t] = 0.0f;
  }
  bool has_head = false;
  int span_end = -1, span_cell = 0;
  if (s0 < e0) {
    int c = lower_bound(s0 + 1) - 1;  // cnt[c] <= s0 < cnt[c + 1]
    int bend = cnt[c + 1];
    bool in_head = cnt[c] < s0;
    for (int pos = s0; pos < e0; ++pos) {
      if (pos == bend) {  // cell c is complete; the next cell with entries starts at bend
        if (in_head) {
          has_head = true;
#pragma unroll
          for (int t = 0; t < KD; ++t) head[t] = acc[t];
        } else {
          gather_store_row<VT, KD>(p, row0 + c, qb, acc);
        }
#pragma unroll
        for (int t = 0; t < KD; ++t) acc[t] = 0.0f;
        in_head = false;
        do {
          ++c;
        } while (cnt[c + 1] == bend);
        bend = cnt[c + 1];
      }
      entry(pos, acc);
    }
    if (in_head) {  // the run ends inside the cell it began in, which began before s0
      has_head = true;
#pragma unroll
      for (int t = 0; t < KD; ++t) head[t] = acc[t];
    } else if (bend > e0) {  // runs on into the next threads: completed after the barrier
#pragma unroll
      for (int t = 0; t < KD; ++t) span_acc[t] = acc[t];
      span_end = bend;
      span_cell = c;
    } else {
      gather_store_row<VT, KD>(p, row0 + c, qb, acc);
    }
  }
  // cells without entries whose (empty) position range starts in this run: zero rows
  {
    const bool last = tid == nt - 1;
    float zero[KD];
#pragma unroll
    for (int t = 0; t < KD; ++t) zero[t] = 0.0f;
    for (int c = min(lower_bound(s0), C); c < C; ++c) {
      const int b0 = cnt[c];
      if (!last && b0 >= s0 + R) break;
      if (cnt[c + 1] == b0) gather_store_row<VT, KD>(p, row0 + c, qb, zero);
    }
  }
  __syncthreads();  // every gather is done: the g rows are free
  float* headp = gq;  // one partial row per thread (the g area holds max(qblock, threads) rows)
  if (has_head) {
    MSDA_LDS float* hp = (MSDA_LDS float*)(lds + p.lds_g) + tid * GS;
#pragma unroll
    for (int t = 0; t < KD; t += 4) *(MSDA_LDS gfloat4*)(hp + t) = gfloat4{head[t], head[t + 1], head[t + 2], head[t + 3]};
  }
  __syncthreads();
  if (span_end >= 0) {
    for (int j = tid + 1; j < nt && j * R < span_end; ++j) {
      float hv[KD];
      load_vec_lds<float, KD>(headp + j * GS, hv);
#pragma unroll
      for (int t = 0; t < KD; ++t) span_acc[t] += hv[t];
    }
    gather_store_row<VT, KD>(p, row0 + span_cell, qb, span_acc);
  }
}

}  // namespace msda

// msda_fused_bwd_kernels.h — the MSDeformAttn prologue around the core backward (msda_fused_bwd).
//
// msda_fused_bwd replaces the JAX autodiff VJP of MSDeformAttn.__call__ from the offsets to the
// core call (src/rfdetr_jax/models/ops.py:388-410): locations from reference points and offsets
// (:388-399, precise_divide :46-62), softmax weights (:403-404), the core (:408-410). It runs as
//  1. fused_prologue_kernel: one thread per (b, q, h) row forms the row's locations and softmax
//     weights (the same arithmetic as msda_fused_fwd's kernels: fused_location_at, softmax_stats /
//     softmax_weight) into the workspace;
//  2. the core backward (bwd_band_kernel) on them, writing grad_value, the gradient of the
//     locations (into grad_sampling_offsets, or the workspace) and of the weights (into
//     grad_attention_logits);
//  3. fused_epilogue_kernel: per row, the softmax VJP in place (grad_logit_k = a_k (dA_k -
//     sum_j a_j dA_j)), the offsets' gradient (the transpose of fused_location_at), and the
//     reference points' gradient summed over points (in order) and heads (a fixed shuffle tree).
// At one level that fits the LDS whole (2 or 4 points, head_dim 16 or 32), the band kernel's
// FZ instantiation does steps 1 and 3 itself, per (query, head) work item, and its per-head
// reference-point partials are added in head order by the part-sum kernel (with query blocks) or
// ref_head_sum_kernel.
#pragma once

#include "msda_band_kernels.h"

namespace msda {

struct FusedRowParams {
  const float* ref;     // [B, Q, L, ref_dim]
  const float* off;     // [B, Q, H, L, P, 2] sampling offsets
  const float* logits;  // [B, Q, H, L * P]
  float* loc;           // prologue: [B, Q, H, L, P, 2] locations
  float* attn;          // prologue: [B, Q, H, L * P] weights
  const float* dloc;    // epilogue: the core's gradient of the locations, or null
  float* doff;          // epilogue: grad_sampling_offsets (may be dloc itself), or null
  float* dlogits;       // epilogue: holds dA on entry, the logits' gradient on exit; or null
  float* dref;          // epilogue: [B, Q, L, ref_dim], or null
  int ref_dim, heads, levels, points;
  int64_t bq_total;     // B * Q
  float inv_points, fpoints;
  float fw[kMaxLevels], fh[kMaxLevels];
};

__device__ __forceinline__ float4 fused_row_ref(const FusedRowParams& p, int64_t bq, int l) {
  const int64_t i = bq * p.levels + l;
  if (p.ref_dim == 4) return *reinterpret_cast<const float4*>(p.ref + i * 4);
  const float2 v = *reinterpret_cast<const float2*>(p.ref + i * 2);
  return make_float4(v.x, v.y, 0.0f, 0.0f);
}

__global__ void __launch_bounds__(256) fused_prologue_kernel(const FusedRowParams p) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // (b, q, h)
  if (row >= p.bq_total * p.heads) return;
  const int LP = p.levels * p.points;
  const int64_t bq = row / p.heads;
  const float* lg = p.logits + row * LP;
  const SoftmaxStats st = softmax_stats(lg, LP);
  const float2* off = reinterpret_cast<const float2*>(p.off) + row * LP;
  float2* loc = reinterpret_cast<float2*>(p.loc) + row * LP;
  float* a = p.attn + row * LP;
  for (int l = 0; l < p.levels; ++l) {
    const float4 r = fused_row_ref(p, bq, l);
    for (int pt = 0; pt < p.points; ++pt) {
      const int k = l * p.points + pt;
      float2 t;
      loc[k] = fused_location_at(off[k], r, t, p.fw[l], p.fh[l], p.ref_dim, p.inv_points, p.fpoints);
      a[k] = softmax_weight(lg[k], st);
    }
  }
}

// 256 threads: 2^hp_shift >= heads lanes per (b, q), so a row's heads are lanes of one wave.
__global__ void __launch_bounds__(256) fused_epilogue_kernel(const FusedRowParams p, int hp_shift) {
  const int hp = 1 << hp_shift;
  const int64_t bq = static_cast<int64_t>(blockIdx.x) * (256 >> hp_shift) + (threadIdx.x >> hp_shift);
  const int h = threadIdx.x & (hp - 1);
  const bool on = bq < p.bq_total && h < p.heads;
  const int LP = p.levels * p.points;
  const int64_t row = bq * p.heads + h;
  if (on && p.dlogits != nullptr) {
    const float* lg = p.logits + row * LP;
    float* dl = p.dlogits + row * LP;
    const SoftmaxStats st = softmax_stats(lg, LP);
    float S = 0.0f;
    for (int k = 0; k < LP; ++k) S = fmaf(softmax_weight(lg[k], st), dl[k], S);  // one rounding per term, in every kernel
    for (int k = 0; k < LP; ++k) dl[k] = softmax_weight(lg[k], st) * (dl[k] - S);
  }
  if (p.dloc == nullptr) return;  // uniform: nothing below is requested
  for (int l = 0; l < p.levels; ++l) {
    float r[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (on) {
      const float4 ref = fused_row_ref(p, bq, l);
      for (int pt = 0; pt < p.points; ++pt) {
        const int64_t k = row * LP + l * p.points + pt;
        const float2 gl = reinterpret_cast<const float2*>(p.dloc)[k];
        float2 t;
        fused_location_at(reinterpret_cast<const float2*>(p.off)[k], ref, t, p.fw[l], p.fh[l], p.ref_dim, p.inv_points,
                          p.fpoints);
        const float2 go = fused_offset_grad(gl, ref, t, p.fw[l], p.fh[l], p.ref_dim, p.inv_points, p.fpoints, r);
        if (p.doff != nullptr) reinterpret_cast<float2*>(p.doff)[k] = go;
      }
    }
    if (p.dref != nullptr) {
      for (int o = 1; o < hp; o <<= 1) {
#pragma unroll
        for (int c = 0; c < 4; ++c) r[c] += __shfl_xor(r[c], o, 64);
      }
      if (on && h == 0) {
        float* d = p.dref + (bq * p.levels + l) * p.ref_dim;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (c < p.ref_dim) d[c] = r[c];
      }
    }
  }
}

// The same two steps with one thread per sample (b, q, h, k), for rows of at most NB samples over at
// most four levels (every RF-DETR shape) and fewer than 2^31 samples. Each lane loads its own
// offset, location gradient and reference point: loads and stores are contiguous runs, and there
// are LP times as many threads to hide latency as the row kernels above have. When LP is a power of
// two a row lies within one wave: each lane loads its own logit (and dA) and forms one exponential,
// and the row's statistics and sums come from the other lanes by shuffles (row_stats_lanes);
// otherwise every lane of a row loads the row's logits (one broadcast address per row) and forms
// them all. The arithmetic and its order are those of the row kernels either way.
__device__ __forceinline__ float level_pick(int l, const float (&a)[kMaxLevels]) {
  return l == 0 ? a[0] : l == 1 ? a[1] : l == 2 ? a[2] : a[3];
}

template <int NB>
__device__ __forceinline__ SoftmaxStats row_stats(const float (&x)[NB], int LP) {
  SoftmaxStats st{-__builtin_inff(), 0.0f};
#pragma unroll
  for (int u = 0; u < NB; ++u)
    if (u < LP) st.m = fmaxf(st.m, x[u]);
#pragma unroll
  for (int u = 0; u < NB; ++u)
    if (u < LP) st.s += expf(x[u] - st.m);
  return st;
}

// The softmax statistics of a row held one logit per lane (xk), its LP lanes consecutive and
// LP-aligned in the wave (LP a power of two dividing 64), for every lane of the row: the maximum by
// a butterfly (exact in any order), the sum of the lanes' exp(x - m) (ek) gathered and added in
// sample order from 0, as row_stats and softmax_stats add them, so the weights are theirs bit for
// bit with one exponential per lane instead of LP. Every lane of the wave must take part.
__device__ __forceinline__ SoftmaxStats row_stats_lanes(float xk, int LP, float& ek) {
  SoftmaxStats st{xk, 0.0f};
  for (int o = LP >> 1; o > 0; o >>= 1) st.m = fmaxf(st.m, __shfl_xor(st.m, o, LP));
  ek = expf(xk - st.m);
  for (int u = 0; u < LP; ++u) st.s += __shfl(ek, u, LP);
  return st;
}

__device__ __forceinline__ bool rows_in_lanes(int LP) { return (LP & (LP - 1)) == 0 && LP <= 64; }

template <int NB>
__global__ void __launch_bounds__(256) fused_prologue_samples_kernel(const FusedRowParams p) {
  const uint32_t LP = static_cast<uint32_t>(p.levels * p.points);
  const uint32_t total = static_cast<uint32_t>(p.bq_total * p.heads) * LP;
  uint32_t idx = blockIdx.x * 256u + threadIdx.x;  // (b, q, h, k)
  if (rows_in_lanes(static_cast<int>(LP))) {  // uniform: one exponential per lane, the row's sums by shuffles
    const bool on = idx < total;
    if (!on) idx = 0;  // whole rows only, so the lanes past the end form rows of their own
    const uint32_t row = idx / LP, k = idx - row * LP;
    const int l = static_cast<int>(k) / p.points;
    const float xk = p.logits[idx];
    float ek;
    const SoftmaxStats st = row_stats_lanes(xk, static_cast<int>(LP), ek);
    if (!on) return;
    const float2 o = reinterpret_cast<const float2*>(p.off)[idx];
    const float4 r = fused_row_ref(p, row / static_cast<uint32_t>(p.heads), l);
    float2 t;
    reinterpret_cast<float2*>(p.loc)[idx] =
        fused_location_at(o, r, t, level_pick(l, p.fw), level_pick(l, p.fh), p.ref_dim, p.inv_points, p.fpoints);
    p.attn[idx] = ek / st.s;  // softmax_weight(xk, st)
    return;
  }
  if (idx >= total) return;
  const uint32_t row = idx / LP, k = idx - row * LP;
  const int l = static_cast<int>(k) / p.points;
  const uint32_t bq = row / static_cast<uint32_t>(p.heads);
  const float* __restrict__ lg = p.logits + static_cast<size_t>(row) * LP;
  float x[NB];
#pragma unroll
  for (int u = 0; u < NB; ++u)
    if (u < static_cast<int>(LP)) x[u] = lg[u];
  const float xk = lg[k];
  const float2 o = reinterpret_cast<const float2*>(p.off)[idx];
  const float4 r = fused_row_ref(p, bq, l);
  const SoftmaxStats st = row_stats<NB>(x, LP);
  float2 t;
  reinterpret_cast<float2*>(p.loc)[idx] =
      fused_location_at(o, r, t, level_pick(l, p.fw), level_pick(l, p.fh), p.ref_dim, p.inv_points, p.fpoints);
  p.attn[idx] = softmax_weight(xk, st);
}

// 256 threads hold G whole (b, q) groups of heads x LP samples (G = 256 / (heads * LP) >= 1). The
// softmax VJP is in place on grad_attention_logits: every thread's loads precede the barrier before
// any store. The reference-point gradient goes through LDS: each sample's share, then per (group,
// level, head) the shares of the level's points in order, then per (group, level) the heads by the
// pairwise tree of the row kernel's xor shuffles over hp >= heads lanes (lane i + lane i + s at
// stride s, the missing heads zero), so the sums are the row kernel's, bit for bit.
// LDS: (G * heads * LP + G * levels * hp) float4.
template <int NB>
__global__ void __launch_bounds__(256) fused_epilogue_samples_kernel(const FusedRowParams p, int G, int hp) {
  extern __shared__ float4 cbuf[];
  const int LP = p.levels * p.points, H = p.heads, per_bq = H * LP;
  const int t = threadIdx.x;
  const int g = t / per_bq, rem = t - g * per_bq, h = rem / LP, k = rem - h * LP, l = k / p.points;
  const uint32_t bq = blockIdx.x * static_cast<uint32_t>(G) + static_cast<uint32_t>(g);
  const bool on = g < G && bq < static_cast<uint32_t>(p.bq_total);
  const uint32_t row = bq * static_cast<uint32_t>(H) + static_cast<uint32_t>(h);
  const uint32_t idx = row * static_cast<uint32_t>(LP) + static_cast<uint32_t>(k);
  const bool want_dl = p.dlogits != nullptr, want_loc = p.dloc != nullptr;  // uniform
  const bool lanes = rows_in_lanes(LP);  // uniform: each lane loads its own logit and dA only
  float x[NB], d[NB];
  float xk = 0.0f, dk = 0.0f;
  float2 gl = make_float2(0.0f, 0.0f), o = make_float2(0.0f, 0.0f);
  float4 ref = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (on) {
    if (want_dl && lanes) {
      xk = p.logits[idx];
      dk = p.dlogits[idx];
    } else if (want_dl) {
      const float* __restrict__ lg = p.logits + static_cast<size_t>(row) * LP;
      const float* __restrict__ dl = p.dlogits + static_cast<size_t>(row) * LP;
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        if (u < LP) {
          x[u] = lg[u];
          d[u] = dl[u];
        }
      }
      xk = lg[k];
      dk = dl[k];
    }
    if (want_loc) {
      gl = reinterpret_cast<const float2*>(p.dloc)[idx];
      o = reinterpret_cast<const float2*>(p.off)[idx];
      ref = fused_row_ref(p, bq, l);
    }
  }
  wait_vmem();
  __syncthreads();  // the rows' dA are read before any of them is overwritten
  if (want_dl && lanes) {  // every lane of the block takes part in the row shuffles
    float ek;
    const SoftmaxStats st = row_stats_lanes(xk, LP, ek);
    const float wk = ek / st.s;  // softmax_weight(xk, st)
    float S = 0.0f;
    for (int u = 0; u < LP; ++u) S = fmaf(__shfl(wk, u, LP), __shfl(dk, u, LP), S);  // as the row kernel, in order
    if (on) p.dlogits[idx] = wk * (dk - S);
  } else if (on && want_dl) {
    const SoftmaxStats st = row_stats<NB>(x, LP);
    float S = 0.0f;
#pragma unroll
    for (int u = 0; u < NB; ++u)
      if (u < LP) S = fmaf(softmax_weight(x[u], st), d[u], S);
    p.dlogits[idx] = softmax_weight(xk, st) * (dk - S);
  }
  if (!want_loc) return;  // uniform
  float r4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (on) {
    const float fw = level_pick(l, p.fw), fh = level_pick(l, p.fh);
    float2 tt;
    fused_location_at(o, ref, tt, fw, fh, p.ref_dim, p.inv_points, p.fpoints);
    const float2 go = fused_offset_grad(gl, ref, tt, fw, fh, p.ref_dim, p.inv_points, p.fpoints, r4);
    if (p.doff != nullptr) reinterpret_cast<float2*>(p.doff)[idx] = go;
  }
  if (p.dref == nullptr) return;  // uniform
  if (g < G) cbuf[t] = make_float4(r4[0], r4[1], r4[2], r4[3]);  // [g][h][k] = t
  __syncthreads();
  const int L = p.levels, P = p.points;
  float4* hs = cbuf + G * per_bq;  // [G][L][hp]
  for (int i = t; i < G * L * hp; i += 256) {
    const int g2 = i / (L * hp), r2 = i - g2 * (L * hp), l2 = r2 / hp, h2 = r2 - l2 * hp;
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (h2 < H) {
      const float4* c = cbuf + (g2 * H + h2) * LP + l2 * P;
      for (int pt = 0; pt < P; ++pt) {
        v.x += c[pt].x;
        v.y += c[pt].y;
        v.z += c[pt].z;
        v.w += c[pt].w;
      }
    }
    hs[i] = v;
  }
  __syncthreads();
  for (int i = t; i < G * L; i += 256) {
    const int g2 = i / L, l2 = i - g2 * L;
    const uint32_t bq2 = blockIdx.x * static_cast<uint32_t>(G) + static_cast<uint32_t>(g2);
    if (bq2 >= static_cast<uint32_t>(p.bq_total)) continue;
    float4* v = hs + i * hp;
    for (int sh = 1; sh < hp; sh <<= 1) {
      for (int j = 0; j < hp; j += 2 * sh) {
        v[j].x += v[j + sh].x;
        v[j].y += v[j + sh].y;
        v[j].z += v[j + sh].z;
        v[j].w += v[j + sh].w;
      }
    }
    float* dd = p.dref + (static_cast<size_t>(bq2) * L + l2) * p.ref_dim;
    dd[0] = v[0].x;
    dd[1] = v[0].y;
    if (p.ref_dim == 4) {
      dd[2] = v[0].z;
      dd[3] = v[0].w;
    }
  }
}

// The reference-point gradient of the band kernel's fused epilogue when no part-sum kernel runs:
// the per-head partials added in head order (ref_head_sum).
__global__ void __launch_bounds__(256) ref_head_sum_kernel(const float* part, float* dref, int heads, int64_t n) {
  ref_head_sum(part, dref, heads, n, static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x, static_cast<int64_t>(gridDim.x) * 256);
}

}  // namespace msda

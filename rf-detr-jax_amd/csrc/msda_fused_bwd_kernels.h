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
    for (int k = 0; k < LP; ++k) S += softmax_weight(lg[k], st) * dl[k];
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

// The reference-point gradient of the band kernel's fused epilogue when no part-sum kernel runs:
// the per-head partials added in head order (ref_head_sum).
__global__ void __launch_bounds__(256) ref_head_sum_kernel(const float* part, float* dref, int heads, int64_t n) {
  ref_head_sum(part, dref, heads, n, static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x, static_cast<int64_t>(gridDim.x) * 256);
}

}  // namespace msda

// attention_kernels.h — gfx950 device code for the decoder's softmax self-attention
// (scaled_dot_product_attention, src/rfdetr_jax/models/layers.py:54-99, inside MultiheadAttention,
// :491-548, with query groups folded onto the batch, src/rfdetr_jax/models/transformer.py:200-210).
//
// A slice z (= g * batch + b, the order of _split_groups, transformer.py:350-354) and head h is one
// workgroup: its L keys and values (or queries and output gradients) are staged in LDS as f32 rows
// of D + 8 floats, and each wave owns blocks of 32 queries (or keys). Tensors are read and written
// in place through element strides (batch, group, head, row; channels contiguous), so the
// decoder's [B, G * P, C] activations need no split, merge or head transposes.
//
// Products run on v_mfma_f32_32x32x2_f32 (lane l supplies A[l % 32][l / 32] and B[l / 32][l % 32];
// its 16 results are D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32]). Scores are formed transposed
// (keys x queries) so that a lane owns one query: its softmax statistics stay in the lane, and the
// probabilities in its result registers are already the B operand of the next product (the same
// reduction slot assignment is used for both operands).
//
// Softmax: scores are scaled by log2(e) / sqrt(D) and exponentiated with exp2 (one rounding
// different from exp of q.k / sqrt(D)); the forward is one pass over the key blocks with a running
// reference score m (moved, and the partial sums rescaled, only when a chunk's maximum exceeds it
// by more than kAtLazy), and stores per query m and log2 of the denominator l relative to m for
// the backward, which recomputes the probabilities as exp2((x - m) - log2 l).
// Blocked positions take the score finfo(float32).min as in the reference (:93-96), and, as
// jnp.where's VJP, pass no gradient to it: the backward sets dS = 0 there (which matters only in a
// row whose every key is blocked, where the weights are uniform). Keys past L take -inf (weight 0).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "msda_kernels.h"  // bf16_t

namespace msda {

typedef float at_f4 __attribute__((ext_vector_type(4)));
typedef float at_f16 __attribute__((ext_vector_type(16)));

enum AttnTensor { kAtQ = 0, kAtK, kAtV, kAtO, kAtGO, kAtGQ, kAtGK, kAtGV, kAtTensors };

struct AttnParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;        // backward: the forward output
  const void* go;       // backward: grad of the output
  void* out;            // forward output
  void* gq;             // backward outputs (each may be null)
  void* gk;
  void* gv;
  float* stats;         // [Z * H * L][4]: m, log2 l (forward), rowsum(dO * O) (backward), unused
  const uint8_t* mask;  // [L, L], non-zero blocks a position, or null
  int64_t st[kAtTensors][4];  // element strides (batch, group, head, row) of each tensor
  int batch, groups, heads, len;
  float scale;   // 1 / sqrt(D)
  float scale2;  // log2(e) / sqrt(D)
  // Dropout on the softmax weights (the DROP kernels): weight (q, k) of (slice, head) zh is dropped
  // when its 16-bit hash (at_drop_bits) is below drop_thr, and kept weights are scaled by drop_scale.
  uint32_t drop_seed[2];  // the call's 64-bit seed, low and high word
  uint32_t drop_thr;      // round(rate * 65536)
  float drop_scale;       // 1 / (1 - rate)
};

constexpr float kAtMaskScore = -3.4028234663852886e38f;  // finfo(float32).min

// ---- attention dropout (layers.py:537-544: flax nn.Dropout on the softmax weights) ------------
// Every kernel that touches weight (q, k) regenerates its keep decision from (seed, zh, q, k), so
// nothing is stored between the forward and the backward. The hash is pcg_hash (the PCG-RXS-M-XS
// output permutation applied to one LCG step; Jarzynski and Olano, "Hash Functions for GPU
// Rendering", JCGT 9(3), 2020). Keys 2 kh and 2 kh + 1 of query q share one 32-bit hash of
// base(zh) ^ (q << 16 | kh): the even key takes its low half, the odd key its high half, and a
// weight is kept when that half is at least drop_thr, i.e. with probability 1 - drop_thr / 65536
// (rate rounded to a multiple of 2^-16). The input is distinct for every (q, kh) while q < 2^16;
// the host bounds the length for dropout accordingly.
__device__ __forceinline__ uint32_t at_pcg(uint32_t v) {
  const uint32_t st = v * 747796405u + 2891336453u;
  const uint32_t w = ((st >> ((st >> 28u) + 4u)) ^ st) * 277803737u;
  return (w >> 22u) ^ w;
}

__device__ __forceinline__ uint32_t at_drop_base(const AttnParams& p, int zh) {
  return at_pcg(p.drop_seed[0] ^ at_pcg(p.drop_seed[1] + static_cast<uint32_t>(zh)));
}

// the shared hash of keys 2 kh and 2 kh + 1 of query q
__device__ __forceinline__ uint32_t at_drop_bits(uint32_t base, int q, int kh) {
  return at_pcg(base ^ ((static_cast<uint32_t>(q) << 16) | static_cast<uint32_t>(kh)));
}

__device__ __forceinline__ bool at_drop_keep(uint32_t base, int q, int key, uint32_t thr) {
  const uint32_t h = at_drop_bits(base, q, key >> 1);
  return ((key & 1) ? (h >> 16) : (h & 0xffffu)) >= thr;
}

// Transposed score blocks (register i: key k0 + 8 (i / 4) + 4 grp + i % 4, k0 even; the lane's
// query q): each value times `kept` if its weight is kept, else 0. Registers i and i + 1 (i even)
// hold keys 2 kh and 2 kh + 1 and share one hash.
__device__ __forceinline__ void at_drop_t(at_f16& s, uint32_t base, int q, int k0, int grp, uint32_t thr, float kept) {
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    const uint32_t h = at_drop_bits(base, q, (k0 + 8 * (i >> 2) + 4 * grp + (i & 3)) >> 1);
    s[i] = (h & 0xffffu) >= thr ? s[i] * kept : 0.0f;
    s[i + 1] = (h >> 16) >= thr ? s[i + 1] * kept : 0.0f;
  }
}

template <typename VT>
__device__ __forceinline__ at_f4 at_ld4(const VT* p, int64_t i) {  // elements i .. i + 3 as f32
  if constexpr (sizeof(VT) == 2) {
    const uint2 u = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p) + i);
    return at_f4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                 __uint_as_float(u.y & 0xffff0000u)};
  } else {
    return *reinterpret_cast<const at_f4*>(p + i);
  }
}

template <typename VT>
__device__ __forceinline__ void at_st1(VT* p, int64_t i, float v) {
  if constexpr (sizeof(VT) == 2) {
    uint32_t u = __float_as_uint(v);  // nearest even, quiet NaN
    if ((u & 0x7fffffffu) > 0x7f800000u) u = (u | 0x00400000u) & 0xffff0000u;
    else u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
    reinterpret_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(u >> 16);
  } else {
    p[i] = v;
  }
}

// 2^x by v_exp_f32 alone: results below 2^-126 flush to zero (a weight that small is below the
// f32 resolution of any row sum it enters), 2^-inf = 0.
__device__ __forceinline__ float at_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ at_f16 at_zero16() {
  at_f16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

// A (slice, head) pair zh = z * H + h, and a tensor's base offset there.
struct AttnSlice {
  int z, h, b, g;
  __device__ AttnSlice(const AttnParams& p, int zh) {
    z = zh / p.heads;
    h = zh - z * p.heads;
    g = z / p.batch;
    b = z - g * p.batch;
  }
  __device__ int64_t base(const AttnParams& p, int t) const {
    return b * p.st[t][0] + g * p.st[t][1] + h * p.st[t][2];
  }
};

// Work split: a workgroup is (slice, head, RB = 2 or 4 blocks of 32 rows on its own side: queries
// for the forward and dQ, keys for dK / dV), one block per wave (the host picks the RB that leaves
// fewest waves without a block); the other side streams through LDS in chunks of 64 rows (two
// blocks), staged from registers loaded one chunk ahead. A workgroup needs 2 x 64 rows of D + 8
// floats (20 KB at D = 32), so several share a CU and their waves fill each other's barrier and
// staging gaps.
constexpr int kAtChunk = 64;  // streamed rows per LDS chunk

template <int D>
constexpr int at_lds_floats() { return 2 * kAtChunk * (D + 8) + 3 * kAtChunk; }  // two row tiles, three per-row floats

// Element offset of row r of a tensor with row stride rs, in 32 bits by the full-rate 24-bit
// multiply (the host bounds rs < 2^24 and L * rs < 2^31).
__device__ __forceinline__ uint32_t at_row_off(int r, int64_t rs) { return __umul24(static_cast<uint32_t>(r), static_cast<uint32_t>(rs)); }

// One tensor's slice of a 64-row chunk in registers: the thread's 4-element vectors, clamped to
// row L - 1 (zeroed when stored).
template <typename VT, int D, int NT>
struct AtChunk {
  static constexpr int C4 = D / 4, NV = kAtChunk * C4 / NT;
  at_f4 v[NV];
  __device__ void load(const VT* src, int64_t rs, int r0, int L) {
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int idx = threadIdx.x + NT * u, row = idx / C4, c4 = idx - row * C4;
      v[u] = at_ld4<VT>(src, at_row_off(min(r0 + row, L - 1), rs) + 4 * c4);
    }
  }
  __device__ void store(float* dst, int r0, int L) const {
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int idx = threadIdx.x + NT * u, row = idx / C4, c4 = idx - row * C4;
      const bool ok = r0 + row < L;
      *reinterpret_cast<at_f4*>(&dst[row * (D + 8) + 4 * c4]) =
          ok ? v[u] : at_f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
};

// Transposed scores of two 32-row blocks of X (LDS rows b * 32 .., row stride D + 8) against the
// lane's column (registers xr[c] = channels 8 c + 4 (l / 32) .. + 3): two independent MFMA chains.
template <int D>
__device__ __forceinline__ void at_scores2(at_f16& s0, at_f16& s1, const float* Xs, const at_f4 (&xr)[D / 8], int col, int grp) {
  constexpr int LD = D + 8;
  s0 = at_zero16();
  s1 = at_zero16();
#pragma unroll
  for (int c = 0; c < D / 8; ++c) {
    const at_f4 a0 = *reinterpret_cast<const at_f4*>(&Xs[col * LD + 8 * c + 4 * grp]);
    const at_f4 a1 = *reinterpret_cast<const at_f4*>(&Xs[(32 + col) * LD + 8 * c + 4 * grp]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[j], xr[c][j], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[j], xr[c][j], s1, 0, 0, 0);
    }
  }
}

// Scores of one 32-row block of X against two register operands (two chains): s0 with xr, s1 with yr.
template <int D>
__device__ __forceinline__ void at_scores_pair(at_f16& s0, at_f16& s1, const float* Xs, const float* Ys, const at_f4 (&xr)[D / 8],
                                               const at_f4 (&yr)[D / 8], int col, int grp) {
  constexpr int LD = D + 8;
  s0 = at_zero16();
  s1 = at_zero16();
#pragma unroll
  for (int c = 0; c < D / 8; ++c) {
    const at_f4 a0 = *reinterpret_cast<const at_f4*>(&Xs[col * LD + 8 * c + 4 * grp]);
    const at_f4 a1 = *reinterpret_cast<const at_f4*>(&Ys[col * LD + 8 * c + 4 * grp]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[j], xr[c][j], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[j], yr[c][j], s1, 0, 0, 0);
    }
  }
}

// acc0 += X0^T w0 and acc1 += X1^T w1 (two chains): X rows from LDS (32-row blocks at X0s, X1s,
// row stride D + 8) one channel per lane, w in result-layout registers (register i is row
// 8 (i / 4) + 4 (l / 32) + i % 4 of the block); acc holds channels 32 nd + .. of the lane's column.
template <int D>
__device__ __forceinline__ void at_accum2(at_f16 (&acc0)[D / 32], at_f16 (&acc1)[D / 32], const float* X0s, const float* X1s,
                                          const at_f16& w0, const at_f16& w1, int col, int grp) {
  constexpr int LD = D + 8;
#pragma unroll
  for (int nd = 0; nd < D / 32; ++nd)
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = (8 * c4 + 4 * grp + j) * LD + 32 * nd + col;
        acc0[nd] = __builtin_amdgcn_mfma_f32_32x32x2f32(X0s[r], w0[4 * c4 + j], acc0[nd], 0, 0, 0);
        acc1[nd] = __builtin_amdgcn_mfma_f32_32x32x2f32(X1s[r], w1[4 * c4 + j], acc1[nd], 0, 0, 0);
      }
}

// at_accum2 for one block (one chain): acc += X^T w, X rows at Xs.
template <int D>
__device__ __forceinline__ void at_accum1(at_f16 (&acc)[D / 32], const float* Xs, const at_f16& w, int col, int grp) {
  constexpr int LD = D + 8;
#pragma unroll
  for (int nd = 0; nd < D / 32; ++nd)
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[nd] = __builtin_amdgcn_mfma_f32_32x32x2f32(Xs[(8 * c4 + 4 * grp + j) * LD + 32 * nd + col], w[4 * c4 + j], acc[nd], 0, 0, 0);
}

// Reductions over the two halves of a wave (lanes l and l ^ 32, which hold the same query) by
// v_permlane32_swap: both lanes get the same bits.
__device__ __forceinline__ float at_max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float at_sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Scale two transposed score blocks (keys k0 + 32 h + 8 (i / 4) + 4 grp + i % 4 of register i, the
// lane's query qi) by scale2, give keys past L the score -inf and blocked keys finfo.min (the mask
// row of qi; qi < 0: no row), and take their maximum into bm. The mask test is hoisted out of the
// per-score code, and full chunks skip the key-range test.
template <bool MASK>
__device__ __forceinline__ void at_scale_scores(at_f16& s0, at_f16& s1, int k0, int L, float scale2, const uint8_t* mask, int qi, int grp,
                                                float& bm) {
  const bool full = k0 + kAtChunk <= L;
  if (!MASK && full) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s0[i] *= scale2;
      s1[i] *= scale2;
      bm = fmaxf(bm, fmaxf(s0[i], s1[i]));
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int key0 = k0 + 8 * (i >> 2) + 4 * grp + (i & 3), key1 = key0 + 32;
    float x0 = s0[i] * scale2, x1 = s1[i] * scale2;
    if (MASK && qi >= 0) {
      const uint8_t* mr = mask + static_cast<int64_t>(qi) * L;
      if (key0 < L && mr[key0] != 0) x0 = kAtMaskScore;
      if (key1 < L && mr[key1] != 0) x1 = kAtMaskScore;
    }
    s0[i] = key0 < L ? x0 : -INFINITY;
    s1[i] = key1 < L ? x1 : -INFINITY;
    bm = fmaxf(bm, fmaxf(s0[i], s1[i]));
  }
}

// Online softmax over one chunk's two score blocks (raw dot products in s0, s1; keys
// k0 + 32 h + 8 (i / 4) + 4 grp + i % 4 of register i, the lane's query qi): turns them into
// exp2(x - m) with x = s log2(e) / sqrt(D) (blocked: finfo.min; past L: -inf), against a running
// reference score m that starts at 0 and moves only when the chunk's maximum exceeds it by more
// than kAtLazy, or, while nothing has been summed (l = 0), lies more than kAtLow below it: weights
// stay within 2^kAtLazy, which the f32 sums and bf16 operands hold as well as weights within 1, and
// no weight that matters flushes to zero. When m moves, the function returns the factor alpha =
// exp2(m_old - m_new) (0 while l = 0) that rescales l here and the caller's partial sums;
// otherwise alpha = 1.
// Without a mask, on a full chunk, each score costs one fma (x - m) before exp2, and the maximum
// is taken on those (a computed float is canonical, so the maximum needs no quieting of its
// operands).
constexpr float kAtLazy = 8.0f;
constexpr float kAtLow = 64.0f;

template <bool MASK>
__device__ __forceinline__ float at_softmax_chunk(at_f16& s0, at_f16& s1, int k0, int L, float scale2, const uint8_t* mask, int qi, int grp,
                                                  float& m, float& l) {
  float bm = -INFINITY, alpha = 1.0f;
  if (!MASK && k0 + kAtChunk <= L) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s0[i] = fmaf(s0[i], scale2, -m);
      s1[i] = fmaf(s1[i], scale2, -m);
      bm = fmaxf(bm, fmaxf(s0[i], s1[i]));
    }
    bm = at_max_halves(bm);  // relative to m; the same in both lanes of a query
    if (bm > kAtLazy || (l == 0.0f && bm < -kAtLow)) {
      alpha = l == 0.0f ? 0.0f : at_exp2(-bm);
      m += bm;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        s0[i] -= bm;
        s1[i] -= bm;
      }
    }
  } else {
    at_scale_scores<MASK>(s0, s1, k0, L, scale2, mask, qi, grp, bm);
    bm = at_max_halves(bm);  // finite: every chunk holds a key below L
    if (bm > m + kAtLazy || (l == 0.0f && bm < m - kAtLow)) {
      alpha = l == 0.0f ? 0.0f : at_exp2(m - bm);
      m = bm;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s0[i] -= m;
      s1[i] -= m;
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    s0[i] = at_exp2(s0[i]);
    s1[i] = at_exp2(s1[i]);
  }
  float rs = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) rs += s0[i] + s1[i];
  l = l * alpha + at_sum_halves(rs);
  return alpha;
}

typedef __bf16 at_bf8 __attribute__((ext_vector_type(8)));
typedef float at_f8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ at_bf8 at_bf8_of(uint2 lo, uint2 hi) { return __builtin_bit_cast(at_bf8, uint4{lo.x, lo.y, hi.x, hi.y}); }

// registers i0 .. i0 + 7 of a result block, rounded to bf16 (v_cvt_pk_bf16_f32, nearest even)
__device__ __forceinline__ at_bf8 at_bf8_regs(const at_f16& v, int i0) {
  const at_f8 f = {v[i0], v[i0 + 1], v[i0 + 2], v[i0 + 3], v[i0 + 4], v[i0 + 5], v[i0 + 6], v[i0 + 7]};
  return __builtin_convertvector(f, at_bf8);
}

// Stores a 32 x 32 result block v * scale (lane l: row r0 + l % 32, channels 8 c + 4 (l / 32) + e in
// register 4 c + e) as rows of dst (row stride rs elements), rows past L skipped, by the whole wave.
// In the result layout one store instruction writes 1 or 2 elements into each of 32 rows; through
// the wave's LDS scratch sc (at_scratch_bytes: 32 rows of 40 bf16 or 36 floats) each lane instead
// writes 16-byte row pieces (whole rows per instruction) when dst and rs are 16-byte aligned, and
// the result layout is stored element by element otherwise.
template <typename VT>
constexpr int at_scratch_bytes() { return sizeof(VT) == 2 ? 32 * 40 * 2 : 32 * 36 * 4; }  // per wave

template <typename VT>
__device__ __forceinline__ void at_store_block(VT* dst, int64_t rs, int r0, int L, const at_f16& v, float scale, void* sc, int lane) {
  const int col = lane & 31, grp = lane >> 5;
  constexpr int PER16 = 16 / sizeof(VT);  // elements per 16-byte piece
  if ((reinterpret_cast<uintptr_t>(dst) & 15) != 0 || (rs % PER16) != 0) {
    if (r0 + col < L) {
#pragma unroll
      for (int i = 0; i < 16; ++i) at_st1<VT>(dst, at_row_off(r0 + col, rs) + 8 * (i >> 2) + 4 * grp + (i & 3), v[i] * scale);
    }
    return;
  }
  if constexpr (sizeof(VT) == 2) {
    uint16_t* t = static_cast<uint16_t*>(sc);  // [32][40]
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const uint4 u = __builtin_bit_cast(uint4, at_bf8_regs(v * scale, 8 * s2));
      *reinterpret_cast<uint2*>(&t[40 * col + 16 * s2 + 4 * grp]) = uint2{u.x, u.y};
      *reinterpret_cast<uint2*>(&t[40 * col + 16 * s2 + 8 + 4 * grp]) = uint2{u.z, u.w};
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int slot = lane + 64 * k, row = slot >> 2, ch = 8 * (slot & 3);
      const uint4 x = *reinterpret_cast<const uint4*>(&t[40 * row + ch]);
      if (r0 + row < L) *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(dst) + at_row_off(r0 + row, rs) + ch) = x;
    }
  } else {
    float* t = static_cast<float*>(sc);  // [32][36]
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *reinterpret_cast<at_f4*>(&t[36 * col + 8 * c + 4 * grp]) = at_f4{v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]} * scale;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int slot = lane + 64 * k, row = slot >> 3, ch = 4 * (slot & 7);
      const at_f4 x = *reinterpret_cast<const at_f4*>(&t[36 * row + ch]);
      if (r0 + row < L) *reinterpret_cast<at_f4*>(reinterpret_cast<float*>(dst) + at_row_off(r0 + row, rs) + ch) = x;
    }
  }
}

// The workgroup's (slice, head) and row chunk: logical id (z * H + h) * chunks + rc, in
// XCD-contiguous order (xcd_logical), so the workgroups of one (slice, head), and the heads of a
// slice, which share the rows' cache lines, run on one XCD.
struct AttnWork {
  int zh, rc;
  AttnSlice sl;
  __device__ AttnWork(const AttnParams& p, int chunks) : AttnWork(p, chunks, xcd_logical(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x))) {}
  __device__ AttnWork(const AttnParams& p, int chunks, int lid) : zh(lid / chunks), rc(lid - zh * chunks), sl(p, zh) {}
};

// Forward: out = softmax(q k^T / sqrt(D), blocked -> finfo.min) v. Each wave owns 32 queries; K and
// V stream through LDS; the running maximum rescales the partial sums. DROP (host: with MASK, the
// mask may then be null): the dropped weights are zeroed before the product with V, the sum l and
// the statistics keep every weight, and the output is scaled by drop_scale / l.
template <typename VT, int D, bool MASK, int RB, bool DROP = false>
__global__ void __launch_bounds__(64 * RB, D == 32 ? (MASK ? 2 : 3) : (MASK ? 1 : 2)) attn_fwd_kernel(const AttnParams p) {
  constexpr int NT = 64 * RB;
  constexpr int LD = D + 8, ND = D / 32;
  extern __shared__ __align__(16) float at_lds[];
  float* Ks = at_lds;
  float* Vs = at_lds + kAtChunk * LD;
  const int L = p.len, nb = (L + 31) / 32, nchunks = (L + kAtChunk - 1) / kAtChunk;
  const AttnWork w(p, (nb + RB - 1) / RB);
  const VT* kp = static_cast<const VT*>(p.k) + w.sl.base(p, kAtK);
  const VT* vp = static_cast<const VT*>(p.v) + w.sl.base(p, kAtV);
  const int lane = threadIdx.x & 63, grp = lane >> 5, col = lane & 31;
  const int qb = w.rc * RB + (threadIdx.x >> 6), qi = qb * 32 + col;
  const bool qv = qi < L;
  const uint32_t dbase = DROP ? at_drop_base(p, w.zh) : 0u;
  at_f4 qr[D / 8];
  {
    const VT* qp = static_cast<const VT*>(p.q) + w.sl.base(p, kAtQ);
#pragma unroll
    for (int c = 0; c < D / 8; ++c) qr[c] = at_ld4<VT>(qp, min(qi, L - 1) * p.st[kAtQ][3] + 8 * c + 4 * grp);
  }
  float m = 0.0f, l = 0.0f;  // reference score and sum (at_softmax_chunk)
  at_f16 o0[ND], o1[ND];
#pragma unroll
  for (int nd = 0; nd < ND; ++nd) o0[nd] = o1[nd] = at_zero16();
  AtChunk<VT, D, NT> kc, vc;
  kc.load(kp, p.st[kAtK][3], 0, L);
  vc.load(vp, p.st[kAtV][3], 0, L);
  for (int j = 0; j < nchunks; ++j) {
    __syncthreads();  // every wave is done with the previous chunk
    kc.store(Ks, j * kAtChunk, L);
    vc.store(Vs, j * kAtChunk, L);
    __syncthreads();
    if (j + 1 < nchunks) {  // in flight during this chunk's arithmetic
      kc.load(kp, p.st[kAtK][3], (j + 1) * kAtChunk, L);
      vc.load(vp, p.st[kAtV][3], (j + 1) * kAtChunk, L);
    }
    if (qb >= nb) continue;
    at_f16 s0, s1;
    at_scores2<D>(s0, s1, Ks, qr, col, grp);
    const int mrow = qv && (!DROP || p.mask != nullptr) ? qi : -1;
    const float alpha = at_softmax_chunk<MASK>(s0, s1, j * kAtChunk, L, p.scale2, p.mask, mrow, grp, m, l);
    if (alpha != 1.0f) {
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
        o0[nd] *= alpha;
        o1[nd] *= alpha;
      }
    }
    if constexpr (DROP) {
      at_drop_t(s0, dbase, qi, j * kAtChunk, grp, p.drop_thr, 1.0f);
      at_drop_t(s1, dbase, qi, j * kAtChunk + 32, grp, p.drop_thr, 1.0f);
    }
    at_accum2<D>(o0, o1, Vs, Vs + 32 * LD, s0, s1, col, grp);  // O^T += V^T P^T, one chain per key block
  }
  __syncthreads();  // the chunk tiles hold the waves' output scratch from here
  if (qb < nb) {
    VT* op = static_cast<VT*>(p.out) + w.sl.base(p, kAtO);
    const float inv = (DROP ? p.drop_scale : 1.0f) / l;
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) at_store_block<VT>(op + 32 * nd, p.st[kAtO][3], qb * 32, L, o0[nd] + o1[nd], inv, at_lds + (threadIdx.x >> 6) * (at_scratch_bytes<VT>() / 4), lane);
    if (qv && grp == 0) {
      float* stats = p.stats + (static_cast<int64_t>(w.zh) * L + qi) * 4;
      stats[0] = m;
      stats[1] = log2f(l);
    }
  }
}

// Backward, query side: dQ = dS K / sqrt(D) with dS = P (dP - rowsum(dO * O)), dP = dO V^T and P
// recomputed from the stored statistics. Each wave owns 32 queries; K and V stream through LDS.
// Also stores rowsum(dO * O) of its queries in the statistics for the key-side kernel (with no
// grad_q requested, that is all it does).
template <typename VT, int D, bool MASK, int RB, bool DROP = false>
__global__ void __launch_bounds__(64 * RB, D == 32 ? ((MASK || RB == 2) ? 2 : 3) : 1) attn_bwd_q_kernel(const AttnParams p) {
  constexpr int NT = 64 * RB;
  constexpr int LD = D + 8, ND = D / 32;
  extern __shared__ __align__(16) float at_lds[];
  float* Ks = at_lds;
  float* Vs = at_lds + kAtChunk * LD;
  const int L = p.len, nb = (L + 31) / 32, nchunks = (L + kAtChunk - 1) / kAtChunk;
  const AttnWork w(p, (nb + RB - 1) / RB);
  const VT* kp = static_cast<const VT*>(p.k) + w.sl.base(p, kAtK);
  const VT* vp = static_cast<const VT*>(p.v) + w.sl.base(p, kAtV);
  const int lane = threadIdx.x & 63, grp = lane >> 5, col = lane & 31;
  const int qb = w.rc * RB + (threadIdx.x >> 6), qi = qb * 32 + col;
  const bool qv = qi < L;
  const int qc = min(qi, L - 1);
  const uint32_t dbase = DROP ? at_drop_base(p, w.zh) : 0u;
  at_f4 qr[D / 8], gr[D / 8];
  float dsum = 0.0f;  // rowsum(dO * O) over this lane's half of the channels, then both halves
  {
    const VT* qp = static_cast<const VT*>(p.q) + w.sl.base(p, kAtQ);
    const VT* gop = static_cast<const VT*>(p.go) + w.sl.base(p, kAtGO);
    const VT* opp = static_cast<const VT*>(p.o) + w.sl.base(p, kAtO);
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
      qr[c] = at_ld4<VT>(qp, qc * p.st[kAtQ][3] + 8 * c + 4 * grp);
      gr[c] = at_ld4<VT>(gop, qc * p.st[kAtGO][3] + 8 * c + 4 * grp);
      const at_f4 ov = at_ld4<VT>(opp, qc * p.st[kAtO][3] + 8 * c + 4 * grp);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) dsum += gr[c][jj] * ov[jj];
    }
  }
  dsum = at_sum_halves(dsum);
  float* stats = p.stats + (static_cast<int64_t>(w.zh) * L + qc) * 4;
  const float m = stats[0], ll = stats[1];
  if (qv && grp == 0 && qb < nb) stats[2] = dsum;  // read by the key-side kernel, launched after this one
  if (p.gq == nullptr) return;                      // only the row sums were asked for
  at_f16 dq0[ND], dq1[ND];
#pragma unroll
  for (int nd = 0; nd < ND; ++nd) dq0[nd] = dq1[nd] = at_zero16();
  AtChunk<VT, D, NT> kc, vc;
  kc.load(kp, p.st[kAtK][3], 0, L);
  vc.load(vp, p.st[kAtV][3], 0, L);
  for (int j = 0; j < nchunks; ++j) {
    __syncthreads();
    kc.store(Ks, j * kAtChunk, L);
    vc.store(Vs, j * kAtChunk, L);
    __syncthreads();
    if (j + 1 < nchunks) {
      kc.load(kp, p.st[kAtK][3], (j + 1) * kAtChunk, L);
      vc.load(vp, p.st[kAtV][3], (j + 1) * kAtChunk, L);
    }
    if (qb >= nb) continue;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {  // the chunk's two key blocks in turn (half the score registers)
      at_f16 s, dp;
      at_scores_pair<D>(s, dp, Ks + 32 * h2 * LD, Vs + 32 * h2 * LD, qr, gr, col, grp);  // S^T, dP^T = V dO^T
      // DROP: dP of the dropped weights' inputs, dP_in = dP * drop_scale where kept, else 0
      if constexpr (DROP) at_drop_t(dp, dbase, qi, j * kAtChunk + 32 * h2, grp, p.drop_thr, p.drop_scale);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = j * kAtChunk + 32 * h2 + 8 * (i >> 2) + 4 * grp + (i & 3);
        float x = s[i] * p.scale2;
        bool blocked = false;  // where(mask, finfo.min, .) passes the score no gradient
        if (key >= L) x = -INFINITY;
        else if (MASK && qv && (!DROP || p.mask != nullptr) && p.mask[static_cast<int64_t>(qi) * L + key] != 0) x = kAtMaskScore, blocked = true;
        s[i] = blocked ? 0.0f : at_exp2((x - m) - ll) * (dp[i] - dsum);  // dS^T
      }
      if (h2 == 0) at_accum1<D>(dq0, Ks, s, col, grp);  // dQ^T += K^T dS^T
      else at_accum1<D>(dq1, Ks + 32 * LD, s, col, grp);
    }
  }
  __syncthreads();  // the chunk tiles hold the waves' output scratch from here
  if (qb < nb) {
    VT* gqp = static_cast<VT*>(p.gq) + w.sl.base(p, kAtGQ);
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) at_store_block<VT>(gqp + 32 * nd, p.st[kAtGQ][3], qb * 32, L, dq0[nd] + dq1[nd], p.scale, at_lds + (threadIdx.x >> 6) * (at_scratch_bytes<VT>() / 4), lane);
  }
}

// Backward, key side: dV = P^T dO and dK = dS^T Q / sqrt(D). Each wave owns 32 keys (K and V rows
// in registers) and forms S and dP untransposed (queries x keys), so a lane owns one key; Q, dO and
// the per-query statistics (with rowsum(dO * O), written by the query-side kernel) stream through
// LDS.
template <typename VT, int D, bool MASK, int RB, bool DROP = false>
__global__ void __launch_bounds__(64 * RB, D == 32 ? (MASK ? 1 : 3) : 1) attn_bwd_kv_kernel(const AttnParams p) {
  constexpr int NT = 64 * RB;
  constexpr int LD = D + 8, ND = D / 32;
  extern __shared__ __align__(16) float at_lds[];
  float* Qs = at_lds;
  float* Gs = Qs + kAtChunk * LD;
  float* Ms = Gs + kAtChunk * LD;  // [64][2]: m, log2 l (rows past L: +inf, so their weight is 0)
  float* Ds = Ms + 2 * kAtChunk;   // [64]: rowsum(dO * O)
  const int L = p.len, nb = (L + 31) / 32, nchunks = (L + kAtChunk - 1) / kAtChunk;
  const AttnWork w(p, (nb + RB - 1) / RB);
  const VT* qp = static_cast<const VT*>(p.q) + w.sl.base(p, kAtQ);
  const VT* gop = static_cast<const VT*>(p.go) + w.sl.base(p, kAtGO);
  const float* stats = p.stats + static_cast<int64_t>(w.zh) * L * 4;
  const int t = threadIdx.x, lane = t & 63, grp = lane >> 5, col = lane & 31;
  const int kb = w.rc * RB + (t >> 6), key = kb * 32 + col;
  const uint32_t dbase = DROP ? at_drop_base(p, w.zh) : 0u;
  at_f4 kr[D / 8], vr[D / 8];
  {
    const VT* kp = static_cast<const VT*>(p.k) + w.sl.base(p, kAtK);
    const VT* vp = static_cast<const VT*>(p.v) + w.sl.base(p, kAtV);
    const int kcl = min(key, L - 1);
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
      kr[c] = at_ld4<VT>(kp, kcl * p.st[kAtK][3] + 8 * c + 4 * grp);
      vr[c] = at_ld4<VT>(vp, kcl * p.st[kAtV][3] + 8 * c + 4 * grp);
    }
  }
  at_f16 dk[ND], dv[ND];
#pragma unroll
  for (int nd = 0; nd < ND; ++nd) dk[nd] = dv[nd] = at_zero16();
  AtChunk<VT, D, NT> qc, gc;
  at_f4 sq = {0.0f, 0.0f, 0.0f, 0.0f};  // threads < 64: m, log2 l, rowsum(dO * O) of chunk row t
  auto prefetch = [&](int r0) {
    qc.load(qp, p.st[kAtQ][3], r0, L);
    gc.load(gop, p.st[kAtGO][3], r0, L);
    if (t < kAtChunk) sq = *reinterpret_cast<const at_f4*>(&stats[4 * min(r0 + t, L - 1)]);
  };
  prefetch(0);
  // per query block of a chunk: S = Q K^T and dP = dO V^T (two chains), the probabilities and dS,
  // then dV^T += dO^T P and dK^T += Q^T dS (two chains)
  auto block = [&](int r0, int h2) {
    at_f16 s, dp;
    at_scores_pair<D>(s, dp, Qs + 32 * h2 * LD, Gs + 32 * h2 * LD, kr, vr, col, grp);
    at_f16 pw;
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      const int ql = 32 * h2 + 8 * c4 + 4 * grp;  // chunk rows of registers 4 c4 .. 4 c4 + 3
      const at_f4 ms0 = *reinterpret_cast<const at_f4*>(&Ms[2 * ql]), ms1 = *reinterpret_cast<const at_f4*>(&Ms[2 * ql + 4]);
      const at_f4 dd = *reinterpret_cast<const at_f4*>(&Ds[ql]);
      const float mq[4] = {ms0[0], ms0[2], ms1[0], ms1[2]}, lq[4] = {ms0[1], ms0[3], ms1[1], ms1[3]};
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int i = 4 * c4 + jj;
        // A lane past L holds the clamped last key (its mask entry too): finite values in its own
        // result column only, which is not stored. Rows past L have m = +inf: weight 0.
        bool blocked = false;  // where(mask, finfo.min, .) passes the score no gradient: dS = 0
        if constexpr (MASK) {
          const int q = r0 + ql + jj;
          float x = s[i] * p.scale2;
          if (q < L && (!DROP || p.mask != nullptr) && p.mask[static_cast<int64_t>(q) * L + min(key, L - 1)] != 0) x = kAtMaskScore, blocked = true;
          pw[i] = at_exp2((x - mq[jj]) - lq[jj]);
        } else {
          pw[i] = at_exp2(fmaf(s[i], p.scale2, -mq[jj]) - lq[jj]);
        }
        if constexpr (DROP) {  // dS from dP * drop_scale where kept; dV from the dropped weights
          const bool keep = at_drop_keep(dbase, r0 + ql + jj, key, p.drop_thr);
          s[i] = blocked ? 0.0f : pw[i] * ((keep ? dp[i] * p.drop_scale : 0.0f) - dd[jj]);
          pw[i] = keep ? pw[i] * p.drop_scale : 0.0f;
        } else {
          s[i] = blocked ? 0.0f : pw[i] * (dp[i] - dd[jj]);  // dS
        }
      }
    }
    at_accum2<D>(dv, dk, Gs + 32 * h2 * LD, Qs + 32 * h2 * LD, pw, s, col, grp);
  };
  for (int j = 0; j < nchunks; ++j) {
    const int r0 = j * kAtChunk;
    __syncthreads();
    qc.store(Qs, r0, L);
    gc.store(Gs, r0, L);
    if (t < kAtChunk) {
      const bool in = r0 + t < L;
      Ms[2 * t] = in ? sq[0] : INFINITY;
      Ms[2 * t + 1] = in ? sq[1] : 0.0f;
      Ds[t] = in ? sq[2] : 0.0f;
    }
    __syncthreads();
    if (j + 1 < nchunks) prefetch(r0 + kAtChunk);
    if (kb >= nb) continue;
    block(r0, 0);
    block(r0, 1);
  }
  __syncthreads();  // the chunk tiles hold the waves' output scratch from here
  if (kb < nb) {
    VT* gkp = static_cast<VT*>(p.gk) + w.sl.base(p, kAtGK);
    VT* gvp = static_cast<VT*>(p.gv) + w.sl.base(p, kAtGV);
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) {
      if (p.gk != nullptr) at_store_block<VT>(gkp + 32 * nd, p.st[kAtGK][3], kb * 32, L, dk[nd], p.scale, at_lds + (threadIdx.x >> 6) * (at_scratch_bytes<VT>() / 4), lane);
      if (p.gv != nullptr) at_store_block<VT>(gvp + 32 * nd, p.st[kAtGV][3], kb * 32, L, dv[nd], 1.0f, at_lds + (threadIdx.x >> 6) * (at_scratch_bytes<VT>() / 4), lane);
    }
  }
}

// ---- bf16 inputs: products on v_mfma_f32_32x32x16_bf16 -------------------------------------
// Same work split, streaming and softmax as the f32 kernels. Operands stay bf16 in LDS, in one
// swizzled row tile [64][D] per streamed tensor: operands along the channels are one 16-byte read
// per MFMA, operands along the streamed rows two transposing reads (ds_read_b64_tr_b16) of the
// same tile, so no transposed copy is staged. v_mfma_f32_32x32x16_bf16: lane
// l supplies 8 elements of A row l % 32 and of B column l % 32 in reduction slots 8 (l / 32) + j,
// and the product pairs slot j of both operands, so any reduction-index assignment shared by A and
// B gives the sum; the result layout is that of the f32 32 x 32 products. Probabilities and dS
// are rounded to bf16 (v_cvt_pk_bf16_f32, nearest even) for the products they enter, as the
// reference rounds the softmax weights to the input dtype (layers.py:96-98); sums are f32.

// channels 16 s + 8 (l / 32) .. + 7 of one row, s < D / 16 (two 8-byte loads: rows are 8-byte aligned)
template <int D>
__device__ __forceinline__ void at_row_bf8(at_bf8 (&r)[D / 16], const uint16_t* src, int64_t off, int grp) {
#pragma unroll
  for (int s = 0; s < D / 16; ++s) {
    const uint16_t* e = src + off + 16 * s + 8 * grp;
    r[s] = at_bf8_of(*reinterpret_cast<const uint2*>(e), *reinterpret_cast<const uint2*>(e + 4));
  }
}

// Swizzled row tiles [64][D] of bf16, without padding: 16-byte chunk c of row r sits at slot
// c ^ at_sw(r), so the rows that 16 lanes read at one chunk index (row operands, one 16-byte read
// per lane) and the four consecutive rows of a transposing read (below) fall on distinct banks.
template <int D>
__device__ __forceinline__ int at_sw(int r) {
  constexpr int CPR = D / 8;  // 16-byte chunks per row
  return (r / (16 / CPR)) & (CPR - 1);
}

// element offset of channels ch .. ch + 3 of row r in a swizzled tile (ch a multiple of 4)
template <int D>
__device__ __forceinline__ int at_swo(int r, int ch) {
  return r * D + 8 * ((ch >> 3) ^ at_sw<D>(r)) + (ch & 7);
}

typedef short at_s4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: within each group of 16 lanes, lane 4a + b receives element b of the 8 bytes
// that lanes a, 4 + a, 8 + a and 12 + a address (in that order): the 16 x 4 block of 16-bit
// elements the group addresses, transposed.
__device__ __forceinline__ uint2 at_read_tr(const uint16_t* p) {
  const at_s4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) at_s4*)(p));
  return __builtin_bit_cast(uint2, r);
}

// A raw bf16 chunk (64 rows x D) in registers: 4-element vectors, rows clamped to L - 1.
template <int D, int NT>
struct AtChunkB {
  static constexpr int C4 = D / 4, NV = kAtChunk * C4 / NT;
  uint2 v[NV];
  __device__ void load(const uint16_t* src, int64_t rs, int r0, int L) {
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int idx = threadIdx.x + NT * u, row = idx / C4, c4 = idx - row * C4;
      v[u] = *reinterpret_cast<const uint2*>(src + at_row_off(min(r0 + row, L - 1), rs) + 4 * c4);
    }
  }
  __device__ void store_sw(uint16_t* dst, int r0, int L) const {  // swizzled [64][D]
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int idx = threadIdx.x + NT * u, row = idx / C4, c4 = idx - row * C4;
      *reinterpret_cast<uint2*>(&dst[at_swo<D>(row, 4 * c4)]) = r0 + row < L ? v[u] : uint2{0u, 0u};
    }
  }
};

// Result-layout scores of two 32-row blocks of swizzled row tiles against register operands (two
// chains): s0 = X[rx .. rx + 31] . xr, s1 = Y[ry .. ry + 31] . yr (the lane's row at col).
template <int D>
__device__ __forceinline__ void at_scores_sw(at_f16& s0, at_f16& s1, const uint16_t* X, int rx, const uint16_t* Y, int ry,
                                             const at_bf8 (&xr)[D / 16], const at_bf8 (&yr)[D / 16], int col, int grp) {
  s0 = at_zero16();
  s1 = at_zero16();
#pragma unroll
  for (int s = 0; s < D / 16; ++s) {
    const at_bf8 a0 = __builtin_bit_cast(at_bf8, *reinterpret_cast<const uint4*>(&X[at_swo<D>(rx + col, 16 * s + 8 * grp)]));
    const at_bf8 a1 = __builtin_bit_cast(at_bf8, *reinterpret_cast<const uint4*>(&Y[at_swo<D>(ry + col, 16 * s + 8 * grp)]));
    s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, xr[s], s0, 0, 0, 0);
    s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, yr[s], s1, 0, 0, 0);
  }
}

// acc0 += X0^T w0 and acc1 += X1^T w1 (two chains) for the 32-row blocks at rows x0 of X0 and x1 of
// X1, swizzled row tiles read by transposing reads, w in result-layout registers. Lane l's operand of MFMA (nd, s) holds
// channel 32 nd + l % 32 at rows 16 s + 8 h + 4 (l / 32) + j (slot 4 h + j), the rows of result
// register 8 s + 4 h + j of w: each of the two reads (h) has lane r of a 16-lane group g address
// row 16 s + 8 h + 4 (l / 32) + r / 4, channels 32 nd + 16 (g % 2) + 4 (r % 4) .. + 3.
template <int D>
__device__ __forceinline__ void at_accum_tr(at_f16 (&acc0)[D / 32], at_f16 (&acc1)[D / 32], const uint16_t* X0, int x0, const uint16_t* X1,
                                            int x1, const at_f16& w0, const at_f16& w1, int lane) {
  const int g = lane >> 4, r = lane & 15, grp = lane >> 5;
  at_bf8 b0[2], b1[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    b0[s] = at_bf8_regs(w0, 8 * s);
    b1[s] = at_bf8_regs(w1, 8 * s);
  }
#pragma unroll
  for (int nd = 0; nd < D / 32; ++nd)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int c = 32 * nd + 16 * (g & 1) + 4 * (r & 3), ro = 16 * s + 4 * grp + (r >> 2);
      const at_bf8 a0 = at_bf8_of(at_read_tr(X0 + at_swo<D>(x0 + ro, c)), at_read_tr(X0 + at_swo<D>(x0 + ro + 8, c)));
      const at_bf8 a1 = at_bf8_of(at_read_tr(X1 + at_swo<D>(x1 + ro, c)), at_read_tr(X1 + at_swo<D>(x1 + ro + 8, c)));
      acc0[nd] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0[s], acc0[nd], 0, 0, 0);
      acc1[nd] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1[s], acc1[nd], 0, 0, 0);
    }
}

// at_accum_tr for one block (one chain): acc += X^T w for the 32-row block at row x of X.
template <int D>
__device__ __forceinline__ void at_accum_tr1(at_f16 (&acc)[D / 32], const uint16_t* X, int x, const at_f16& w, int lane) {
  const int g = lane >> 4, r = lane & 15, grp = lane >> 5;
  at_bf8 b[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) b[s] = at_bf8_regs(w, 8 * s);
#pragma unroll
  for (int nd = 0; nd < D / 32; ++nd)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int c = 32 * nd + 16 * (g & 1) + 4 * (r & 3), ro = 16 * s + 4 * grp + (r >> 2);
      const at_bf8 a = at_bf8_of(at_read_tr(X + at_swo<D>(x + ro, c)), at_read_tr(X + at_swo<D>(x + ro + 8, c)));
      acc[nd] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b[s], acc[nd], 0, 0, 0);
    }
}

template <int D, bool MASK, int RB, bool DROP = false>
__global__ void __launch_bounds__(64 * RB, D == 32 ? 3 : 2) attn_fwd_bf16_kernel(const AttnParams p) {
  constexpr int NT = 64 * RB, ND = D / 32;
  extern __shared__ __align__(16) float at_lds[];
  uint16_t* Kr = reinterpret_cast<uint16_t*>(at_lds);  // swizzled [64][D] key and value rows
  uint16_t* Vr = Kr + kAtChunk * D;
  const int L = p.len, nb = (L + 31) / 32, nchunks = (L + kAtChunk - 1) / kAtChunk;
  const AttnWork w(p, (nb + RB - 1) / RB);
  const uint16_t* kp = static_cast<const uint16_t*>(p.k) + w.sl.base(p, kAtK);
  const uint16_t* vp = static_cast<const uint16_t*>(p.v) + w.sl.base(p, kAtV);
  const int lane = threadIdx.x & 63, grp = lane >> 5, col = lane & 31;
  const int qb = w.rc * RB + (threadIdx.x >> 6), qi = qb * 32 + col;
  const bool qv = qi < L;
  const uint32_t dbase = DROP ? at_drop_base(p, w.zh) : 0u;
  at_bf8 qr[D / 16];
  at_row_bf8<D>(qr, static_cast<const uint16_t*>(p.q) + w.sl.base(p, kAtQ), min(qi, L - 1) * p.st[kAtQ][3], grp);
  float m = 0.0f, l = 0.0f;  // reference score and sum (at_softmax_chunk)
  at_f16 o0[ND], o1[ND];
#pragma unroll
  for (int nd = 0; nd < ND; ++nd) o0[nd] = o1[nd] = at_zero16();
  AtChunkB<D, NT> kc, vc;
  kc.load(kp, p.st[kAtK][3], 0, L);
  vc.load(vp, p.st[kAtV][3], 0, L);
  for (int j = 0; j < nchunks; ++j) {
    __syncthreads();
    kc.store_sw(Kr, j * kAtChunk, L);
    vc.store_sw(Vr, j * kAtChunk, L);
    __syncthreads();
    if (j + 1 < nchunks) {
      kc.load(kp, p.st[kAtK][3], (j + 1) * kAtChunk, L);
      vc.load(vp, p.st[kAtV][3], (j + 1) * kAtChunk, L);
    }
    if (qb >= nb) continue;
    at_f16 s0, s1;
    at_scores_sw<D>(s0, s1, Kr, 0, Kr, 32, qr, qr, col, grp);  // S^T for the chunk's two key blocks
    const int mrow = qv && (!DROP || p.mask != nullptr) ? qi : -1;
    const float alpha = at_softmax_chunk<MASK>(s0, s1, j * kAtChunk, L, p.scale2, p.mask, mrow, grp, m, l);
    if (alpha != 1.0f) {
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
        o0[nd] *= alpha;
        o1[nd] *= alpha;
      }
    }
    if constexpr (DROP) {
      at_drop_t(s0, dbase, qi, j * kAtChunk, grp, p.drop_thr, 1.0f);
      at_drop_t(s1, dbase, qi, j * kAtChunk + 32, grp, p.drop_thr, 1.0f);
    }
    at_accum_tr<D>(o0, o1, Vr, 0, Vr, 32, s0, s1, lane);  // O^T += V^T P^T
  }
  __syncthreads();  // the chunk tiles hold the waves' output scratch from here
  if (qb < nb) {
    bf16_t* op = static_cast<bf16_t*>(p.out) + w.sl.base(p, kAtO);
    const float inv = (DROP ? p.drop_scale : 1.0f) / l;
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) at_store_block<bf16_t>(op + 32 * nd, p.st[kAtO][3], qb * 32, L, o0[nd] + o1[nd], inv, at_lds + (threadIdx.x >> 6) * (at_scratch_bytes<bf16_t>() / 4), lane);
    if (qv && grp == 0) {
      float* stats = p.stats + (static_cast<int64_t>(w.zh) * L + qi) * 4;
      stats[0] = m;
      stats[1] = log2f(l);
    }
  }
}

// ---- bf16, head_dim 32, no mask (the decoder's self-attention) --------------------------------
// The softmax's vector work bounds the kernel above (v_exp_f32 occupies two issue slots of a
// full-rate op, the rest one each; the matrix unit idles most of the time), so this forward moves
// what it can off the vector unit:
//  - the scores leave the MFMA already scaled and shifted: the query row is held as
//    q' = q log2(e) / sqrt(D) split into bf16 hi + lo (|q' - hi - lo| <= 2^-16 |q'|: two products
//    per operand instead of one f32 multiply), and the accumulator starts from -m (16 registers),
//    so x - m costs no vector op;
//  - the chunk maximum takes one v_max3_f32 per two scores;
//  - row sums add the bf16-rounded weights that enter the product with V (v_dot2_f32_bf16 against
//    (1, 1), one per two weights), each half-wave keeping its own sum until the end: the output is
//    sum(bf16(P) v) / sum(bf16(P)), and the statistics hold that sum;
//  - the whole key and value slice is staged in LDS once (global_load_lds_dwordx4 into swizzled
//    [Lp][32] tiles, Lp = L rounded up to 64; rows past L are copies of row L - 1 whose scores are
//    set to -inf), chunk 0 first: the later chunks land while chunk 0 is processed, and the key
//    loop has one barrier and no staging code.
// The host routes here only 16-byte aligned key and value rows with L <= kAtFwdD32MaxLen.
constexpr int kAtFwdD32MaxLen = 512;

__device__ __forceinline__ float at_max3(float a, float b, float c) { return fmaxf(fmaxf(a, b), c); }

// sum of the eight bf16 weights of w, as v_dot2_f32_bf16 against (1, 1) added to acc
__device__ __forceinline__ float at_sum_bf8(const at_bf8& w, float acc) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  const bf2 one = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(w, w, 0, 1), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(w, w, 2, 3), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(w, w, 4, 5), one, acc, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(w, w, 6, 7), one, acc, false);
}

// Stores a 32 x 32 result block v * scale (lane l: row r0 + l % 32, channels 8 c + 4 (l / 32) + e in
// register 4 c + e) as bf16 rows of dst (row stride rs elements, rows past L skipped) straight from
// the result layout: four 8-byte pieces per lane when dst and rs allow, element by element
// otherwise (the same rounding as at_store_block, without its LDS round trip and barrier).
__device__ __forceinline__ void at_store_block_direct(bf16_t* dst, int64_t rs, int r0, int L, const at_f16& v, float scale, int lane) {
  const int col = lane & 31, grp = lane >> 5;
  if (r0 + col >= L) return;
  if ((reinterpret_cast<uintptr_t>(dst) & 7) != 0 || (rs & 3) != 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) at_st1<bf16_t>(dst, at_row_off(r0 + col, rs) + 8 * (i >> 2) + 4 * grp + (i & 3), v[i] * scale);
    return;
  }
  uint16_t* row = reinterpret_cast<uint16_t*>(dst) + at_row_off(r0 + col, rs) + 4 * grp;
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    const uint4 u = __builtin_bit_cast(uint4, at_bf8_regs(v * scale, 8 * s2));
    *reinterpret_cast<uint2*>(row + 16 * s2) = uint2{u.x, u.y};
    *reinterpret_cast<uint2*>(row + 16 * s2 + 8) = uint2{u.z, u.w};
  }
}

template <int RB>
__global__ void __launch_bounds__(64 * RB, 4) attn_fwd_bf16_d32_kernel(const AttnParams p) {
  constexpr int D = 32;
  // Chunk 0's rows sit in their own static arrays: the compiler then knows that the transfers of
  // the later chunks, still in flight while chunk 0 is processed, do not write what it reads.
  __shared__ __align__(16) uint16_t K0[kAtChunk * D], V0[kAtChunk * D];
  extern __shared__ __align__(16) float at_lds[];
  const int L = p.len, nb = (L + 31) / 32, nch = (L + kAtChunk - 1) / kAtChunk, npc = nch * (kAtChunk / 16);
  uint16_t* Kr = reinterpret_cast<uint16_t*>(at_lds);  // swizzled [Lp - 64][32] key rows of chunks 1 ..
  uint16_t* Vr = Kr + (nch - 1) * kAtChunk * D;        // and value rows
  // XCD-contiguous logical order: the workgroups of one (slice, head) share an L2
  const int chunks = (nb + RB - 1) / RB, lid = xcd_logical(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int zh = lid / chunks, rc = lid - zh * chunks;
  const AttnSlice sl(p, zh);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane >> 5, col = lane & 31;
  const uint16_t* kp = static_cast<const uint16_t*>(p.k) + sl.base(p, kAtK);
  const uint16_t* vp = static_cast<const uint16_t*>(p.v) + sl.base(p, kAtV);
  // 16-row piece pc (1 KB per tensor, one global_load_lds_dwordx4 per lane and tensor) into kd, vd:
  // lane -> row 16 pc + lane / 4, LDS slot lane % 4, which holds the row's 16-byte chunk
  // (lane % 4) ^ at_sw(row)
  auto stage = [&](int pc, uint16_t* kd, uint16_t* vd) {
    const int row = pc * 16 + (lane >> 2), c = (lane & 3) ^ at_sw<D>(row), r = min(row, L - 1);
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint4*>(kp + at_row_off(r, p.st[kAtK][3]) + 8 * c), (MSDA_LDS void*)(kd), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint4*>(vp + at_row_off(r, p.st[kAtV][3]) + 8 * c), (MSDA_LDS void*)(vd), 16, 0, 0);
  };
  for (int pc = wave; pc < kAtChunk / 16; pc += RB) stage(pc, K0 + pc * 16 * D, V0 + pc * 16 * D);
  const int qb = rc * RB + wave, qi = qb * 32 + col;
  const bool active = qb < nb;
  at_bf8 qh[2], ql[2];  // q' = q log2(e) / sqrt(D) = hi + lo, channels 16 s + 8 grp .. + 7
  {
    at_bf8 qr[2];
    at_row_bf8<D>(qr, static_cast<const uint16_t*>(p.q) + sl.base(p, kAtQ), at_row_off(min(qi, L - 1), p.st[kAtQ][3]), grp);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const at_f8 f = __builtin_convertvector(qr[s], at_f8) * p.scale2;
      qh[s] = __builtin_convertvector(f, at_bf8);
      ql[s] = __builtin_convertvector(f - __builtin_convertvector(qh[s], at_f8), at_bf8);
    }
  }
  wait_vmem();  // this wave's chunk-0 transfers, before the barrier publishes them
  __syncthreads();
  for (int pc = kAtChunk / 16 + wave; pc < npc; pc += RB) stage(pc, Kr + (pc - 4) * 16 * D, Vr + (pc - 4) * 16 * D);
  float m = 0.0f, ll = 0.0f;  // reference score (at_softmax_chunk); this half-wave's sum of weights
  at_f16 negm = at_zero16(), o = at_zero16();
  const int g = lane >> 4, r = lane & 15, c = 16 * (g & 1) + 4 * (r & 3);
  // One chunk of 64 keys from swizzled tiles Kj, Vj (the swizzle repeats every 16 rows, so a
  // chunk's offsets are those of a 64-row tile).
  auto chunk = [&](const uint16_t* Kj, const uint16_t* Vj, int j) {
    const int k0 = j * kAtChunk;
    // S^T - m of the chunk's two key blocks: keys k0 + 32 h + 8 (i / 4) + 4 grp + i % 4 of register i
    at_f16 s0, s1;
    {
      at_bf8 a0[2], a1[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        a0[s] = __builtin_bit_cast(at_bf8, *reinterpret_cast<const uint4*>(&Kj[at_swo<D>(col, 16 * s + 8 * grp)]));
        a1[s] = __builtin_bit_cast(at_bf8, *reinterpret_cast<const uint4*>(&Kj[at_swo<D>(32 + col, 16 * s + 8 * grp)]));
      }
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[0], qh[0], negm, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[0], qh[0], negm, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[1], qh[1], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[1], qh[1], s1, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[0], ql[0], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[0], ql[0], s1, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[1], ql[1], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[1], ql[1], s1, 0, 0, 0);
    }
    if (k0 + kAtChunk > L) {  // the last chunk: keys past L weigh 0
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = k0 + 8 * (i >> 2) + 4 * grp + (i & 3);
        if (key >= L) s0[i] = -INFINITY;
        if (key + 32 >= L) s1[i] = -INFINITY;
      }
    }
    float bm0 = at_max3(s0[0], s0[1], s1[0]), bm1 = at_max3(s0[2], s0[3], s1[1]);
#pragma unroll
    for (int i = 2; i < 16; i += 2) {
      bm0 = at_max3(bm0, s0[i], s1[i]);
      bm1 = at_max3(bm1, s0[i + 1], s1[i + 1]);
    }
    const float bm = at_max_halves(fmaxf(bm0, bm1));  // relative to m; finite: the chunk holds a key below L
    if (bm > kAtLazy || (j == 0 && bm < -kAtLow)) {     // move m (at_softmax_chunk; at j = 0 nothing is summed yet)
      const float alpha = j == 0 ? 0.0f : at_exp2(-bm);
      m += bm;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        negm[i] = -m;
        s0[i] -= bm;
        s1[i] -= bm;
      }
      o *= alpha;
      ll *= alpha;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s0[i] = at_exp2(s0[i]);
      s1[i] = at_exp2(s1[i]);
    }
    at_bf8 b0[2], b1[2];  // result registers 8 s .. 8 s + 7 of each block, rounded (the B operands of P V)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      b0[s] = at_bf8_regs(s0, 8 * s);
      b1[s] = at_bf8_regs(s1, 8 * s);
    }
    ll = at_sum_bf8(b0[0], ll) + at_sum_bf8(b1[0], at_sum_bf8(b0[1], at_sum_bf8(b1[1], 0.0f)));
    // O^T += V^T P^T (at_accum_tr, one accumulator)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int ro = 32 * h + 16 * s + 4 * grp + (r >> 2);
        const at_bf8 a = at_bf8_of(at_read_tr(Vj + at_swo<D>(ro, c)), at_read_tr(Vj + at_swo<D>(ro + 8, c)));
        o = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, h == 0 ? b0[s] : b1[s], o, 0, 0, 0);
      }
  };
  if (active) chunk(K0, V0, 0);
  if (nch > 1) {
    wait_vmem();  // this wave's transfers of the later chunks
    __syncthreads();
  }
  for (int j = 1; active && j < nch; ++j) chunk(Kr + (j - 1) * kAtChunk * D, Vr + (j - 1) * kAtChunk * D, j);
  if (active) {
    const float l = at_sum_halves(ll);
    at_store_block_direct(static_cast<bf16_t*>(p.out) + sl.base(p, kAtO), p.st[kAtO][3], qb * 32, L, o, 1.0f / l, lane);
    if (qi < L && grp == 0) {
      float* stats = p.stats + (static_cast<int64_t>(zh) * L + qi) * 4;
      stats[0] = m;
      stats[1] = log2f(l);
    }
  }
}

template <int D, bool MASK, int RB, bool DROP = false>
__global__ void __launch_bounds__(64 * RB, D == 32 ? (MASK ? 2 : 3) : 1) attn_bwd_q_bf16_kernel(const AttnParams p) {
  constexpr int NT = 64 * RB, ND = D / 32;
  extern __shared__ __align__(16) float at_lds[];
  uint16_t* Kr = reinterpret_cast<uint16_t*>(at_lds);  // swizzled [64][D] key and value rows
  uint16_t* Vr = Kr + kAtChunk * D;
  const int L = p.len, nb = (L + 31) / 32, nchunks = (L + kAtChunk - 1) / kAtChunk;
  const AttnWork w(p, (nb + RB - 1) / RB);
  const uint16_t* kp = static_cast<const uint16_t*>(p.k) + w.sl.base(p, kAtK);
  const uint16_t* vp = static_cast<const uint16_t*>(p.v) + w.sl.base(p, kAtV);
  const int lane = threadIdx.x & 63, grp = lane >> 5, col = lane & 31;
  const int qb = w.rc * RB + (threadIdx.x >> 6), qi = qb * 32 + col;
  const bool qv = qi < L;
  const int qc = min(qi, L - 1);
  const uint32_t dbase = DROP ? at_drop_base(p, w.zh) : 0u;
  at_bf8 qr[D / 16], gr[D / 16];
  float dsum = 0.0f;
  {
    const uint16_t* qp = static_cast<const uint16_t*>(p.q) + w.sl.base(p, kAtQ);
    const uint16_t* gop = static_cast<const uint16_t*>(p.go) + w.sl.base(p, kAtGO);
    const uint16_t* opp = static_cast<const uint16_t*>(p.o) + w.sl.base(p, kAtO);
    at_row_bf8<D>(qr, qp, qc * p.st[kAtQ][3], grp);
    at_row_bf8<D>(gr, gop, qc * p.st[kAtGO][3], grp);
#pragma unroll
    for (int s = 0; s < D / 16; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t off = 16 * s + 8 * grp + 4 * h;
        const at_f4 g = at_ld4<bf16_t>(reinterpret_cast<const bf16_t*>(gop), qc * p.st[kAtGO][3] + off);
        const at_f4 o = at_ld4<bf16_t>(reinterpret_cast<const bf16_t*>(opp), qc * p.st[kAtO][3] + off);
        dsum += g[0] * o[0] + g[1] * o[1] + g[2] * o[2] + g[3] * o[3];
      }
  }
  dsum = at_sum_halves(dsum);
  float* stats = p.stats + (static_cast<int64_t>(w.zh) * L + qc) * 4;
  const float m = stats[0], ll = stats[1];
  if (qv && grp == 0 && qb < nb) stats[2] = dsum;
  if (p.gq == nullptr) return;
  at_f16 dq0[ND], dq1[ND];
#pragma unroll
  for (int nd = 0; nd < ND; ++nd) dq0[nd] = dq1[nd] = at_zero16();
  AtChunkB<D, NT> kc, vc;
  kc.load(kp, p.st[kAtK][3], 0, L);
  vc.load(vp, p.st[kAtV][3], 0, L);
  for (int j = 0; j < nchunks; ++j) {
    __syncthreads();
    kc.store_sw(Kr, j * kAtChunk, L);
    vc.store_sw(Vr, j * kAtChunk, L);
    __syncthreads();
    if (j + 1 < nchunks) {
      kc.load(kp, p.st[kAtK][3], (j + 1) * kAtChunk, L);
      vc.load(vp, p.st[kAtV][3], (j + 1) * kAtChunk, L);
    }
    if (qb >= nb) continue;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {  // the chunk's two key blocks in turn (half the score registers)
      at_f16 s, dp;
      at_scores_sw<D>(s, dp, Kr, 32 * h2, Vr, 32 * h2, qr, gr, col, grp);  // S^T and dP^T = V dO^T
      if constexpr (DROP) at_drop_t(dp, dbase, qi, j * kAtChunk + 32 * h2, grp, p.drop_thr, p.drop_scale);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = j * kAtChunk + 32 * h2 + 8 * (i >> 2) + 4 * grp + (i & 3);
        float x = s[i] * p.scale2;
        bool blocked = false;  // where(mask, finfo.min, .) passes the score no gradient
        if (key >= L) x = -INFINITY;
        else if (MASK && qv && (!DROP || p.mask != nullptr) && p.mask[static_cast<int64_t>(qi) * L + key] != 0) x = kAtMaskScore, blocked = true;
        s[i] = blocked ? 0.0f : at_exp2((x - m) - ll) * (dp[i] - dsum);  // dS^T
      }
      if (h2 == 0) at_accum_tr1<D>(dq0, Kr, 0, s, lane);  // dQ^T += K^T dS^T
      else at_accum_tr1<D>(dq1, Kr, 32, s, lane);
    }
  }
  __syncthreads();  // the chunk tiles hold the waves' output scratch from here
  if (qb < nb) {
    bf16_t* gqp = static_cast<bf16_t*>(p.gq) + w.sl.base(p, kAtGQ);
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) at_store_block<bf16_t>(gqp + 32 * nd, p.st[kAtGQ][3], qb * 32, L, dq0[nd] + dq1[nd], p.scale, at_lds + (threadIdx.x >> 6) * (at_scratch_bytes<bf16_t>() / 4), lane);
  }
}

template <int D, bool MASK, int RB, bool DROP = false>
__global__ void __launch_bounds__(64 * RB, D == 32 ? (MASK ? 2 : 3) : 1) attn_bwd_kv_bf16_kernel(const AttnParams p) {
  constexpr int NT = 64 * RB, ND = D / 32;
  extern __shared__ __align__(16) float at_lds[];
  uint16_t* Qr = reinterpret_cast<uint16_t*>(at_lds);  // swizzled [64][D] query and output-gradient rows
  uint16_t* Gr = Qr + kAtChunk * D;
  float* Ms = reinterpret_cast<float*>(Gr + kAtChunk * D);  // [64][2]: m, log2 l (rows past L: +inf)
  float* Ds = Ms + 2 * kAtChunk;                          // [64]: rowsum(dO * O)
  const int L = p.len, nb = (L + 31) / 32, nchunks = (L + kAtChunk - 1) / kAtChunk;
  const AttnWork w(p, (nb + RB - 1) / RB);
  const uint16_t* qp = static_cast<const uint16_t*>(p.q) + w.sl.base(p, kAtQ);
  const uint16_t* gop = static_cast<const uint16_t*>(p.go) + w.sl.base(p, kAtGO);
  const float* stats = p.stats + static_cast<int64_t>(w.zh) * L * 4;
  const int t = threadIdx.x, lane = t & 63, grp = lane >> 5, col = lane & 31;
  const int kb = w.rc * RB + (t >> 6), key = kb * 32 + col;
  const uint32_t dbase = DROP ? at_drop_base(p, w.zh) : 0u;
  at_bf8 kr[D / 16], vr[D / 16];
  at_row_bf8<D>(kr, static_cast<const uint16_t*>(p.k) + w.sl.base(p, kAtK), min(key, L - 1) * p.st[kAtK][3], grp);
  at_row_bf8<D>(vr, static_cast<const uint16_t*>(p.v) + w.sl.base(p, kAtV), min(key, L - 1) * p.st[kAtV][3], grp);
  at_f16 dk[ND], dv[ND];
#pragma unroll
  for (int nd = 0; nd < ND; ++nd) dk[nd] = dv[nd] = at_zero16();
  AtChunkB<D, NT> qc, gc;
  at_f4 sq = {0.0f, 0.0f, 0.0f, 0.0f};
  auto prefetch = [&](int r0) {
    qc.load(qp, p.st[kAtQ][3], r0, L);
    gc.load(gop, p.st[kAtGO][3], r0, L);
    if (t < kAtChunk) sq = *reinterpret_cast<const at_f4*>(&stats[4 * min(r0 + t, L - 1)]);
  };
  prefetch(0);
  for (int j = 0; j < nchunks; ++j) {
    const int r0 = j * kAtChunk;
    __syncthreads();
    qc.store_sw(Qr, r0, L);
    gc.store_sw(Gr, r0, L);
    if (t < kAtChunk) {
      const bool in = r0 + t < L;
      Ms[2 * t] = in ? sq[0] : INFINITY;
      Ms[2 * t + 1] = in ? sq[1] : 0.0f;
      Ds[t] = in ? sq[2] : 0.0f;
    }
    __syncthreads();
    if (j + 1 < nchunks) prefetch(r0 + kAtChunk);
    if (kb >= nb) continue;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {  // the chunk's two query blocks
      at_f16 s, dp;
      at_scores_sw<D>(s, dp, Qr, 32 * h2, Gr, 32 * h2, kr, vr, col, grp);  // S = Q K^T, dP = dO V^T
      at_f16 pw;
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {
        const int ql = 32 * h2 + 8 * c4 + 4 * grp;
        const at_f4 ms0 = *reinterpret_cast<const at_f4*>(&Ms[2 * ql]), ms1 = *reinterpret_cast<const at_f4*>(&Ms[2 * ql + 4]);
        const at_f4 dd = *reinterpret_cast<const at_f4*>(&Ds[ql]);
        const float mq[4] = {ms0[0], ms0[2], ms1[0], ms1[2]}, lq[4] = {ms0[1], ms0[3], ms1[1], ms1[3]};
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int i = 4 * c4 + jj;
          // lanes past L and rows past L as in the f32 kernel
          bool blocked = false;  // as in the f32 kernel
          if constexpr (MASK) {
            const int q = r0 + ql + jj;
            float x = s[i] * p.scale2;
            if (q < L && (!DROP || p.mask != nullptr) && p.mask[static_cast<int64_t>(q) * L + min(key, L - 1)] != 0) x = kAtMaskScore, blocked = true;
            pw[i] = at_exp2((x - mq[jj]) - lq[jj]);
          } else {
            pw[i] = at_exp2(fmaf(s[i], p.scale2, -mq[jj]) - lq[jj]);
          }
          if constexpr (DROP) {  // as in the f32 kernel
            const bool keep = at_drop_keep(dbase, r0 + ql + jj, key, p.drop_thr);
            s[i] = blocked ? 0.0f : pw[i] * ((keep ? dp[i] * p.drop_scale : 0.0f) - dd[jj]);
            pw[i] = keep ? pw[i] * p.drop_scale : 0.0f;
          } else {
            s[i] = blocked ? 0.0f : pw[i] * (dp[i] - dd[jj]);  // dS
          }
        }
      }
      at_accum_tr<D>(dv, dk, Gr, 32 * h2, Qr, 32 * h2, pw, s, lane);  // dV^T += dO^T P, dK^T += Q^T dS
    }
  }
  __syncthreads();  // the chunk tiles hold the waves' output scratch from here
  if (kb < nb) {
    bf16_t* gkp = static_cast<bf16_t*>(p.gk) + w.sl.base(p, kAtGK);
    bf16_t* gvp = static_cast<bf16_t*>(p.gv) + w.sl.base(p, kAtGV);
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) {
      if (p.gk != nullptr) at_store_block<bf16_t>(gkp + 32 * nd, p.st[kAtGK][3], kb * 32, L, dk[nd], p.scale, at_lds + (threadIdx.x >> 6) * (at_scratch_bytes<bf16_t>() / 4), lane);
      if (p.gv != nullptr) at_store_block<bf16_t>(gvp + 32 * nd, p.st[kAtGV][3], kb * 32, L, dv[nd], 1.0f, at_lds + (threadIdx.x >> 6) * (at_scratch_bytes<bf16_t>() / 4), lane);
    }
  }
}


// Fused backward (bf16, D = 32, L <= 32 kAtFusedBlocks, no mask: a masked kernel would not fit three
// waves per SIMD without spilling): a workgroup is one (slice, head). Waves 0 .. nb - 1 own one key
// block each and form S, dP, P and dS of each (query block, key block) pair once: they accumulate
// the block's dK and dV (as attn_bwd_kv_bf16_kernel) and write dS into LDS tiles [32 keys][32
// queries]. Waves nb and nb + 1 stage the query-side rows (Q, dO, and rowsum(dO * O) from O) one
// chunk ahead and form dQ of the previous chunk's two query blocks, one block each, over the first
// key blocks, dQ^T = K^T dS^T, from a swizzled copy of K and the dS tiles by transposing reads;
// key waves 0 .. 3 form the rest in two parts into LDS, which the dQ waves add one chunk later
// before storing the block. The row tiles, dS tiles and parts are double buffered by chunk parity:
// one barrier per chunk.
constexpr int kAtFusedBlocks = 10;  // key-block waves; with the two dQ waves, 768 threads (three waves per SIMD)

// Dynamic LDS bytes of the fused kernel for nb key blocks: the swizzled key rows [32 nb][32] and
// two sets of dS tiles [nb][2][32][32] (bf16). The query-side row tiles and per-row m, log2 l and
// rowsum are static arrays, so the compiler knows that the dS stores leave them alone.
constexpr int at_fused_lds_bytes(int nb) { return nb * (2048 + 2 * 4096); }

__device__ __forceinline__ float at_bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float at_bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

__global__ void __launch_bounds__(64 * (kAtFusedBlocks + 2), 3) attn_bwd_fused_bf16_kernel(const AttnParams p) {
  constexpr int D = 32;
  __shared__ __align__(16) uint16_t Qr[2][kAtChunk * D];  // swizzled [64][D] query and output-gradient rows
  __shared__ __align__(16) uint16_t Gr[2][kAtChunk * D];
  __shared__ __align__(16) float Ms[2][kAtChunk];  // [64]: -(m + log2 l) (rows past L: -inf)
  __shared__ __align__(16) float Ds[2][kAtChunk];  // [64]: -rowsum(dO * O)
  __shared__ __align__(16) float Xq[2][2][2][16 * 64];   // by parity, part and query block: the helpers' partial dQ^T
  extern __shared__ __align__(16) float at_lds[];
  const int L = p.len, nb = (L + 31) / 32, nchunks = (L + kAtChunk - 1) / kAtChunk;
  uint16_t* Kt = reinterpret_cast<uint16_t*>(at_lds);  // swizzled [32 nb][D] key rows (0 past L)
  uint16_t* St = Kt + 32 * nb * D;                      // dS tiles: 1024 elements each, set, block, query block
  // XCD-contiguous logical order: the heads of a slice, which share the rows' cache lines, run on one XCD
  const int zh = xcd_logical(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const AttnSlice sl(p, zh);
  const uint16_t* kp = static_cast<const uint16_t*>(p.k) + sl.base(p, kAtK);
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, grp = lane >> 5, col = lane & 31;
  // dQ^T of a query block sums over the key blocks: [0, n0) by the dQ wave of that block, [n0, n1)
  // by key wave 0 or 1 (part 0) and [n1, nb) by key wave 2 or 3 (part 1), whose partial sums pass
  // through LDS; the dQ waves also stage the rows, so they take the smallest share (2 of 10 key
  // blocks measured faster than 3 or 4).
  const int helpers = nb >= 4 ? 4 : (nb >= 2 ? 2 : 0);
  const int n0 = helpers == 4 ? max(1, 2 * nb / 10) : helpers == 2 ? (nb + 1) / 2 : nb;
  const int n1 = helpers == 4 ? n0 + (nb - n0 + 1) / 2 : nb;
  if (wave < nb) {  // key block kb = wave (uniform per wave)
    const int kb = wave, key = kb * 32 + col;
    uint2 kc[4];  // the block's rows of the key copy: row 8 u + lane / 8, channels 4 (lane % 8) .. + 3
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int row = kb * 32 + 8 * u + (lane >> 3);
      kc[u] = row < L ? *reinterpret_cast<const uint2*>(kp + at_row_off(row, p.st[kAtK][3]) + 4 * (lane & 7)) : uint2{0u, 0u};
    }
    at_bf8 kh[2], kl[2], vr[2];  // k' = k log2(e) / sqrt(D) = hi + lo (as the forward's query rows)
    {
      at_bf8 kr[2];
      at_row_bf8<D>(kr, kp, min(key, L - 1) * p.st[kAtK][3], grp);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const at_f8 f = __builtin_convertvector(kr[s], at_f8) * p.scale2;
        kh[s] = __builtin_convertvector(f, at_bf8);
        kl[s] = __builtin_convertvector(f - __builtin_convertvector(kh[s], at_f8), at_bf8);
      }
    }
    at_row_bf8<D>(vr, static_cast<const uint16_t*>(p.v) + sl.base(p, kAtV), min(key, L - 1) * p.st[kAtV][3], grp);
#pragma unroll
    for (int u = 0; u < 4; ++u) *reinterpret_cast<uint2*>(&Kt[at_swo<D>(kb * 32 + 8 * u + (lane >> 3), 4 * (lane & 7))]) = kc[u];
    at_f16 dk[1] = {at_zero16()}, dv[1] = {at_zero16()};
    for (int j = 0; j <= nchunks + 1; ++j) {
      __syncthreads();  // chunk j staged; the dS tiles of chunk j - 2 read; the halves of chunk j - 3 added
      if (kb < helpers && j >= 1 && j <= nchunks) {
        // part kb / 2 of dQ^T of query block kb % 2 of chunk j - 1 into Xq (result layout)
        const int part = kb >> 1, kbeg = part == 0 ? n0 : n1, kend = part == 0 ? n1 : nb;
        const int bp = (j - 1) & 1, g16 = lane >> 4, r = lane & 15;
        const int tc = 16 * (g16 & 1) + 4 * (r & 3), tro = 4 * grp + (r >> 2);
        at_f16 acc0 = at_zero16(), acc1 = at_zero16();
        for (int kb2 = kbeg; kb2 < kend; ++kb2) {
          const uint16_t* Th = St + ((bp * nb + kb2) * 2 + (kb & 1)) * 1024;
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            const int ro = 16 * s2 + tro;
            const at_bf8 ka = at_bf8_of(at_read_tr(Kt + at_swo<D>(32 * kb2 + ro, tc)), at_read_tr(Kt + at_swo<D>(32 * kb2 + ro + 8, tc)));
            const at_bf8 sb = at_bf8_of(at_read_tr(Th + at_swo<D>(ro, tc)), at_read_tr(Th + at_swo<D>(ro + 8, tc)));
            if (s2 == 0) acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, sb, acc0, 0, 0, 0);
            else acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, sb, acc1, 0, 0, 0);
          }
        }
        float* x = Xq[bp][part][kb & 1];
#pragma unroll
        for (int c = 0; c < 4; ++c)
          *reinterpret_cast<at_f4*>(&x[4 * (c * 64 + lane)]) = at_f4{acc0[4 * c] + acc1[4 * c], acc0[4 * c + 1] + acc1[4 * c + 1],
                                                                    acc0[4 * c + 2] + acc1[4 * c + 2], acc0[4 * c + 3] + acc1[4 * c + 3]};
      }
      if (j >= nchunks) continue;
      const int b = j & 1;
      if (kb == 0 && j * kAtChunk + lane < L)  // rowsum(dO * O) into the statistics (their entry 2)
        p.stats[(static_cast<int64_t>(zh) * L + j * kAtChunk + lane) * 4 + 2] = -Ds[b][lane];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {  // the chunk's two query blocks
        // S - m - log2 l = Q k'^T - (m + log2 l) and dP - rowsum = dO V^T - rowsum: the
        // accumulators start from the per-query shifts (register i: query 32 h2 + 8 (i / 4) +
        // 4 grp + i % 4 of the chunk), so P = exp2 of the first and dS = P times the second.
        at_f16 s, dp;
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
          const int ql = 32 * h2 + 8 * c4 + 4 * grp;
          const at_f4 ms = *reinterpret_cast<const at_f4*>(&Ms[b][ql]), dd = *reinterpret_cast<const at_f4*>(&Ds[b][ql]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s[4 * c4 + e] = ms[e];
            dp[4 * c4 + e] = dd[e];
          }
        }
        {
          at_bf8 qa[2], ga[2];
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            qa[s2] = __builtin_bit_cast(at_bf8, *reinterpret_cast<const uint4*>(&Qr[b][at_swo<D>(32 * h2 + col, 16 * s2 + 8 * grp)]));
            ga[s2] = __builtin_bit_cast(at_bf8, *reinterpret_cast<const uint4*>(&Gr[b][at_swo<D>(32 * h2 + col, 16 * s2 + 8 * grp)]));
          }
          s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[0], kh[0], s, 0, 0, 0);
          dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ga[0], vr[0], dp, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[1], kh[1], s, 0, 0, 0);
          dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ga[1], vr[1], dp, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[0], kl[0], s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[1], kl[1], s, 0, 0, 0);
        }
        at_f16 pw;
        // A lane past L holds the clamped last key: its weights are finite, and its rows of the
        // key copy are 0, so it adds nothing to dQ. Rows past L have a shift of -inf: weight 0.
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          pw[i] = at_exp2(s[i]);
          s[i] = pw[i] * dp[i];  // dS
        }
        at_accum_tr<D>(dv, dk, Gr[b], 32 * h2, Qr[b], 32 * h2, pw, s, lane);  // dV^T += dO^T P, dK^T += Q^T dS
        // dS^T tile: row = key (this lane's col), columns = the block's queries
        uint16_t* Th = St + ((b * nb + kb) * 2 + h2) * 1024;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const uint4 u = __builtin_bit_cast(uint4, at_bf8_regs(s, 8 * s2));
          *reinterpret_cast<uint2*>(&Th[at_swo<D>(col, 16 * s2 + 4 * grp)]) = uint2{u.x, u.y};
          *reinterpret_cast<uint2*>(&Th[at_swo<D>(col, 16 * s2 + 8 + 4 * grp)]) = uint2{u.z, u.w};
        }
      }
    }
    // the last dQ passes read the other dS tile set before the last barrier: this wave's output scratch now
    uint16_t* sc = St + (((nchunks & 1) * nb + kb) * 2) * 1024;
    if (p.gk != nullptr) at_store_block(static_cast<bf16_t*>(p.gk) + sl.base(p, kAtGK), p.st[kAtGK][3], kb * 32, L, dk[0], p.scale, sc, lane);
    if (p.gv != nullptr) at_store_block(static_cast<bf16_t*>(p.gv) + sl.base(p, kAtGV), p.st[kAtGV][3], kb * 32, L, dv[0], 1.0f, sc, lane);
    return;
  }
  // The two dQ waves. Staging: thread tq holds row tq / 2 of the chunk, channels 16 (tq % 2) .. + 15.
  const int tq = t - 64 * nb, h2q = tq >> 6;  // h2q: the query block of each chunk this wave forms dQ for
  const uint16_t* qp = static_cast<const uint16_t*>(p.q) + sl.base(p, kAtQ);
  const uint16_t* gop = static_cast<const uint16_t*>(p.go) + sl.base(p, kAtGO);
  const uint16_t* opp = static_cast<const uint16_t*>(p.o) + sl.base(p, kAtO);
  float* stats = p.stats + static_cast<int64_t>(zh) * L * 4;
  const int srow = tq >> 1, shalf = tq & 1;
  uint4 qv[2], gv[2], ov[2];
  float2 sq = {0.0f, 0.0f};  // m, log2 l (8 bytes: no register of a wider load left idle in flight)
  auto prefetch = [&](int r0) {
    const int r = min(r0 + srow, L - 1);
    auto ld16 = [](const uint16_t* e) {  // rows are 8-byte aligned
      const uint2 lo = *reinterpret_cast<const uint2*>(e), hi = *reinterpret_cast<const uint2*>(e + 4);
      return uint4{lo.x, lo.y, hi.x, hi.y};
    };
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 16 * shalf + 8 * h;
      qv[h] = ld16(qp + at_row_off(r, p.st[kAtQ][3]) + c);
      gv[h] = ld16(gop + at_row_off(r, p.st[kAtGO][3]) + c);
      ov[h] = ld16(opp + at_row_off(r, p.st[kAtO][3]) + c);
    }
    if (shalf == 0) sq = *reinterpret_cast<const float2*>(&stats[4 * r]);
  };
  auto stage = [&](int r0, int b) {
    const bool in = r0 + srow < L;
    float dd = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 16 * shalf + 8 * h;  // a 16-byte chunk of the swizzled row
      *reinterpret_cast<uint4*>(&Qr[b][srow * D + 8 * ((c >> 3) ^ at_sw<D>(srow))]) = in ? qv[h] : uint4{0u, 0u, 0u, 0u};
      *reinterpret_cast<uint4*>(&Gr[b][srow * D + 8 * ((c >> 3) ^ at_sw<D>(srow))]) = in ? gv[h] : uint4{0u, 0u, 0u, 0u};
      const uint32_t g4[4] = {gv[h].x, gv[h].y, gv[h].z, gv[h].w}, o4[4] = {ov[h].x, ov[h].y, ov[h].z, ov[h].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) dd += at_bf16_lo(g4[e]) * at_bf16_lo(o4[e]) + at_bf16_hi(g4[e]) * at_bf16_hi(o4[e]);
    }
    // the row's other half: the neighbouring lane (DPP quad_perm [1, 0, 3, 2])
    dd += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(dd), 0xB1, 0xF, 0xF, false));
    if (shalf == 0) {
      Ms[b][srow] = in ? -(sq.x + sq.y) : -INFINITY;
      Ds[b][srow] = in ? -dd : 0.0f;
    }
  };
  prefetch(0);
  stage(0, 0);
  if (nchunks > 1) prefetch(kAtChunk);
  bf16_t* gqp = static_cast<bf16_t*>(p.gq) + sl.base(p, kAtGQ);
  const int g16 = lane >> 4, r = lane & 15;
  const int tc = 16 * (g16 & 1) + 4 * (r & 3), tro = 4 * grp + (r >> 2);  // transposing-read lane offsets
  at_f16 held = at_zero16();  // dQ^T of this wave's query block of the previous chunk over key blocks [0, n0)
  for (int j = 0; j <= nchunks + 1; ++j) {
    __syncthreads();  // chunk j staged; the dS tiles of chunk j - 1 and the halves of chunk j - 2 written
    if (j >= 2) {  // chunk j - 2: add key wave h2q's half and store
      for (int part = 0; 2 * part < helpers; ++part) {
        const float* x = Xq[j & 1][part][h2q];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const at_f4 h4 = *reinterpret_cast<const at_f4*>(&x[4 * (c * 64 + lane)]);
#pragma unroll
          for (int e = 0; e < 4; ++e) held[4 * c + e] += h4[e];
        }
      }
      // straight from the result layout: measured faster here than through LDS (the dK / dV stores
      // at the end are not: through LDS they hold the workgroup's end less)
      at_store_block_direct(gqp, p.st[kAtGQ][3], (j - 2) * kAtChunk + 32 * h2q, L, held, p.scale, lane);
    }
    if (j + 1 < nchunks) {
      stage((j + 1) * kAtChunk, (j + 1) & 1);
      if (j + 2 < nchunks) prefetch((j + 2) * kAtChunk);
    }
    if (j == 0 || j > nchunks) continue;
    const int jp = j - 1, bp = jp & 1;
    // dQ^T = sum over key blocks of K^T dS^T: two chains (the two 16-key halves of each block),
    // the next block's operands read while the current block's products run
    at_f16 acc0 = at_zero16(), acc1 = at_zero16();
    at_bf8 ka[2], sb[2];
    auto operands = [&](int kb2) {
      const uint16_t* Th = St + ((bp * nb + kb2) * 2 + h2q) * 1024;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const int ro = 16 * s2 + tro;
        ka[s2] = at_bf8_of(at_read_tr(Kt + at_swo<D>(32 * kb2 + ro, tc)), at_read_tr(Kt + at_swo<D>(32 * kb2 + ro + 8, tc)));
        sb[s2] = at_bf8_of(at_read_tr(Th + at_swo<D>(ro, tc)), at_read_tr(Th + at_swo<D>(ro + 8, tc)));
      }
    };
    operands(0);
    for (int kb2 = 0; kb2 < n0; ++kb2) {
      const at_bf8 a0 = ka[0], a1 = ka[1], b0 = sb[0], b1 = sb[1];
      if (kb2 + 1 < n0) operands(kb2 + 1);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc1, 0, 0, 0);
    }
    held = acc0 + acc1;  // result column: the lane's query; rows: channels
  }
}

// Fused backward, f32 (D = 32, L <= 32 kAtFusedBlocks, no mask): the bf16 kernel's split, phase by
// phase over 32-row query blocks, since f32 dS tiles of two 64-row chunks would not fit in LDS.
// Key waves form S, dP, P and dS of their key block against the phase's query block, accumulate
// dK and dV, and write dS into an f32 tile [32 keys][32 queries]. The two dQ waves stage the next
// query block (Q, dO, rowsum(dO * O), 4 threads per row) and form dQ^T = K^T dS^T of the previous
// block over half of the key blocks each (v_mfma_f32_32x32x2_f32, K from an LDS copy, two chains)
// into LDS; one phase later key wave 0, which has time to spare, adds the halves and stores the
// block's rows. Row tiles, dS tiles and the halves are double buffered by phase parity: one
// barrier per phase.
constexpr int at_fused_f32_lds_bytes(int nb) { return nb * (32 * 32 * 4 + 2 * 32 * 32 * 4); }  // K copy, two dS tile sets

// element (r, c) of a swizzled f32 tile [32][32]: 16-byte chunk c / 4 of row r at slot (c / 4) ^ ((r / 2) % 8)
__device__ __forceinline__ int at_f32sw(int r, int c) { return r * 32 + 4 * ((c >> 2) ^ ((r >> 1) & 7)) + (c & 3); }

__global__ void __launch_bounds__(64 * (kAtFusedBlocks + 2), 3) attn_bwd_fused_f32_kernel(const AttnParams p) {
  constexpr int D = 32, LD = D + 8;
  __shared__ __align__(16) float Qs[2][32 * LD];  // query rows of the phase's block, by parity
  __shared__ __align__(16) float Gs[2][32 * LD];  // output-gradient rows
  __shared__ __align__(16) float Ms[2][2 * 32];   // m, log2 l (rows past L: +inf)
  __shared__ __align__(16) float Ds[2][32];       // rowsum(dO * O)
  __shared__ __align__(16) float Xq[2][2][16 * 64];  // the dQ waves' halves of dQ^T (result layout), by parity
  extern __shared__ __align__(16) float at_lds[];
  const int L = p.len, nb = (L + 31) / 32;  // key blocks; also the query blocks (phases)
  float* Kf = at_lds;                       // [32 nb][32] key rows (0 past L)
  float* St = Kf + 32 * nb * D;             // dS tiles: 1024 floats each, parity, key block
  const int zh = xcd_logical(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));  // as the bf16 kernel
  const AttnSlice sl(p, zh);
  const float* kp = static_cast<const float*>(p.k) + sl.base(p, kAtK);
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, grp = lane >> 5, col = lane & 31;
  if (wave < nb) {  // key block kb = wave (uniform per wave)
    const int kb = wave, key = kb * 32 + col, kcl = min(key, L - 1);
    at_f4 kc[4];  // the block's rows of the key copy: row 8 u + lane / 8, channels 4 (lane % 8) .. + 3
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int row = kb * 32 + 8 * u + (lane >> 3);
      kc[u] = row < L ? *reinterpret_cast<const at_f4*>(kp + at_row_off(row, p.st[kAtK][3]) + 4 * (lane & 7)) : at_f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    at_f4 kr[D / 8], vr[D / 8];
    const float* vp = static_cast<const float*>(p.v) + sl.base(p, kAtV);
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
      kr[c] = *reinterpret_cast<const at_f4*>(kp + at_row_off(kcl, p.st[kAtK][3]) + 8 * c + 4 * grp);
      vr[c] = *reinterpret_cast<const at_f4*>(vp + at_row_off(kcl, p.st[kAtV][3]) + 8 * c + 4 * grp);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) *reinterpret_cast<at_f4*>(&Kf[(kb * 32 + 8 * u + (lane >> 3)) * D + 4 * (lane & 7)]) = kc[u];
    at_f16 dk[1] = {at_zero16()}, dv[1] = {at_zero16()};
    float* gqp = static_cast<float*>(p.gq) + sl.base(p, kAtGQ);
    const bool gq16 = (reinterpret_cast<uintptr_t>(gqp) & 15) == 0 && (p.st[kAtGQ][3] & 3) == 0;
    for (int j = 0; j <= nb + 1; ++j) {
      __syncthreads();  // query block j staged; the dS tiles of block j - 2 read; the halves of block j - 2 written
      if (kb == 0 && j >= 2) {
        // dQ rows of block j - 2: slot u of this lane is query (lane + 64 u) / 8, channels
        // 8 c + 4 h .. + 3 with c = ((lane + 64 u) % 8) / 2 and h = lane % 2 (8 lanes to a row)
        const float* x0 = Xq[j & 1][0];
        const float* x1 = Xq[j & 1][1];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int sl8 = lane + 64 * u, qr = sl8 >> 3, c = (sl8 & 7) >> 1, h = sl8 & 1;
          const int x = 4 * (c * 64 + qr + 32 * h);
          const at_f4 v = (*reinterpret_cast<const at_f4*>(&x0[x]) + *reinterpret_cast<const at_f4*>(&x1[x])) * p.scale;
          const int q = (j - 2) * 32 + qr, d0 = 8 * c + 4 * h;
          if (q < L) {
            if (gq16) {
              *reinterpret_cast<at_f4*>(gqp + at_row_off(q, p.st[kAtGQ][3]) + d0) = v;
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) gqp[at_row_off(q, p.st[kAtGQ][3]) + d0 + e] = v[e];
            }
          }
        }
      }
      if (j >= nb) continue;
      const int b = j & 1;
      if (kb == 0 && lane < 32 && j * 32 + lane < L)  // rowsum(dO * O) into the statistics (their entry 2)
        p.stats[(static_cast<int64_t>(zh) * L + j * 32 + lane) * 4 + 2] = Ds[b][lane];
      at_f16 s, dp;
      at_scores_pair<D>(s, dp, Qs[b], Gs[b], kr, vr, col, grp);  // S = Q K^T, dP = dO V^T
      at_f16 pw;
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {
        const int ql = 8 * c4 + 4 * grp;
        const at_f4 ms0 = *reinterpret_cast<const at_f4*>(&Ms[b][2 * ql]), ms1 = *reinterpret_cast<const at_f4*>(&Ms[b][2 * ql + 4]);
        const at_f4 dd = *reinterpret_cast<const at_f4*>(&Ds[b][ql]);
        const float mq[4] = {ms0[0], ms0[2], ms1[0], ms1[2]}, lq[4] = {ms0[1], ms0[3], ms1[1], ms1[3]};
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int i = 4 * c4 + jj;
          // a lane past L holds the clamped last key: finite weights, and its rows of the key copy
          // are 0, so it adds nothing to dQ; rows past L have m = +inf: weight 0
          pw[i] = at_exp2(fmaf(s[i], p.scale2, -mq[jj]) - lq[jj]);
          s[i] = pw[i] * (dp[i] - dd[jj]);  // dS
        }
      }
      at_accum2<D>(dv, dk, Gs[b], Qs[b], pw, s, col, grp);  // dV^T += dO^T P, dK^T += Q^T dS
      float* T = St + (b * nb + kb) * 1024;  // dS^T tile: row = key (this lane's col), columns = queries
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<at_f4*>(&T[at_f32sw(col, 8 * c + 4 * grp)]) = at_f4{s[4 * c], s[4 * c + 1], s[4 * c + 2], s[4 * c + 3]};
    }
    // the dQ waves read the last dS tiles before the last barrier: they hold the output scratch now
    float* sc = St + kb * (at_scratch_bytes<float>() / 4);
    if (p.gk != nullptr) at_store_block<float>(static_cast<float*>(p.gk) + sl.base(p, kAtGK), p.st[kAtGK][3], kb * 32, L, dk[0], p.scale, sc, lane);
    if (p.gv != nullptr) at_store_block<float>(static_cast<float*>(p.gv) + sl.base(p, kAtGV), p.st[kAtGV][3], kb * 32, L, dv[0], 1.0f, sc, lane);
    return;
  }
  // The two dQ waves. Staging: thread tq holds row tq / 4 of the block, channels 8 (tq % 4) .. + 7.
  const int tq = t - 64 * nb, dqw = tq >> 6;
  const float* qp = static_cast<const float*>(p.q) + sl.base(p, kAtQ);
  const float* gop = static_cast<const float*>(p.go) + sl.base(p, kAtGO);
  const float* opp = static_cast<const float*>(p.o) + sl.base(p, kAtO);
  float* stats = p.stats + static_cast<int64_t>(zh) * L * 4;
  const int srow = tq >> 2, sq4 = tq & 3;
  at_f4 qv[2], gv[2], ov[2];
  float2 sq = {0.0f, 0.0f};  // m, log2 l (8 bytes: no register of a wider load left idle in flight)
  auto prefetch = [&](int r0) {
    const int r = min(r0 + srow, L - 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 8 * sq4 + 4 * h;
      qv[h] = *reinterpret_cast<const at_f4*>(qp + at_row_off(r, p.st[kAtQ][3]) + c);
      gv[h] = *reinterpret_cast<const at_f4*>(gop + at_row_off(r, p.st[kAtGO][3]) + c);
      ov[h] = *reinterpret_cast<const at_f4*>(opp + at_row_off(r, p.st[kAtO][3]) + c);
    }
    if (sq4 == 0) sq = *reinterpret_cast<const float2*>(&stats[4 * r]);
  };
  auto stage = [&](int r0, int b) {
    const bool in = r0 + srow < L;
    const at_f4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    float dd = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 8 * sq4 + 4 * h;
      *reinterpret_cast<at_f4*>(&Qs[b][srow * LD + c]) = in ? qv[h] : z;
      *reinterpret_cast<at_f4*>(&Gs[b][srow * LD + c]) = in ? gv[h] : z;
      dd += gv[h][0] * ov[h][0] + gv[h][1] * ov[h][1] + gv[h][2] * ov[h][2] + gv[h][3] * ov[h][3];
    }
    // the row's four quarters: neighbouring lanes (DPP quad_perm [1, 0, 3, 2], then [2, 3, 0, 1])
    dd += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(dd), 0xB1, 0xF, 0xF, false));
    dd += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(dd), 0x4E, 0xF, 0xF, false));
    if (sq4 == 0) {
      Ms[b][2 * srow] = in ? sq.x : INFINITY;
      Ms[b][2 * srow + 1] = in ? sq.y : 0.0f;
      Ds[b][srow] = in ? dd : 0.0f;
    }
  };
  prefetch(0);
  stage(0, 0);
  if (nb > 1) prefetch(32);
  const int nh = (nb + 1) / 2, kb0 = dqw == 0 ? 0 : nh, kb1 = dqw == 0 ? nh : nb;  // this wave's key blocks
  for (int j = 0; j <= nb + 1; ++j) {
    __syncthreads();  // block j staged; the dS tiles of block j - 1 written; the halves of block j - 3 read
    if (j + 1 < nb) {
      stage((j + 1) * 32, (j + 1) & 1);
      if (j + 2 < nb) prefetch((j + 2) * 32);
    }
    if (j == 0 || j > nb) continue;
    const int bp = (j - 1) & 1;  // block j - 1: dQ^T over this wave's key blocks
    at_f16 acc0 = at_zero16(), acc1 = at_zero16();
    for (int kb2 = kb0; kb2 < kb1; ++kb2) {
      const float* T = St + (bp * nb + kb2) * 1024;
      const float* K = Kf + kb2 * 32 * D;
#pragma unroll
      for (int s2 = 0; s2 < 16; s2 += 2) {
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(K[(s2 + grp) * D + col], T[at_f32sw(s2 + grp, col)], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(K[(s2 + 16 + grp) * D + col], T[at_f32sw(s2 + 16 + grp, col)], acc1, 0, 0, 0);
      }
    }
    float* x = Xq[(j + 1) & 1][dqw];  // block j - 1's parity
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *reinterpret_cast<at_f4*>(&x[4 * (c * 64 + lane)]) = at_f4{acc0[4 * c] + acc1[4 * c], acc0[4 * c + 1] + acc1[4 * c + 1],
                                                                acc0[4 * c + 2] + acc1[4 * c + 2], acc0[4 * c + 3] + acc1[4 * c + 3]};
  }
}

// keep[zh][q][k] = 1 where the DROP kernels keep weight (q, k) of (slice, head) zh, else 0: one
// thread per key pair (2 kh, 2 kh + 1) of a row, grid-stride over the zh * L * ceil(L / 2) pairs.
__global__ void __launch_bounds__(256) attn_drop_keep_kernel(const AttnParams p, uint8_t* __restrict__ keep, int64_t pairs) {
  const int L = p.len, hp = (L + 1) / 2;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < pairs; i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t row = i / hp;  // zh * L + q
    const int kh = static_cast<int>(i - row * hp);
    const int zh = static_cast<int>(row / L), q = static_cast<int>(row - static_cast<int64_t>(zh) * L);
    const uint32_t h = at_drop_bits(at_drop_base(p, zh), q, kh);
    uint8_t* dst = keep + row * L + 2 * kh;
    dst[0] = (h & 0xffffu) >= p.drop_thr ? 1 : 0;
    if (2 * kh + 1 < L) dst[1] = (h >> 16) >= p.drop_thr ? 1 : 0;
  }
}

}  // namespace msda

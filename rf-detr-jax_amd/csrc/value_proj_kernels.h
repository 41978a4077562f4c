// value_proj_kernels.h — gfx950 device code for MSDeformAttn's value projection with its epilogue
// fused: value = where(padding_mask, 0, input @ W^T + b), split into heads and written as
// [B * H, S, D] (src/rfdetr_jax/models/ops.py:377-379, :405-407; Linear, models/layers.py:258-280).
//
// One MFMA GEMM kernel (gemm_kernel) serves the forward and both backward products through tile
// loaders and epilogues:
//   forward   Y[m, n]  = sum_k X[m, k] W[n, k]          (m = (b, s), n = (h, d)); epilogue adds the
//             bias, zeroes masked rows and stores Y[m, n] at value[(b * H + h) * S + s][d];
//   grad_in   dX[m, k] = sum_n dY[m, n] W[n, k]          (dY read from grad_value [B*H, S, D], masked
//             rows zero);
//   grad_w    dW[n, k] = sum_m dY[m, n] X[m, k], and db[n] = sum_m dY[m, n] as column k = K of the
//             same product (X extended by a column of ones), split over m into partial sums that
//             wg_reduce_kernel adds in a fixed order.
// Products run on v_mfma_f32_16x16x4_f32 (f32 operands; bf16 inputs are widened exactly, and the
// weight is rounded to bf16 first when the input is bf16, as weight.astype(x.dtype) does).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace msda {

typedef float vp_f4 __attribute__((ext_vector_type(4)));

constexpr int kGemmBM = 64;   // rows of a workgroup tile
constexpr int kGemmBN = 64;   // columns of a workgroup tile
constexpr int kGemmBK = 64;   // reduction slice staged in LDS per step
constexpr int kGemmLd = kGemmBK + 4;  // LDS row stride: 16-byte rows; the 16 rows an operand read covers span all 64 banks once
constexpr int kGemmPer = kGemmBM * kGemmBK / 256;  // elements of each operand tile a thread stages per step

__device__ __forceinline__ float vp_load(const void* base, int64_t i, bool bf16) {
  if (bf16) return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(base)[i]) << 16);
  return static_cast<const float*>(base)[i];
}

// The same with the dtype fixed at compile time (no branch between a load and its use, so the
// loads of a staging step are all in flight together).
template <typename VT>
__device__ __forceinline__ float vp_ld(const void* base, int64_t i) {
  if constexpr (sizeof(VT) == 2) return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(base)[i]) << 16);
  else return static_cast<const float*>(base)[i];
}

__device__ __forceinline__ float vp_round_bf16(float f) {  // nearest even, quiet NaN
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return __uint_as_float((u | 0x00400000u) & 0xffff0000u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xffff0000u);
}

__device__ __forceinline__ void vp_store(void* base, int64_t i, float v, bool bf16) {
  if (bf16) static_cast<uint16_t*>(base)[i] = static_cast<uint16_t>(__float_as_uint(vp_round_bf16(v)) >> 16);
  else static_cast<float*>(base)[i] = v;
}

struct ValueProjParams {
  const void* x;          // [B, S, K] input (dtype)
  const float* w;         // [N, K] weight (f32)
  const float* bias;      // [N] or null
  const uint8_t* mask;    // [B, S] (non-zero = padded) or null
  void* value;            // forward output [B * H, S, D] (dtype)
  const void* gvalue;     // backward: grad of value [B * H, S, D] (dtype)
  void* gx;               // backward: grad of input [B, S, K] (dtype)
  float* gw_part;         // backward: partial sums [splits][N][K + 1] (last column: bias)
  float* gw;              // backward: grad of weight [N, K] (f32), or null
  float* gb;              // backward: grad of bias [N] (f32), or null
  int bf16;               // input / value dtype is bf16
  int batch, seq, k, n, heads, dim;  // M = batch * seq, N = heads * dim
  int splits;             // grad_w: slices of the m range
  uint32_t dim_magic;     // ceil(2^32 / dim): n / dim = umulhi(n, dim_magic) for n * dim < 2^32
  uint32_t seq_magic;     // ceil(2^32 / seq): m / seq = umulhi(m, seq_magic) for m * seq < 2^32
};

__device__ __forceinline__ int vp_div_dim(const ValueProjParams& p, int n) {
  return static_cast<int>(__umulhi(static_cast<uint32_t>(n), p.dim_magic));
}

// The [B*H, S, D] layout as 32-bit element offsets (every tensor here has fewer than 2^32
// elements, checked on the host): element (m, n) of the [B*S, H*D] view is at
// row_part(m) + col_part(n), row_part(m) = (b H S + s) D for m = (b, s), col_part(n) = h S D + d for
// n = (h, d). Padded rows are zeroed by the callers (in the epilogue or in LDS), so the loads
// themselves carry no condition.
__device__ __forceinline__ uint32_t vp_row_part(const ValueProjParams& p, int m) {
  const uint32_t b = __umulhi(static_cast<uint32_t>(m), p.seq_magic), s = static_cast<uint32_t>(m) - b * static_cast<uint32_t>(p.seq);
  return (b * static_cast<uint32_t>(p.heads) * static_cast<uint32_t>(p.seq) + s) * static_cast<uint32_t>(p.dim);
}

__device__ __forceinline__ uint32_t vp_col_part(const ValueProjParams& p, int n) {
  const uint32_t h = static_cast<uint32_t>(vp_div_dim(p, n)), d = static_cast<uint32_t>(n) - h * static_cast<uint32_t>(p.dim);
  return h * static_cast<uint32_t>(p.seq) * static_cast<uint32_t>(p.dim) + d;
}

// a weight value as the product sees it (rounded to bf16 when the input is bf16)
template <typename VT>
__device__ __forceinline__ float vp_wv(float v) {
  if constexpr (sizeof(VT) == 2) return vp_round_bf16(v);
  else return v;
}

// weight element (n, k) as the product sees it
template <typename VT>
__device__ __forceinline__ float vp_w(const ValueProjParams& p, int n, int k) {
  const float v = p.w[static_cast<uint32_t>(n) * static_cast<uint32_t>(p.k) + static_cast<uint32_t>(k)];
  if constexpr (sizeof(VT) == 2) return vp_round_bf16(v);
  else return v;
}

enum GemmKind { kGemmForward = 0, kGemmGradInput = 1, kGemmGradWeight = 2 };

// A[r, kk] and B[kk, c] of each product (rows r of the output, columns c, reduction kk), for
// indices inside the matrices (the caller clamps and selects).
template <int KIND, typename VT>
struct GemmDims {
  __device__ static int rows(const ValueProjParams& p) { return KIND == kGemmGradWeight ? p.n : p.batch * p.seq; }
  __device__ static int cols(const ValueProjParams& p) { return KIND == kGemmForward ? p.n : KIND == kGemmGradInput ? p.k : p.k + 1; }
  __device__ static int red(const ValueProjParams& p) { return KIND == kGemmForward ? p.k : KIND == kGemmGradInput ? p.n : p.batch * p.seq; }
  // rb: the staged row's dY base (grad_input, fixed per row) or unused
  __device__ static float a(const ValueProjParams& p, int r, int kk) {
    if (KIND == kGemmForward) return vp_ld<VT>(p.x, static_cast<uint32_t>(r) * static_cast<uint32_t>(p.k) + static_cast<uint32_t>(kk));
    if (KIND == kGemmGradInput) return vp_ld<VT>(p.gvalue, vp_row_part(p, r) + vp_col_part(p, kk));
    return vp_ld<VT>(p.gvalue, vp_row_part(p, kk) + vp_col_part(p, r));  // dY^T
  }
  __device__ static float b(const ValueProjParams& p, int kk, int c) {
    if (KIND == kGemmForward) return vp_w<VT>(p, c, kk);    // W^T
    if (KIND == kGemmGradInput) return vp_w<VT>(p, kk, c);  // W
    // X, with the bias column c == K of ones (padded rows are zeroed in LDS)
    const float x = vp_ld<VT>(p.x, static_cast<uint32_t>(kk) * static_cast<uint32_t>(p.k) + static_cast<uint32_t>(min(c, p.k - 1)));
    return c == p.k ? 1.0f : x;
  }
};

// Workgroup: a 64 x 64 output tile (and, for grad_w, one slice of the reduction); 4 waves, each a
// 32 x 32 quarter as 2 x 2 MFMA 16 x 16 blocks. Per 64-wide reduction step the workgroup stages
// A[64][64] and B[64][64] (B stored by column, rows of 68 floats) in LDS; the next step's elements are loaded into
// registers while the MFMAs of the current one run, so each step waits for memory only as long as
// its loads outlast the arithmetic. Operand layout of v_mfma_f32_16x16x4_f32: lane l supplies
// A[l % 16][l / 16] and B[l / 16][l % 16]; its four results are D[4 (l / 16) + j][l % 16], j = 0..3.
template <int KIND, typename VT>
__global__ void __launch_bounds__(256) gemm_kernel(const ValueProjParams p) {
  __shared__ __align__(16) float As[kGemmBM * kGemmLd];
  __shared__ __align__(16) float Bs[kGemmBN * kGemmLd];
  using Dm = GemmDims<KIND, VT>;
  const int R = Dm::rows(p), C = Dm::cols(p), Kr = Dm::red(p);
  const int tiles_c = (C + kGemmBN - 1) / kGemmBN;
  int id = blockIdx.x;
  const int split = KIND == kGemmGradWeight ? id % p.splits : 0;
  if (KIND == kGemmGradWeight) id /= p.splits;
  const int r0 = (id / tiles_c) * kGemmBM, c0 = (id % tiles_c) * kGemmBN;
  int k_lo = 0, k_hi = Kr;
  if (KIND == kGemmGradWeight) {
    const int per = ((Kr + p.splits - 1) / p.splits + kGemmBK - 1) / kGemmBK * kGemmBK;
    k_lo = min(Kr, split * per);
    k_hi = min(Kr, k_lo + per);
  }
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wr = (wave >> 1) * 32, wc = (wave & 1) * 32;  // the wave's quarter
  // Staging order: consecutive threads follow the operand's contiguous direction in memory (along
  // the reduction for X, W and grad_input's dY; along the rows for grad_w's dY^T, whose rows are
  // the channels d of a head; along the columns for grad_w's X).
  auto a_pos = [&](int i, int& row, int& kk) {
    const int e = t + 256 * i;
    if (KIND == kGemmGradWeight) {
      row = e & 63;
      kk = e >> 6;
    } else {
      row = e >> 6;
      kk = e & 63;
    }
  };
  auto b_pos = [&](int i, int& col, int& kk) {
    const int e = t + 256 * i;
    if (KIND == kGemmGradWeight) {
      col = e & 63;
      kk = e >> 6;
    } else {
      col = e >> 6;
      kk = e & 63;
    }
  };
  float ra[kGemmPer], rb[kGemmPer];
  // A tile that lies inside the matrices (rows and columns; the reduction is checked per step)
  // stages without conditions, so all of a step's loads are in flight together, from a uniform
  // base plus a 32-bit element offset formed once per staged element: each step adds a uniform
  // increment. Edge tiles clamp their indices and select zero outside.
  const bool interior = r0 + kGemmBM <= R && c0 + kGemmBN <= C;
  // A operands whose offset advances uniformly with the reduction: X (forward), and dY of
  // grad_input when 64 is a multiple of D (a step then moves 64 / D whole heads)
  const bool a_lin = KIND == kGemmForward || (KIND == kGemmGradInput && 64 % p.dim == 0);
  uint32_t aoff[kGemmPer], boff[kGemmPer];
  uint32_t a_inc = 0, b_inc = 0;
  {
    const uint32_t K = static_cast<uint32_t>(p.k);
    if (KIND == kGemmForward) {
      a_inc = kGemmBK;
      b_inc = kGemmBK;
    } else if (KIND == kGemmGradInput) {
      a_inc = kGemmBK * static_cast<uint32_t>(p.seq);
      b_inc = kGemmBK * K;
    } else {
      b_inc = kGemmBK * K;
    }
#pragma unroll
    for (int i = 0; i < kGemmPer; ++i) {
      int row, kk, col, kb;
      a_pos(i, row, kk);
      b_pos(i, col, kb);
      const int gr = min(r0 + row, R - 1), gk = min(k_lo + kk, max(Kr - 1, 0));
      const int gc = min(c0 + col, C - 1), gkb = k_lo + kb;
      if (KIND == kGemmForward) {
        aoff[i] = static_cast<uint32_t>(gr) * K + static_cast<uint32_t>(gk);
        boff[i] = static_cast<uint32_t>(gc) * K + static_cast<uint32_t>(gkb);
      } else if (KIND == kGemmGradInput) {
        aoff[i] = a_lin ? vp_row_part(p, gr) + vp_col_part(p, gk) : 0u;
        boff[i] = static_cast<uint32_t>(gkb) * K + static_cast<uint32_t>(gc);
      } else {
        aoff[i] = 0u;
        boff[i] = static_cast<uint32_t>(gkb) * K + static_cast<uint32_t>(min(gc, p.k - 1));
      }
    }
  }
  const void* a_base = KIND == kGemmForward ? p.x : p.gvalue;
  const void* b_base = KIND == kGemmForward || KIND == kGemmGradInput ? static_cast<const void*>(p.w) : p.x;
  auto load = [&](int k0, bool checked) {
    const uint32_t step = static_cast<uint32_t>((k0 - k_lo) / kGemmBK);
#pragma unroll
    for (int i = 0; i < kGemmPer; ++i) {
      int row, kk;
      a_pos(i, row, kk);
      int col, kb;
      b_pos(i, col, kb);
      const int gr = r0 + row, gk = k0 + kk, gc = c0 + col, gkb = k0 + kb;
      if (!checked) {
        if (a_lin) ra[i] = vp_ld<VT>(a_base, aoff[i] + step * a_inc);
        else ra[i] = Dm::a(p, gr, gk);
        if (KIND == kGemmGradWeight) {
          const float x = vp_ld<VT>(b_base, boff[i] + step * b_inc);
          rb[i] = gc == p.k ? 1.0f : x;  // the bias column (its offset is clamped into X)
        } else {
          rb[i] = vp_wv<VT>(p.w[boff[i] + step * b_inc]);
        }
      } else {
        const float va = Dm::a(p, min(gr, R - 1), min(gk, Kr - 1));
        const float vb = Dm::b(p, min(gkb, Kr - 1), min(gc, C - 1));
        ra[i] = (gr < R && gk < k_hi) ? va : 0.0f;
        rb[i] = (gc < C && gkb < k_hi) ? vb : 0.0f;
      }
    }
  };
  auto store = [&](int k0) {
#pragma unroll
    for (int i = 0; i < kGemmPer; ++i) {
      int row, kk;
      a_pos(i, row, kk);
      As[row * kGemmLd + kk] = ra[i];
      int col, kb;
      b_pos(i, col, kb);
      Bs[col * kGemmLd + kb] = rb[i];
    }
    if constexpr (KIND == kGemmGradWeight) {
      // padded rows m drop out of the reduction: zero their X entries (and bias ones) in LDS
      if (p.mask != nullptr) {
        __syncthreads();
        const int kk = t & 63, part = t >> 6;  // four threads per reduction index, 16 columns each
        const int m = k0 + kk;
        if (m < k_hi && p.mask[m]) {
#pragma unroll
          for (int c = 0; c < 16; ++c) Bs[(part * 16 + c) * kGemmLd + kk] = 0.0f;
        }
      }
    }
  };
  vp_f4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = vp_f4{0.0f, 0.0f, 0.0f, 0.0f};
  if (k_lo < k_hi) {
    load(k_lo, !interior || k_lo + kGemmBK > k_hi);
    store(k_lo);
    __syncthreads();
  }
  for (int k0 = k_lo; k0 < k_hi; k0 += kGemmBK) {
    const bool more = k0 + kGemmBK < k_hi;
    if (more) load(k0 + kGemmBK, !interior || k0 + 2 * kGemmBK > k_hi);  // in flight during this step's MFMAs
    // 16 reduction indices per group of four MFMA steps: lane group g = l / 16 takes indices
    // kk + 4 g .. kk + 4 g + 3 for steps 0..3 (one 16-byte LDS read each for A and B; the sum over
    // the reduction is the same whichever step an index goes to, as long as A and B agree)
#pragma unroll
    for (int kk = 0; kk < kGemmBK; kk += 16) {
      const int ka = kk + 4 * (lane >> 4);
      vp_f4 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const vp_f4*>(&As[(wr + 16 * i + (lane & 15)) * kGemmLd + ka]);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const vp_f4*>(&Bs[(wc + 16 * j + (lane & 15)) * kGemmLd + ka]);
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][st], b[j][st], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
    if (more) {
      store(k0 + kGemmBK);
      __syncthreads();
    }
  }
  // epilogue: a lane's results lie in 8 rows (i, v) and 2 columns (j); their masks, biases and
  // output offsets are formed once, with clamped indices and no branches, before the stores
  const bool bf = p.bf16 != 0;
  int rr[2][4], cc[2];
  bool rmask[2][4];
  uint32_t rpart[2][4], cpart[2];  // forward: the output offset is rpart + cpart
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      rr[i][v] = r0 + wr + 16 * i + 4 * (lane >> 4) + v;
      rmask[i][v] = false;
      rpart[i][v] = KIND == kGemmForward ? vp_row_part(p, min(rr[i][v], R - 1)) : 0u;
      if (KIND != kGemmGradWeight && p.mask != nullptr) rmask[i][v] = p.mask[min(rr[i][v], R - 1)] != 0;
    }
  float bias[2] = {0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    cc[j] = c0 + wc + 16 * j + (lane & 15);
    cpart[j] = KIND == kGemmForward ? vp_col_part(p, min(cc[j], C - 1)) : 0u;
    if (KIND == kGemmForward && p.bias != nullptr) {
      const float bv = p.bias[min(cc[j], C - 1)];
      bias[j] = bf ? vp_round_bf16(bv) : bv;
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = rr[i][v], c = cc[j];
        if (r >= R || c >= C) continue;
        float y = acc[i][j][v];
        if (KIND == kGemmForward) {
          // Linear (layers.py:276-279), then where(mask, 0, value) (ops.py:378-379)
          y = rmask[i][v] ? 0.0f : y + bias[j];
          vp_store(p.value, rpart[i][v] + cpart[j], y, bf);
        } else if (KIND == kGemmGradInput) {
          // padded rows have no gradient (where(mask, 0, value), ops.py:378-379)
          vp_store(p.gx, static_cast<uint32_t>(r) * static_cast<uint32_t>(p.k) + static_cast<uint32_t>(c), rmask[i][v] ? 0.0f : y, bf);
        } else {
          p.gw_part[(static_cast<int64_t>(split) * p.n + r) * (p.k + 1) + c] = y;
        }
      }
}

// grad_weight [N, K] and grad_bias [N] from the split partial sums, added in split order.
__global__ void __launch_bounds__(256) wg_reduce_kernel(const ValueProjParams p) {
  const int64_t total = static_cast<int64_t>(p.n) * (p.k + 1);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256) {
    float s = 0.0f;
    for (int sp = 0; sp < p.splits; ++sp) s += p.gw_part[sp * total + i];
    const int r = static_cast<int>(i / (p.k + 1)), c = static_cast<int>(i - static_cast<int64_t>(r) * (p.k + 1));
    if (c < p.k) {
      if (p.gw != nullptr) p.gw[static_cast<int64_t>(r) * p.k + c] = s;
    } else if (p.gb != nullptr) {
      p.gb[r] = s;
    }
  }
}

}  // namespace msda

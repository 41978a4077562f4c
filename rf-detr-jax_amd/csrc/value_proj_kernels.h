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
typedef float vp_f16 __attribute__((ext_vector_type(16)));

constexpr int kGemmBM = 64;   // rows of a workgroup tile
constexpr int kGemmBN = 64;   // columns of a workgroup tile
constexpr int kGemmBK = 64;   // reduction slice staged in LDS per step
constexpr int kGemmLd = kGemmBK + 4;  // LDS row stride: 16-byte rows; the 16 rows an operand read covers span all 64 banks once
constexpr int kGemmPer = kGemmBM * kGemmBK / 256;  // elements of each operand tile a thread stages per step

// Element i of a value-dtype tensor as f32, the dtype fixed at compile time (no branch between a
// load and its use, so the loads of a staging step are all in flight together).
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
  float* gw_part;         // backward: partial sums of grad_weight [splits][N][K], then of grad_bias [splits][N]
  float* gw;              // backward: grad of weight [N, K] (f32), or null
  float* gb;              // backward: grad of bias [N] (f32), or null
  int bf16;               // input / value dtype is bf16
  int batch, seq, k, n, heads, dim;  // M = batch * seq, N = heads * dim
  int splits;             // grad_w: slices of the m range
  uint32_t dim_magic;     // ceil(2^32 / dim): n / dim = umulhi(n, dim_magic) for n * dim < 2^32; 0 for dim 1
  uint32_t seq_magic;     // ceil(2^32 / seq): m / seq = umulhi(m, seq_magic) for m * seq < 2^32; 0 for seq 1
};

// x / divisor by its magic (vp_magic); a divisor of 1 has no 32-bit magic (2^32) and is marked 0.
__device__ __forceinline__ uint32_t vp_div(uint32_t x, uint32_t magic) { return magic != 0u ? __umulhi(x, magic) : x; }

__device__ __forceinline__ int vp_div_dim(const ValueProjParams& p, int n) {
  return static_cast<int>(vp_div(static_cast<uint32_t>(n), p.dim_magic));
}

// The [B*H, S, D] layout as 32-bit element offsets (every tensor here has fewer than 2^32
// elements, checked on the host): element (m, n) of the [B*S, H*D] view is at
// row_part(m) + col_part(n), row_part(m) = (b H S + s) D for m = (b, s), col_part(n) = h S D + d for
// n = (h, d). Padded rows are zeroed by the callers (in the epilogue or in LDS), so the loads
// themselves carry no condition.
__device__ __forceinline__ uint32_t vp_row_part(const ValueProjParams& p, int m) {
  const uint32_t b = vp_div(static_cast<uint32_t>(m), p.seq_magic), s = static_cast<uint32_t>(m) - b * static_cast<uint32_t>(p.seq);
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

// Epilogue inputs of a lane: its results lie in 8 rows (i, v) and 2 columns (j) of the tile. The
// mask bytes and biases are loaded before the main loop (their latency hides behind it) and
// without branches: a missing mask or bias reads another tensor of at least as many elements, and
// the value is ignored.
struct VpEpi {
  int pad[2][4];  // mask bytes of the rows (forward, grad_input)
  float bias[2];  // forward
};

template <int KIND>
__device__ __forceinline__ void vp_epi_load(const ValueProjParams& p, int R, int C, int r0, int c0, int wr, int wc, int lane, VpEpi& e) {
  // R = M rows for the forward and grad_input: the input (forward) and grad_value (grad_input) have
  // at least M elements and are never NULL when those kernels run
  const uint8_t* msrc = p.mask != nullptr ? p.mask : static_cast<const uint8_t*>(KIND == kGemmForward ? p.x : p.gvalue);
  const float* bsrc = p.bias != nullptr ? p.bias : p.w;  // N floats either way
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) e.pad[i][v] = KIND == kGemmGradWeight ? 0 : msrc[min(r0 + wr + 16 * i + 4 * (lane >> 4) + v, R - 1)];
#pragma unroll
  for (int j = 0; j < 2; ++j) e.bias[j] = KIND == kGemmForward ? bsrc[min(c0 + wc + 16 * j + (lane & 15), C - 1)] : 0.0f;
}

// Stores of a lane's 16 results: forward adds the bias, zeroes padded rows and writes the
// [B * H, S, D] layout; grad_input zeroes padded rows; grad_w writes slice `split` of the partial
// sums [splits][N][K + 1] (columns c < C).
template <int KIND, typename VT>
__device__ __forceinline__ void vp_epilogue(const ValueProjParams& p, const vp_f4 (&acc)[2][2], const VpEpi& e, int R, int C, int r0,
                                            int c0, int wr, int wc, int lane, int split) {
  constexpr bool bf = sizeof(VT) == 2;
  const bool has_mask = p.mask != nullptr;
  int rr[2][4], cc[2];
  bool rmask[2][4];
  uint32_t rpart[2][4], cpart[2];  // forward: the output offset is rpart + cpart
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      rr[i][v] = r0 + wr + 16 * i + 4 * (lane >> 4) + v;
      rmask[i][v] = KIND != kGemmGradWeight && has_mask && e.pad[i][v] != 0;
      rpart[i][v] = KIND == kGemmForward ? vp_row_part(p, min(rr[i][v], R - 1)) : 0u;
    }
  float bias[2] = {0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    cc[j] = c0 + wc + 16 * j + (lane & 15);
    cpart[j] = KIND == kGemmForward ? vp_col_part(p, min(cc[j], C - 1)) : 0u;
    if (KIND == kGemmForward && p.bias != nullptr) bias[j] = bf ? vp_round_bf16(e.bias[j]) : e.bias[j];
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
          // Linear (layers.py:276-279), then where(mask, 0, value) (ops.py:377-378)
          y = rmask[i][v] ? 0.0f : y + bias[j];
          vp_store(p.value, rpart[i][v] + cpart[j], y, bf);
        } else if (KIND == kGemmGradInput) {
          // padded rows have no gradient (where(mask, 0, value), ops.py:377-378)
          vp_store(p.gx, static_cast<uint32_t>(r) * static_cast<uint32_t>(p.k) + static_cast<uint32_t>(c), rmask[i][v] ? 0.0f : y, bf);
        } else {
          const int64_t nk = static_cast<int64_t>(p.n) * p.k;  // column K is the bias (column of ones)
          if (c < p.k) p.gw_part[(static_cast<int64_t>(split) * p.n + r) * p.k + c] = y;
          else p.gw_part[nk * p.splits + static_cast<int64_t>(split) * p.n + r] = y;
        }
      }
}

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
  VpEpi epi;
  vp_epi_load<KIND>(p, R, C, r0, c0, wr, wc, lane, epi);
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
  vp_epilogue<KIND, VT>(p, acc, epi, R, C, r0, c0, wr, wc, lane, split);
}

// ---- 16-byte operand path ---------------------------------------------------------------------
// Used when every operand vector of four consecutive elements is contiguous and aligned (K and D
// multiples of 4, aligned base pointers; checked on the host). Same LDS row layout as gemm_kernel;
// the differences:
//   * tiles of BM = 32 or 64 rows x 64 columns (the host takes 32 when 64-row tiles would leave
//     CUs with uneven work), 8 BM threads. The product runs on v_mfma_f32_32x32x2_f32 (on gfx950
//     it sustains the full f32 matrix rate, 64 cycles per 4096 flops; 16x16x4 sustains 40-48
//     cycles per 2048). Each wave owns one 32 x 32 block and half of every step's reduction (groups
//     of 8 indices alternate between the two waves of a block), so one wave's staging arithmetic,
//     LDS traffic and barrier waits overlap the other's MFMAs; the two halves are added in LDS at
//     the end;
//   * each thread loads its 4-element vectors of A and B (16-byte loads for f32, 8-byte for bf16)
//     two steps ahead of the MFMAs (two register sets) into two LDS buffers, so a step's loads have
//     two steps of arithmetic to arrive and each step has one barrier;
//   * loads clamp their indices into the matrices; what lies past the reduction's end, outside the
//     matrices or on padded rows is replaced by zeros when stored to LDS (no branch between a load
//     and the MFMAs it overlaps);
//   * an operand stored along the reduction in memory (X and W in the forward, dY in grad_input)
//     is copied vector by vector; one stored along the rows or columns (W in grad_input, dY^T and X
//     in grad_w) is loaded as 4-row vectors at consecutive reduction indices and transposed in
//     registers;
//   * the output tile goes through LDS so each thread stores whole 4-element vectors;
//   * grad_w has no column of ones: the bias gradient is the sum of the staged dY^T rows, formed by
//     the workgroups of the first column tile; padded rows m are zeroed in dY^T's registers.
template <int BM>
struct G4 {
  static constexpr int kThreads = 8 * BM;
  static constexpr int kBlocks = BM / 16;                              // 32 x 32 blocks x 2 halves = waves
  static constexpr int kNA = BM * kGemmBK / 4 / kThreads;              // A vectors per thread and step (2)
  static constexpr int kNB = kGemmBN * kGemmBK / 4 / kThreads;         // B vectors per thread and step
  static constexpr int kEQ = BM * kGemmBN / 4 / kThreads;              // output vectors per thread (2)
  static constexpr int kABuf = BM * kGemmLd, kBBuf = kGemmBN * kGemmLd;  // floats of one buffer
  static constexpr int kLdsBytes = 2 * (kABuf + kBBuf) * static_cast<int>(sizeof(float));
};

template <typename VT>
__device__ __forceinline__ vp_f4 vp_ld4(const void* base, uint32_t i) {  // elements i .. i + 3
  if constexpr (sizeof(VT) == 2) {
    const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + i);
    return vp_f4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                 __uint_as_float(u.y & 0xffff0000u)};
  } else {
    return *reinterpret_cast<const vp_f4*>(static_cast<const float*>(base) + i);
  }
}

template <typename VT>
__device__ __forceinline__ vp_f4 vp_ldw4(const float* w, uint32_t i) {  // weight, as the product sees it
  const vp_f4 v = *reinterpret_cast<const vp_f4*>(w + i);
  return vp_f4{vp_wv<VT>(v[0]), vp_wv<VT>(v[1]), vp_wv<VT>(v[2]), vp_wv<VT>(v[3])};
}

template <typename VT>
__device__ __forceinline__ void vp_store4(void* base, uint32_t i, vp_f4 v) {  // elements i .. i + 3, i % 4 == 0
  if constexpr (sizeof(VT) == 2) {
    const uint32_t h0 = __float_as_uint(vp_round_bf16(v[0])) >> 16, h1 = __float_as_uint(vp_round_bf16(v[1])) >> 16;
    const uint32_t h2 = __float_as_uint(vp_round_bf16(v[2])) >> 16, h3 = __float_as_uint(vp_round_bf16(v[3])) >> 16;
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + i) = uint2{h0 | (h1 << 16), h2 | (h3 << 16)};
  } else {
    *reinterpret_cast<vp_f4*>(static_cast<float*>(base) + i) = v;
  }
}

__device__ __forceinline__ vp_f4 vp_sel4(bool ok, vp_f4 v) {
  return vp_f4{ok ? v[0] : 0.0f, ok ? v[1] : 0.0f, ok ? v[2] : 0.0f, ok ? v[3] : 0.0f};
}

// Staging geometry of one operand tile of ROWS rows x 64 reduction offsets: along the reduction
// ("k-major"), vector j of the thread is tile row e >> 4, offsets 4 (e & 15) .. + 3, e = t + TH j
// (16 consecutive threads read one 256-byte row segment); along the rows, the thread covers rows
// 4 bq .. 4 bq + 3 at offsets kk0 + j, j < NV (ROWS / 4 consecutive threads read consecutive rows).
template <int ROWS, int TH>
struct G4Geo {
  static constexpr int NV = ROWS * kGemmBK / 4 / TH;
  static constexpr int RQ = ROWS / 4;
  __device__ static int krow(int t, int j) { return (t + TH * j) >> 4; }
  __device__ static int kvec(int t, int j) { return 4 * ((t + TH * j) & 15); }
  __device__ static int bq(int t) { return t % RQ; }
  __device__ static int kk0(int t) { return (t / RQ) * NV; }
  template <bool KMAJOR>
  __device__ static void put(float* S, int t, const vp_f4 (&v)[NV]) {
    if constexpr (KMAJOR) {
#pragma unroll
      for (int j = 0; j < NV; ++j) *reinterpret_cast<vp_f4*>(&S[krow(t, j) * kGemmLd + kvec(t, j)]) = v[j];
    } else {
      // transposed: row 4 bq + jj takes element jj of each vector (NV consecutive offsets)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float* d = &S[(4 * bq(t) + jj) * kGemmLd + kk0(t)];
        if constexpr (NV == 4) *reinterpret_cast<vp_f4*>(d) = vp_f4{v[0][jj], v[1][jj], v[2][jj], v[3][jj]};
        else if constexpr (NV == 2) *reinterpret_cast<float2*>(d) = float2{v[0][jj], v[1][jj]};
        else static_assert(NV == 2 || NV == 4, "two or four offsets per transposed row");
      }
    }
  }
};

template <int KIND, typename VT, int BM>
__global__ void __launch_bounds__(G4<BM>::kThreads) gemm4_kernel(const ValueProjParams p) {
  using Cfg = G4<BM>;
  constexpr int TH = Cfg::kThreads;
  using GA = G4Geo<BM, TH>;
  using GB = G4Geo<kGemmBN, TH>;
  constexpr int NA = GA::NV, NB = GB::NV;
  constexpr bool kA_kmajor = KIND != kGemmGradWeight;  // A along the reduction: X (forward), dY (grad_input)
  constexpr bool kB_kmajor = KIND == kGemmForward;     // B along the reduction: W (forward)
  extern __shared__ __align__(16) float g4_lds[];
  const int M = p.batch * p.seq, N = p.n, K = p.k;
  const int R = KIND == kGemmGradWeight ? N : M;
  const int C = KIND == kGemmForward ? N : K;
  const int Kr = KIND == kGemmForward ? K : KIND == kGemmGradInput ? N : M;
  const int tiles_c = (C + kGemmBN - 1) / kGemmBN;
  // Workgroups are dispatched to the 8 XCDs in turn (id % 8); the tile order is remapped so that
  // each XCD runs a contiguous range of tiles: the column tiles of a row of tiles (which read the
  // same A rows) and, in grad_w, the tiles of one reduction slice share that XCD's L2.
  int id;
  {
    const int g = static_cast<int>(gridDim.x), h = static_cast<int>(blockIdx.x), per = g >> 3, rem = g & 7, xcd = h & 7;
    id = xcd * per + min(xcd, rem) + (h >> 3);
  }
  const int tiles = KIND == kGemmGradWeight ? static_cast<int>(gridDim.x) / p.splits : 0;
  const int split = KIND == kGemmGradWeight ? id / tiles : 0;  // slice-major
  if (KIND == kGemmGradWeight) id -= split * tiles;
  const int r0 = (id / tiles_c) * BM, c0 = (id % tiles_c) * kGemmBN;
  int k_lo = 0, k_hi = Kr;
  if (KIND == kGemmGradWeight) {
    const int per = ((Kr + p.splits - 1) / p.splits + kGemmBK - 1) / kGemmBK * kGemmBK;
    k_lo = min(Kr, split * per);
    k_hi = min(Kr, k_lo + per);
  }
  const int nsteps = (k_hi - k_lo + kGemmBK - 1) / kGemmBK;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int blk = wave % Cfg::kBlocks, kpart = wave / Cfg::kBlocks;  // 32 x 32 block, reduction half
  const int wr = (blk >> 1) * 32, wc = (blk & 1) * 32;               // the block's rows and columns
  // epilogue inputs of the thread's output vectors (rows (t >> 4) + (TH / 16) q, columns
  // 4 (t & 15) .. + 3), loaded now so that their latency hides behind the main loop; a missing mask
  // or bias reads another tensor of at least as many elements and is ignored
  int epad[Cfg::kEQ];
  float ebias[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int q = 0; q < Cfg::kEQ; ++q) epad[q] = 0;
  if (KIND != kGemmGradWeight) {
    const uint8_t* msrc = p.mask != nullptr ? p.mask : static_cast<const uint8_t*>(KIND == kGemmForward ? p.x : p.gvalue);
#pragma unroll
    for (int q = 0; q < Cfg::kEQ; ++q) epad[q] = msrc[min(r0 + (t >> 4) + (TH / 16) * q, R - 1)];
  }
  if (KIND == kGemmForward) {
    const float* bsrc = p.bias != nullptr ? p.bias : p.w;
#pragma unroll
    for (int u = 0; u < 4; ++u) ebias[u] = bsrc[min(c0 + 4 * (t & 15) + u, C - 1)];
  }
  // Per-vector row (or column) parts of the addresses and their validity, fixed over the steps.
  uint32_t abase[NA], bbase[NB];
  bool a_ok[NA], b_ok[NB];
#pragma unroll
  for (int j = 0; j < NA; ++j) {
    if (KIND == kGemmForward) {
      a_ok[j] = r0 + GA::krow(t, j) < M;
      abase[j] = static_cast<uint32_t>(min(r0 + GA::krow(t, j), M - 1)) * static_cast<uint32_t>(K);
    } else if (KIND == kGemmGradInput) {
      a_ok[j] = r0 + GA::krow(t, j) < M;
      abase[j] = vp_row_part(p, min(r0 + GA::krow(t, j), M - 1));
    } else {
      a_ok[j] = r0 + 4 * GA::bq(t) < N;  // dY^T rows n .. n + 3: one head's channels
      abase[j] = vp_col_part(p, min(r0 + 4 * GA::bq(t), N - 4));
    }
  }
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    if (KIND == kGemmForward) {
      b_ok[j] = c0 + GB::krow(t, j) < N;
      bbase[j] = static_cast<uint32_t>(min(c0 + GB::krow(t, j), N - 1)) * static_cast<uint32_t>(K);
    } else {
      b_ok[j] = c0 + 4 * GB::bq(t) < K;  // W[n][c .. c + 3] (grad_input), X[m][c .. c + 3] (grad_w)
      bbase[j] = static_cast<uint32_t>(min(c0 + 4 * GB::bq(t), K - 4));
    }
  }
  const void* a_src = KIND == kGemmForward ? p.x : p.gvalue;
  const bool has_mask = p.mask != nullptr;
  const uint8_t* mask_src = has_mask ? p.mask : static_cast<const uint8_t*>(p.x);  // M bytes either way
  // reduction offset of vector j at step s, and whether it lies inside the product
  auto a_k = [&](int s, int j) { return k_lo + s * kGemmBK + (kA_kmajor ? GA::kvec(t, j) : GA::kk0(t) + j); };
  auto b_k = [&](int s, int j) { return k_lo + s * kGemmBK + (kB_kmajor ? GB::kvec(t, j) : GB::kk0(t) + j); };
  // A register set holds one step's vectors as loaded; the validity selects (zeros outside the
  // matrices, past the reduction's end and on padded rows) are applied when the set is stored, so
  // no instruction between a load and the MFMAs it overlaps waits for it.
  struct Set {
    vp_f4 a[NA], b[NB];
    int pad[NA];  // grad_w: the mask byte of row m (read from X when there is no mask, then unused)
  };
  // Loads clamp their indices into the matrices (rows and columns were clamped above, the
  // reduction index is clamped here), so every address is valid without a condition.
  auto load = [&](int s, Set& g) {
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      const int k = a_k(s, j);
      if (KIND == kGemmForward) g.a[j] = vp_ld4<VT>(a_src, abase[j] + static_cast<uint32_t>(min(k, K - 4)));
      else if (KIND == kGemmGradInput) g.a[j] = vp_ld4<VT>(a_src, abase[j] + vp_col_part(p, min(k, N - 4)));  // dY[m][n .. n + 3]
      else g.a[j] = vp_ld4<VT>(a_src, vp_row_part(p, min(k, M - 1)) + abase[j]);  // dY^T[n .. n + 3][m]
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int k = b_k(s, j);
      if (KIND == kGemmForward) g.b[j] = vp_ldw4<VT>(p.w, bbase[j] + static_cast<uint32_t>(min(k, K - 4)));
      else if (KIND == kGemmGradInput)  // W[n][c .. c + 3]
        g.b[j] = vp_ldw4<VT>(p.w, static_cast<uint32_t>(min(k, N - 1)) * static_cast<uint32_t>(K) + bbase[j]);
      else  // X[m][c .. c + 3]
        g.b[j] = vp_ld4<VT>(p.x, static_cast<uint32_t>(min(k, M - 1)) * static_cast<uint32_t>(K) + bbase[j]);
    }
    if (KIND == kGemmGradWeight) {  // the mask bytes after the vectors (compared when stored)
#pragma unroll
      for (int j = 0; j < NA; ++j) g.pad[j] = mask_src[min(a_k(s, j), M - 1)];
    }
  };
  auto store = [&](int s, const Set& g, float* As, float* Bs) {
    vp_f4 ra[NA], rb[NB];
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      const bool ok = a_ok[j] && a_k(s, j) < k_hi && (KIND != kGemmGradWeight || !has_mask || g.pad[j] == 0);
      ra[j] = vp_sel4(ok, g.a[j]);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) rb[j] = vp_sel4(b_ok[j] && b_k(s, j) < k_hi, g.b[j]);
    GA::template put<kA_kmajor>(As, t, ra);
    GB::template put<kB_kmajor>(Bs, t, rb);
  };
  // two accumulators (alternate MFMA steps) so a wave always has two independent MFMA chains
  vp_f16 acc, acc2;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = acc2[i] = 0.0f;
  // grad_w's bias gradient: the workgroups of the first column tile sum dY^T rows (row t >> 3,
  // reduction offsets 8 (t & 7) .. + 7 of each step, in order; then over the 8 lanes of a row)
  const bool bias_rows = KIND == kGemmGradWeight && c0 == 0;
  float bsum = 0.0f;
  // Reduction groups of 8 indices: this wave takes groups 2 q + kpart of each step. In group g,
  // lanes 0-31 take indices 8 g + st and lanes 32-63 take 8 g + 4 + st for MFMA steps st = 0..3
  // (v_mfma_f32_32x32x2_f32: lane l supplies A[l % 32][l / 32] and B[l / 32][l % 32]), so each
  // operand of a group is one 16-byte LDS read. The operands of the next group are read while the
  // MFMAs of the current one run (two register sets; the scheduling barriers keep that order).
  auto compute = [&](const float* As, const float* Bs) {
    vp_f4 a[2], b[2];
    auto rd = [&](int q, vp_f4& ra, vp_f4& rb) {
      const int ka = 8 * (2 * q + kpart) + 4 * (lane >> 5);
      ra = *reinterpret_cast<const vp_f4*>(&As[(wr + (lane & 31)) * kGemmLd + ka]);
      rb = *reinterpret_cast<const vp_f4*>(&Bs[(wc + (lane & 31)) * kGemmLd + ka]);
    };
    rd(0, a[0], b[0]);
#pragma unroll
    for (int q = 0; q < kGemmBK / 16; ++q) {
      if (q + 1 < kGemmBK / 16) rd(q + 1, a[(q + 1) & 1], b[(q + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int st = 0; st < 4; st += 2) {
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[q & 1][st], b[q & 1][st], acc, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[q & 1][st + 1], b[q & 1][st + 1], acc2, 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (bias_rows) {
      const float* row = &As[(t >> 3) * kGemmLd + 8 * (t & 7)];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const vp_f4 v = *reinterpret_cast<const vp_f4*>(row + 4 * q);
        bsum += v[0];
        bsum += v[1];
        bsum += v[2];
        bsum += v[3];
      }
    }
  };
  float* A0 = g4_lds;
  float* B0 = A0 + Cfg::kABuf;
  float* A1 = B0 + Cfg::kBBuf;
  float* B1 = A1 + Cfg::kABuf;
  if (nsteps > 0) {
    // Steps go in pairs with no branch inside (an odd count adds one step of zeros), and the
    // scheduling barriers keep each step's loads ahead of the MFMAs they overlap: the compiler
    // would otherwise sink them below the arithmetic and drain them at once.
    Set g0, g1;
    load(0, g0);
    load(1, g1);  // past the end: zeros
    __builtin_amdgcn_sched_barrier(0);
    store(0, g0, A0, B0);
    __syncthreads();
    for (int s = 0; s < nsteps; s += 2) {
      // step s: next-but-one loads into set 0, MFMAs on buffer 0, set 1 (step s + 1) into buffer 1
      load(s + 2, g0);
      __builtin_amdgcn_sched_barrier(0);
      compute(A0, B0);
      __builtin_amdgcn_sched_barrier(0);
      store(s + 1, g1, A1, B1);
      __syncthreads();
      load(s + 3, g1);
      __builtin_amdgcn_sched_barrier(0);
      compute(A1, B1);
      __builtin_amdgcn_sched_barrier(0);
      store(s + 2, g0, A0, B0);
      __syncthreads();
    }
  }
  if (bias_rows) {
    float v = bsum;
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 4, 64);
    const int r = r0 + (t >> 3);
    if ((t & 7) == 0 && r < N) p.gw_part[static_cast<int64_t>(N) * K * p.splits + static_cast<int64_t>(split) * N + r] = v;
  }
  // Epilogue through LDS (free after the last step's barrier; with no steps it was never used):
  // the first reduction half writes its blocks (row stride kGemmLd), the second adds its own, then
  // each thread stores 4-element vectors of output rows. C is a multiple of 4, so a vector is
  // inside the output or outside it as a whole. The 32 x 32 result layout: lane l holds
  // D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32], i = 0..15.
  acc += acc2;
  float* T = g4_lds;
  auto tix = [&](int i) { return (wr + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3)) * kGemmLd + wc + (lane & 31); };
  if (kpart == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) T[tix(i)] = acc[i];
  }
  __syncthreads();
  if (kpart == 1) {
#pragma unroll
    for (int i = 0; i < 16; ++i) T[tix(i)] += acc[i];
  }
  __syncthreads();
  vp_f4 bias4 = {0.0f, 0.0f, 0.0f, 0.0f};
  if (KIND == kGemmForward && p.bias != nullptr)
    bias4 = vp_f4{vp_wv<VT>(ebias[0]), vp_wv<VT>(ebias[1]), vp_wv<VT>(ebias[2]), vp_wv<VT>(ebias[3])};
  const int cv = 4 * (t & 15), c = c0 + cv;
  const uint32_t cpart = KIND == kGemmForward ? vp_col_part(p, min(c, C - 4)) : 0u;
#pragma unroll
  for (int q = 0; q < Cfg::kEQ; ++q) {
    const int row = (t >> 4) + (TH / 16) * q, r = r0 + row;
    if (r >= R || c >= C) continue;
    vp_f4 y = *reinterpret_cast<const vp_f4*>(&T[row * kGemmLd + cv]);
    const bool padded = KIND != kGemmGradWeight && has_mask && epad[q] != 0;
    if (KIND == kGemmForward) {
      // Linear (layers.py:276-279), then where(mask, 0, value) (ops.py:377-378)
      y = padded ? vp_f4{0.0f, 0.0f, 0.0f, 0.0f} : y + bias4;
      vp_store4<VT>(p.value, vp_row_part(p, r) + cpart, y);
    } else if (KIND == kGemmGradInput) {
      // padded rows have no gradient (where(mask, 0, value), ops.py:377-378)
      if (padded) y = vp_f4{0.0f, 0.0f, 0.0f, 0.0f};
      vp_store4<VT>(p.gx, static_cast<uint32_t>(r) * static_cast<uint32_t>(K) + static_cast<uint32_t>(c), y);
    } else {
      *reinterpret_cast<vp_f4*>(&p.gw_part[(static_cast<int64_t>(split) * N + r) * K + c]) = y;
    }
  }
}

// grad_weight [N, K] and grad_bias [N] from the split partial sums, added in split order (the
// loads of eight splits are issued before their additions).
__global__ void __launch_bounds__(256) wg_reduce_kernel(const ValueProjParams p) {
  const int64_t nk = static_cast<int64_t>(p.n) * p.k, total = nk + p.n;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256) {
    const bool w = i < nk;
    const float* src = w ? p.gw_part + i : p.gw_part + nk * p.splits + (i - nk);
    const int64_t stride = w ? nk : p.n;
    float s = 0.0f;
    int sp = 0;
    for (; sp + 8 <= p.splits; sp += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = src[(sp + u) * stride];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; sp < p.splits; ++sp) s += src[sp * stride];
    if (w) {
      if (p.gw != nullptr) p.gw[i] = s;
    } else if (p.gb != nullptr) {
      p.gb[i - nk] = s;
    }
  }
}

}  // namespace msda

// attention_abi.hip — C ABI of the decoder self-attention kernels (include/msda.h): validation,
// launch planning, kernel launches. Validation runs before any HIP call.
#include "msda.h"
#include "msda_launch.h"
#include "attention_kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>

namespace {

using msda_host::aligned_to;
using msda_host::fail;

// f32 kernels: two row tiles [64][D + 8] and three floats per row (more than the four waves' output
// scratch, which reuses them after the last chunk)
int lds_bytes(int d) { return (d == 32 ? msda::at_lds_floats<32>() : msda::at_lds_floats<64>()) * 4; }
static_assert(msda::at_lds_floats<32>() * 4 >= 4 * msda::at_scratch_bytes<float>(), "f32 attention LDS holds the output scratch");

// bf16 kernels: two swizzled row tiles [64][D] of bf16, and (key side) three floats per row; at
// least the four waves' output scratch, which reuses them after the last chunk
int lds_bf16(int d, bool rows_f32) {
  return std::max(2 * msda::kAtChunk * d * 2 + (rows_f32 ? 3 * msda::kAtChunk * 4 : 0), 4 * msda::at_scratch_bytes<msda::bf16_t>());
}

int at_validate(int dtype, int batch, int groups, int heads, int len, int head_dim, const int64_t* strides, int ntensors) {
  if (dtype != MSDA_DTYPE_F32 && dtype != MSDA_DTYPE_BF16) return fail(MSDA_ERR_UNSUPPORTED, "attention: unsupported dtype code %d", dtype);
  if (batch < 0 || groups < 0 || heads < 0 || len < 0) return fail(MSDA_ERR_INVALID_ARGUMENT, "attention: negative extent");
  if (head_dim != 32 && head_dim != 64) return fail(MSDA_ERR_UNSUPPORTED, "attention: head_dim %d (32 or 64 supported)", head_dim);
  if (static_cast<int64_t>(batch) * groups * heads >= (int64_t{1} << 31) || len > 65536)
    return fail(MSDA_ERR_UNSUPPORTED, "attention: too many slices or rows");
  if (strides == nullptr) return fail(MSDA_ERR_INVALID_ARGUMENT, "attention: NULL strides");
  for (int i = 0; i < 4 * ntensors; ++i)
    if (strides[i] < 0 || strides[i] % 4 != 0)
      return fail(MSDA_ERR_INVALID_ARGUMENT, "attention: stride %d (%lld) must be a non-negative multiple of 4", i,
                  static_cast<long long>(strides[i]));
  for (int t = 0; t < ntensors; ++t)  // the kernels form row offsets within a (slice, head) in 32 bits
    if (strides[4 * t + 3] >= (int64_t{1} << 24) || static_cast<int64_t>(len) * strides[4 * t + 3] >= (int64_t{1} << 31))
      return fail(MSDA_ERR_UNSUPPORTED, "attention: row stride %lld of tensor %d too large for %d rows",
                  static_cast<long long>(strides[4 * t + 3]), t, len);
  return MSDA_OK;
}

msda::AttnParams at_params(int dtype, int batch, int groups, int heads, int len, int head_dim, const int64_t* strides, int ntensors,
                           const int* order) {
  msda::AttnParams p{};
  p.batch = batch;
  p.groups = groups;
  p.heads = heads;
  p.len = len;
  p.scale = 1.0f / std::sqrt(static_cast<float>(head_dim));
  p.scale2 = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(head_dim)));
  for (int t = 0; t < ntensors; ++t)
    for (int j = 0; j < 4; ++j) p.st[order[t]][j] = strides[4 * t + j];
  (void)dtype;
  return p;
}

// Row blocks per workgroup of the f32 query-side backward: 4, unless that leaves more waves without
// a block than 2 does (at 300 rows, 10 blocks: 4 per workgroup idles 2 of 12 waves, 2 per
// workgroup none). The other kernels always take 4: fewer workgroups per (slice, head) stage the
// streamed side, which outweighs the idle waves (measured at 300 rows: forward bf16 53.4 against
// 58.9 us, f32 131.5 against 133.3, 8 blocks 81.6; bf16 grad_q step 188.5 against 194.0 us; f32
// grad_q was slower with 4).
int at_row_blocks(int len) {
  const int nb = (len + 31) / 32;
  const int idle4 = (4 - nb % 4) % 4, idle2 = nb % 2;
  return idle2 < idle4 ? 2 : 4;
}

template <typename K>
int at_launch(K kernel, std::atomic<int> (&granted)[msda_host::kMaxDevices], const msda::AttnParams& p, int lds, int rb, hipStream_t st,
              const char* what) {
  const int rc = msda_host::allow_lds(kernel, lds, granted);
  if (rc != MSDA_OK) return rc;
  // (slice, head) pairs x chunks of rb row blocks of 32 (one per wave)
  const int64_t chunks = ((p.len + 31) / 32 + rb - 1) / rb;
  const int64_t grid = static_cast<int64_t>(p.batch) * p.groups * p.heads * chunks;
  if (grid >= (int64_t{1} << 31)) return fail(MSDA_ERR_UNSUPPORTED, "attention: too many workgroups");
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(64 * rb), lds, st, p);
  return msda_host::check_launch(what);
}

// The mask and dropout are template parameters: without them the kernels carry no per-score mask
// or hash code (and need fewer registers). Dropout runs in the MASK instantiations, whose mask
// pointer may then be null.
template <typename VT, int D, bool MASK, int RB, bool DROP = false>
int fwd_rb(const msda::AttnParams& p, hipStream_t st) {
  static std::atomic<int> granted[msda_host::kMaxDevices];
  return at_launch(msda::attn_fwd_kernel<VT, D, MASK, RB, DROP>, granted, p, lds_bytes(D), RB, st, "attention forward");
}

template <typename VT, int D, bool MASK, bool DROP = false>
int fwd_typed(const msda::AttnParams& p, hipStream_t st) {
  return fwd_rb<VT, D, MASK, 4, DROP>(p, st);
}

template <typename VT, int D, bool MASK, int RB, bool DROP = false>
int bwd_rb(const msda::AttnParams& p, bool want_kv, hipStream_t st) {
  int rc = MSDA_OK;
  {  // grad_q, and rowsum(dO * O) into the statistics for the key side (alone when grad_q is NULL)
    static std::atomic<int> granted[msda_host::kMaxDevices];
    if ((rc = at_launch(msda::attn_bwd_q_kernel<VT, D, MASK, RB, DROP>, granted, p, lds_bytes(D), RB, st,
                        "attention backward (queries)")) != MSDA_OK)
      return rc;
  }
  if (want_kv) {  // 4 key blocks per workgroup: with 2, the staging registers of the Q and dO chunks cost an occupancy step
    static std::atomic<int> granted[msda_host::kMaxDevices];
    rc = at_launch(msda::attn_bwd_kv_kernel<VT, D, MASK, 4, DROP>, granted, p, lds_bytes(D), 4, st, "attention backward (keys, values)");
  }
  return rc;
}

template <typename VT, int D, bool MASK, bool DROP = false>
int bwd_typed(const msda::AttnParams& p, bool want_kv, hipStream_t st) {
  return at_row_blocks(p.len) == 2 ? bwd_rb<VT, D, MASK, 2, DROP>(p, want_kv, st) : bwd_rb<VT, D, MASK, 4, DROP>(p, want_kv, st);
}

// bf16 inputs: the bf16-MFMA kernels
template <int D, bool MASK, int RB, bool DROP = false>
int fwd_b_rb(const msda::AttnParams& p, hipStream_t st) {
  static std::atomic<int> granted[msda_host::kMaxDevices];
  return at_launch(msda::attn_fwd_bf16_kernel<D, MASK, RB, DROP>, granted, p, lds_bf16(D, false), RB, st, "attention forward");
}

template <int D, bool MASK, bool DROP = false>
int fwd_b(const msda::AttnParams& p, hipStream_t st) {
  return fwd_b_rb<D, MASK, 4, DROP>(p, st);
}

// Every row of tensor t starts on a 16-byte boundary (base pointer and all four strides).
bool rows16(const void* base, const msda::AttnParams& p, int t) {
  return aligned_to(base, 16) && p.st[t][0] % 8 == 0 && p.st[t][1] % 8 == 0 && p.st[t][2] % 8 == 0 && p.st[t][3] % 8 == 0;
}

// The bf16 forward for head_dim 32 without a mask stages the whole key and value slice in LDS
// (MSDA_ATTN_FWD_D32=0 selects the chunked kernel).
bool use_fwd_d32(const msda::AttnParams& p, int d) {
  return d == 32 && p.mask == nullptr && p.len <= msda::kAtFwdD32MaxLen && rows16(p.k, p, msda::kAtK) && rows16(p.v, p, msda::kAtV) &&
         msda_host::knob("MSDA_ATTN_FWD_D32", 1) != 0;
}

// Four query blocks per workgroup (four workgroups of four waves fill a CU's LDS). Measured at
// 300 rows (10 blocks): five per workgroup, which idles no wave and stages a third less, took 44.8
// against 36 us at four waves per SIMD (three workgroups per CU), and 58.6 us at five (spills).
int fwd_d32(const msda::AttnParams& p, hipStream_t st) {
  static std::atomic<int> granted[msda_host::kMaxDevices];
  // dynamic: the key and value rows of chunks 1 .. (chunk 0 has static arrays)
  const int tiles = ((p.len + msda::kAtChunk - 1) / msda::kAtChunk - 1) * msda::kAtChunk * 32 * 2 * 2;
  return at_launch(msda::attn_fwd_bf16_d32_kernel<4>, granted, p, tiles, 4, st, "attention forward");
}

template <int D, bool MASK, int RB, bool DROP = false>
int bwd_b_rb(const msda::AttnParams& p, bool want_kv, hipStream_t st) {
  int rc = MSDA_OK;
  {
    static std::atomic<int> granted[msda_host::kMaxDevices];
    if ((rc = at_launch(msda::attn_bwd_q_bf16_kernel<D, MASK, RB, DROP>, granted, p, lds_bf16(D, false), RB, st,
                        "attention backward (queries)")) != MSDA_OK)
      return rc;
  }
  if (want_kv) {
    static std::atomic<int> granted[msda_host::kMaxDevices];
    rc = at_launch(msda::attn_bwd_kv_bf16_kernel<D, MASK, 4, DROP>, granted, p, lds_bf16(D, true), 4, st,
                   "attention backward (keys, values)");
  }
  return rc;
}

template <int D, bool MASK, bool DROP = false>
int bwd_b(const msda::AttnParams& p, bool want_kv, hipStream_t st) {
  return bwd_b_rb<D, MASK, 4, DROP>(p, want_kv, st);
}

// The fused backward: one workgroup per (slice, head), one wave per key block and two dQ waves.
template <typename K>
int bwd_fused_launch(K kernel, std::atomic<int> (&granted)[msda_host::kMaxDevices], const msda::AttnParams& p, int lds, hipStream_t st) {
  const int rc = msda_host::allow_lds(kernel, lds, granted);
  if (rc != MSDA_OK) return rc;
  const int64_t grid = static_cast<int64_t>(p.batch) * p.groups * p.heads;
  if (grid >= (int64_t{1} << 31)) return fail(MSDA_ERR_UNSUPPORTED, "attention: too many workgroups");
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(64 * ((p.len + 31) / 32 + 2)), lds, st, p);
  return msda_host::check_launch("attention backward (fused)");
}

int bwd_fused(const msda::AttnParams& p, bool bf16, hipStream_t st) {
  const int nb = (p.len + 31) / 32;
  if (bf16) {
    static std::atomic<int> granted[msda_host::kMaxDevices];
    return bwd_fused_launch(msda::attn_bwd_fused_bf16_kernel, granted, p, msda::at_fused_lds_bytes(nb), st);
  }
  static std::atomic<int> granted[msda_host::kMaxDevices];
  return bwd_fused_launch(msda::attn_bwd_fused_f32_kernel, granted, p, msda::at_fused_f32_lds_bytes(nb), st);
}

// The fused kernels serve head_dim 32 without a mask, with at most 32 kAtFusedBlocks rows, when
// grad_q and grad_k or grad_v are wanted (MSDA_ATTN_FUSED=0 selects the two kernels): they form
// S and dP once per block pair instead of once in each kernel.
bool use_fused(const msda::AttnParams& p, int d, bool want_kv) {
  return d == 32 && p.mask == nullptr && want_kv && p.gq != nullptr && p.len <= 32 * msda::kAtFusedBlocks &&
         msda_host::knob("MSDA_ATTN_FUSED", 1) != 0;
}

// Dropout (rate > 0) runs in the chunked kernels' MASK + DROP instantiations, neither the fused
// backward nor the staged bf16 forward.
int fwd_dispatch(const msda::AttnParams& p, int d, bool bf16, bool drop, hipStream_t st) {
  if (drop) {
    if (bf16) return d == 32 ? fwd_b<32, true, true>(p, st) : fwd_b<64, true, true>(p, st);
    return d == 32 ? fwd_typed<float, 32, true, true>(p, st) : fwd_typed<float, 64, true, true>(p, st);
  }
  const bool m = p.mask != nullptr;
  if (bf16) {
    if (use_fwd_d32(p, d)) return fwd_d32(p, st);
    if (d == 32) return m ? fwd_b<32, true>(p, st) : fwd_b<32, false>(p, st);
    return m ? fwd_b<64, true>(p, st) : fwd_b<64, false>(p, st);
  }
  if (d == 32) return m ? fwd_typed<float, 32, true>(p, st) : fwd_typed<float, 32, false>(p, st);
  return m ? fwd_typed<float, 64, true>(p, st) : fwd_typed<float, 64, false>(p, st);
}

int bwd_dispatch(const msda::AttnParams& p, int d, bool bf16, bool want_kv, bool drop, hipStream_t st) {
  if (drop) {
    if (bf16) return d == 32 ? bwd_b<32, true, true>(p, want_kv, st) : bwd_b<64, true, true>(p, want_kv, st);
    return d == 32 ? bwd_typed<float, 32, true, true>(p, want_kv, st) : bwd_typed<float, 64, true, true>(p, want_kv, st);
  }
  const bool m = p.mask != nullptr;
  if (use_fused(p, d, want_kv)) return bwd_fused(p, bf16, st);
  if (bf16) {
    if (d == 32) return m ? bwd_b<32, true>(p, want_kv, st) : bwd_b<32, false>(p, want_kv, st);
    return m ? bwd_b<64, true>(p, want_kv, st) : bwd_b<64, false>(p, want_kv, st);
  }
  if (d == 32) return m ? bwd_typed<float, 32, true>(p, want_kv, st) : bwd_typed<float, 32, false>(p, want_kv, st);
  return m ? bwd_typed<float, 64, true>(p, want_kv, st) : bwd_typed<float, 64, false>(p, want_kv, st);
}

// Dropout arguments: rate in [0, 1) (0: none), the call's seed. Fills p's dropout fields. The
// hash inputs (q << 16 | k / 2) are distinct for the at most 65536 rows the callers admit.
int at_dropout(msda::AttnParams* p, float rate, uint64_t seed) {
  if (!(rate >= 0.0f && rate < 1.0f)) return fail(MSDA_ERR_INVALID_ARGUMENT, "attention: dropout rate %g outside [0, 1)", static_cast<double>(rate));
  p->drop_seed[0] = static_cast<uint32_t>(seed);
  p->drop_seed[1] = static_cast<uint32_t>(seed >> 32);
  p->drop_thr = static_cast<uint32_t>(std::min(65536.0, std::nearbyint(static_cast<double>(rate) * 65536.0)));
  p->drop_scale = static_cast<float>(1.0 / (1.0 - static_cast<double>(rate)));
  return MSDA_OK;
}

int attention_fwd(const void* q, const void* k, const void* v, int dtype, void* out, float* stats, int batch, int groups, int heads,
                  int len, int head_dim, const int64_t* strides, const uint8_t* mask, float rate, uint64_t seed, void* stream) {
  msda_host::clear_error();
  int rc = at_validate(dtype, batch, groups, heads, len, head_dim, strides, 4);
  if (rc != MSDA_OK) return rc;
  static const int order[4] = {msda::kAtQ, msda::kAtK, msda::kAtV, msda::kAtO};
  msda::AttnParams p = at_params(dtype, batch, groups, heads, len, head_dim, strides, 4, order);
  if ((rc = at_dropout(&p, rate, seed)) != MSDA_OK) return rc;
  if (batch == 0 || groups == 0 || heads == 0 || len == 0) return MSDA_OK;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || stats == nullptr)
    return fail(MSDA_ERR_INVALID_ARGUMENT, "msda_attention_fwd: NULL tensor pointer");
  const size_t a = dtype == MSDA_DTYPE_BF16 ? 8 : 16;
  if (!aligned_to(q, a) || !aligned_to(k, a) || !aligned_to(v, a) || !aligned_to(out, a / 4) || !aligned_to(stats, 16))
    return fail(MSDA_ERR_INVALID_ARGUMENT, "attention: q, k, v must be aligned to 4 elements");
  p.q = q;
  p.k = k;
  p.v = v;
  p.out = out;
  p.stats = stats;
  p.mask = mask;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return fwd_dispatch(p, head_dim, dtype == MSDA_DTYPE_BF16, rate > 0.0f, st);
}

int attention_bwd(const void* q, const void* k, const void* v, const void* out, float* stats, const void* grad_out, int dtype,
                  void* grad_q, void* grad_k, void* grad_v, int batch, int groups, int heads, int len, int head_dim,
                  const int64_t* strides, const uint8_t* mask, float rate, uint64_t seed, void* stream) {
  msda_host::clear_error();
  int rc = at_validate(dtype, batch, groups, heads, len, head_dim, strides, 8);
  if (rc != MSDA_OK) return rc;
  static const int order[8] = {msda::kAtQ, msda::kAtK, msda::kAtV, msda::kAtO, msda::kAtGO, msda::kAtGQ, msda::kAtGK, msda::kAtGV};
  msda::AttnParams p = at_params(dtype, batch, groups, heads, len, head_dim, strides, 8, order);
  if ((rc = at_dropout(&p, rate, seed)) != MSDA_OK) return rc;
  const bool want_q = grad_q != nullptr, want_kv = grad_k != nullptr || grad_v != nullptr;
  if (batch == 0 || groups == 0 || heads == 0 || len == 0 || (!want_q && !want_kv)) return MSDA_OK;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || stats == nullptr || grad_out == nullptr)
    return fail(MSDA_ERR_INVALID_ARGUMENT, "msda_attention_bwd: NULL tensor pointer");
  const size_t a = dtype == MSDA_DTYPE_BF16 ? 8 : 16;
  if (!aligned_to(q, a) || !aligned_to(k, a) || !aligned_to(v, a) || !aligned_to(out, a) || !aligned_to(grad_out, a) ||
      !aligned_to(grad_q, a / 4) || !aligned_to(grad_k, a / 4) || !aligned_to(grad_v, a / 4) || !aligned_to(stats, 16))
    return fail(MSDA_ERR_INVALID_ARGUMENT, "attention: q, k, v, out, grad_out must be aligned to 4 elements");
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = out;
  p.go = grad_out;
  p.gq = grad_q;
  p.gk = grad_k;
  p.gv = grad_v;
  p.stats = stats;
  p.mask = mask;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return bwd_dispatch(p, head_dim, dtype == MSDA_DTYPE_BF16, want_kv, rate > 0.0f, st);
}

}  // namespace

extern "C" {

int msda_attention_fwd(const void* q, const void* k, const void* v, int dtype, void* out, float* stats, int batch, int groups, int heads,
                       int len, int head_dim, const int64_t* strides, const uint8_t* mask, void* stream) {
  return attention_fwd(q, k, v, dtype, out, stats, batch, groups, heads, len, head_dim, strides, mask, 0.0f, 0, stream);
}

int msda_attention_bwd(const void* q, const void* k, const void* v, const void* out, float* stats, const void* grad_out, int dtype,
                       void* grad_q, void* grad_k, void* grad_v, int batch, int groups, int heads, int len, int head_dim,
                       const int64_t* strides, const uint8_t* mask, void* stream) {
  return attention_bwd(q, k, v, out, stats, grad_out, dtype, grad_q, grad_k, grad_v, batch, groups, heads, len, head_dim, strides, mask,
                       0.0f, 0, stream);
}

int msda_attention_fwd_dropout(const void* q, const void* k, const void* v, int dtype, void* out, float* stats, int batch, int groups,
                               int heads, int len, int head_dim, const int64_t* strides, const uint8_t* mask, float rate, uint64_t seed,
                               void* stream) {
  return attention_fwd(q, k, v, dtype, out, stats, batch, groups, heads, len, head_dim, strides, mask, rate, seed, stream);
}

int msda_attention_bwd_dropout(const void* q, const void* k, const void* v, const void* out, float* stats, const void* grad_out, int dtype,
                               void* grad_q, void* grad_k, void* grad_v, int batch, int groups, int heads, int len, int head_dim,
                               const int64_t* strides, const uint8_t* mask, float rate, uint64_t seed, void* stream) {
  return attention_bwd(q, k, v, out, stats, grad_out, dtype, grad_q, grad_k, grad_v, batch, groups, heads, len, head_dim, strides, mask,
                       rate, seed, stream);
}

int msda_attention_dropout_keep(int batch, int groups, int heads, int len, float rate, uint64_t seed, uint8_t* keep, void* stream) {
  msda_host::clear_error();
  if (batch < 0 || groups < 0 || heads < 0 || len < 0) return fail(MSDA_ERR_INVALID_ARGUMENT, "attention: negative extent");
  if (static_cast<int64_t>(batch) * groups * heads >= (int64_t{1} << 31) || len > 65536)
    return fail(MSDA_ERR_UNSUPPORTED, "attention: too many slices or rows");
  msda::AttnParams p{};
  p.batch = batch;
  p.groups = groups;
  p.heads = heads;
  p.len = len;
  int rc = at_dropout(&p, rate, seed);
  if (rc != MSDA_OK) return rc;
  const int64_t pairs = static_cast<int64_t>(batch) * groups * heads * len * ((len + 1) / 2);
  if (pairs == 0) return MSDA_OK;
  if (keep == nullptr) return fail(MSDA_ERR_INVALID_ARGUMENT, "msda_attention_dropout_keep: NULL keep");
  const int grid = static_cast<int>(std::min<int64_t>((pairs + 255) / 256, 4096));
  hipLaunchKernelGGL(msda::attn_drop_keep_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), p, keep, pairs);
  return msda_host::check_launch("attention dropout keep mask");
}

}  // extern "C"

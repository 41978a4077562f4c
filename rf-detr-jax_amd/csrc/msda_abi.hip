// msda_abi.hip — C ABI (include/msda.h): argument validation, launch planning, kernel dispatch.
//
// Validation runs before any HIP call, so malformed calls fail with MSDA_ERR_INVALID_ARGUMENT /
// MSDA_ERR_UNSUPPORTED on any host (no GPU needed). Launch planning reads two device attributes
// (LDS per workgroup, CU count) once per device.
#include "msda.h"
#include "msda_kernels.h"
#include "msda_launch.h"
#include "msda_fused_bwd_kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>
#include <unordered_map>

namespace {
thread_local std::string g_last_error;
}  // namespace

namespace msda_host {

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

// The attribute is raised once per (instantiation, device) to the largest size requested so far,
// so steady-state launches (including ones under stream capture) make no extra runtime call.
int raise_lds_limit(const void* kernel, int bytes, std::atomic<int>* granted) {
  if (bytes <= 65536) return MSDA_OK;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return fail(MSDA_ERR_DEVICE, "hipGetDevice failed");
  if (granted[dev].load(std::memory_order_relaxed) >= bytes) return MSDA_OK;
  hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(MSDA_ERR_LAUNCH, "hipFuncSetAttribute(%d bytes LDS): %s", bytes, hipGetErrorString(e));
  }
  int cur = granted[dev].load(std::memory_order_relaxed);
  while (cur < bytes && !granted[dev].compare_exchange_weak(cur, bytes)) {
  }
  return MSDA_OK;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MSDA_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return MSDA_OK;
}

}  // namespace msda_host

namespace {

using msda_host::fail;
using msda_host::kMaxDevices;

// ------------------------------------------------------------------------------------------
// shape validation shared by forward and backward

struct Shape {
  int batch, heads, dim, queries, levels, points;
  int64_t len_value;
  int h[msda::kMaxLevels], w[msda::kMaxLevels];
  int64_t start[msda::kMaxLevels];
};

int validate(Shape* s, int batch, int heads, int dim, int queries, int levels, int points,
             const int32_t* spatial_shapes, const int32_t* level_start_index, int64_t len_value) {
  if (batch < 0 || queries < 0) return fail(MSDA_ERR_INVALID_ARGUMENT, "batch (%d) and len_query (%d) must be >= 0", batch, queries);
  if (heads < 1 || dim < 1 || points < 1) return fail(MSDA_ERR_INVALID_ARGUMENT, "n_heads (%d), head_dim (%d) and n_points (%d) must be >= 1", heads, dim, points);
  if (levels < 1 || levels > MSDA_MAX_LEVELS) return fail(MSDA_ERR_INVALID_ARGUMENT, "n_levels must be in [1, %d], got %d", MSDA_MAX_LEVELS, levels);
  if (spatial_shapes == nullptr) return fail(MSDA_ERR_INVALID_ARGUMENT, "spatial_shapes is NULL");
  int64_t acc = 0;
  for (int l = 0; l < levels; ++l) {
    const int hl = spatial_shapes[2 * l], wl = spatial_shapes[2 * l + 1];
    if (hl < 1 || wl < 1) return fail(MSDA_ERR_INVALID_ARGUMENT, "spatial_shapes[%d] = (%d, %d) must be positive", l, hl, wl);
    if (level_start_index != nullptr && level_start_index[l] != acc)
      return fail(MSDA_ERR_INVALID_ARGUMENT, "level_start_index[%d] = %d, expected %lld (prefix sum of H*W)", l,
                  level_start_index[l], static_cast<long long>(acc));
    s->h[l] = hl;
    s->w[l] = wl;
    s->start[l] = acc;
    acc += static_cast<int64_t>(hl) * wl;
  }
  if (acc != len_value) return fail(MSDA_ERR_INVALID_ARGUMENT, "len_value = %lld but sum(H*W) = %lld", static_cast<long long>(len_value), static_cast<long long>(acc));
  // Index arithmetic inside a slice is 32-bit.
  if (len_value * dim > (int64_t{1} << 30)) return fail(MSDA_ERR_UNSUPPORTED, "len_value * head_dim = %lld exceeds 2^30", static_cast<long long>(len_value * dim));
  if (static_cast<int64_t>(batch) * heads * 4096 > (int64_t{1} << 31)) return fail(MSDA_ERR_UNSUPPORTED, "batch * n_heads too large");
  if (static_cast<int64_t>(levels) * points > 4096) return fail(MSDA_ERR_UNSUPPORTED, "n_levels * n_points = %d exceeds 4096", levels * points);
  s->batch = batch;
  s->heads = heads;
  s->dim = dim;
  s->queries = queries;
  s->levels = levels;
  s->points = points;
  s->len_value = len_value;
  return MSDA_OK;
}

int check_dtype(int dt, const char* what) {
  if (dt != MSDA_DTYPE_F32 && dt != MSDA_DTYPE_BF16) return fail(MSDA_ERR_UNSUPPORTED, "%s: unsupported dtype code %d", what, dt);
  return MSDA_OK;
}

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Channels per lane (VEC): the largest power of two <= max_vec that divides head_dim and keeps
// every listed pointer aligned to min(VEC * element size, 16) bytes. max_vec = 16 gives one lane
// per query for head_dim 16 (the RF-DETR shape).
int pick_vec(int dim, int max_vec, std::initializer_list<std::pair<const void*, int>> ptrs) {
  auto fits = [&](int vec) {
    if (dim % vec != 0) return false;
    for (auto& pr : ptrs) {
      const size_t a = std::min<size_t>(static_cast<size_t>(vec) * pr.second, 16);
      if (pr.first != nullptr && !aligned(pr.first, a)) return false;
    }
    return true;
  };
  int vec = 16;
  while (vec > 1 && (vec > max_vec || !fits(vec))) vec >>= 1;
  return vec;
}

int lpq_shift_for(int dim, int vec) {
  const int lanes = (dim + vec - 1) / vec;
  int shift = 0;
  while ((1 << shift) < lanes) ++shift;
  return shift;
}

// ------------------------------------------------------------------------------------------
// per-device attributes (one-time, idempotent initialisation)

// The scratch of msda_bwd_noalloc: a file-scope device array (each GPU the library runs on holds
// its own copy until the process ends). Host code never uses the array's name as an address (on
// the host it is only a stand-in for the symbol): its device address is looked up with
// hipGetSymbolAddress once per device, with that device current, when the library first reads the
// device's attributes (the first call of any entry point on it; a caller that captures
// msda_bwd_noalloc into a graph has normally made a call before, outside the capture), and kept here.
// 16 MiB: the nano group-DETR backward (batch 8, 16 heads, one 24x24 level, 3900 queries) needs
// 9.4 MiB of partial sums; query blocks exist only while the grid is short of one resident wave of
// workgroups, so most shapes need less or none. Shapes that need more are refused.
constexpr int64_t kNoAllocScratchBytes = int64_t{16} << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
std::atomic<void*> g_scratch_ptr[kMaxDevices];

int resolve_scratch(int dev) {
  if (g_scratch_ptr[dev].load(std::memory_order_acquire) != nullptr) return MSDA_OK;
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr) {
    (void)hipGetLastError();
    return fail(MSDA_ERR_DEVICE, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
  }
  g_scratch_ptr[dev].store(ptr, std::memory_order_release);
  return MSDA_OK;
}

int noalloc_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MSDA_ERR_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(MSDA_ERR_DEVICE, "device index %d out of range", dev);
  const int rc = resolve_scratch(dev);  // normally done already by device_info
  if (rc != MSDA_OK) return rc;
  *out = g_scratch_ptr[dev].load(std::memory_order_acquire);
  return MSDA_OK;
}

struct DevInfo {
  int lds_bytes;
  int cus;
};

std::atomic<int> g_dev_lds[kMaxDevices];
std::atomic<int> g_dev_cus[kMaxDevices];

int device_info(DevInfo* info) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MSDA_ERR_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(MSDA_ERR_DEVICE, "device index %d out of range", dev);
  int lds = g_dev_lds[dev].load(std::memory_order_relaxed);
  int cus = g_dev_cus[dev].load(std::memory_order_relaxed);
  if (lds <= 0 || cus <= 0) {
    e = hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e != hipSuccess) return fail(MSDA_ERR_DEVICE, "hipDeviceGetAttribute(LDS): %s", hipGetErrorString(e));
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return fail(MSDA_ERR_DEVICE, "hipDeviceGetAttribute(CUs): %s", hipGetErrorString(e));
    // msda_bwd_noalloc's scratch address (a failure is reported by that entry point)
    if (resolve_scratch(dev) != MSDA_OK) g_last_error.clear();
    g_dev_lds[dev].store(lds, std::memory_order_relaxed);
    g_dev_cus[dev].store(cus, std::memory_order_relaxed);
  }
  info->lds_bytes = lds;
  info->cus = cus;
  return MSDA_OK;
}

// Tuning knobs (MSDA_* names): launch-shape choices. With every knob at its default the plans and
// the backward's workspace size depend on the shape and the device only; the knobs that opt into
// the sorted-gather backward (MSDA_BWD_GATHER*) or force banded plans (MSDA_BWD_FORCE_BANDS) change
// the size the query returns, so a caller that sets them queries the size afterwards. Each is read
// from the environment once, at its first use, and msda_set_tuning() overrides it for the rest of
// the process, so a plan does not change between calls unless asked to.
std::mutex g_knob_mu;
std::unordered_map<std::string, std::pair<bool, int>> g_knob_env;  // name -> (set, value)
std::unordered_map<std::string, std::pair<bool, int>> g_knob_set;  // msda_set_tuning overrides

int env_int(const char* name, int dflt) {
  std::lock_guard<std::mutex> lock(g_knob_mu);
  auto o = g_knob_set.find(name);
  if (o != g_knob_set.end()) return o->second.first ? o->second.second : dflt;
  auto it = g_knob_env.find(name);
  if (it == g_knob_env.end()) {
    const char* v = std::getenv(name);
    const bool set = v != nullptr && *v != 0;
    it = g_knob_env.emplace(name, std::make_pair(set, set ? std::atoi(v) : 0)).first;
  }
  return it->second.first ? it->second.second : dflt;
}

inline int align16(int64_t x) { return static_cast<int>((x + 15) & ~int64_t{15}); }

// Samples per (query, head) = levels * points. Up to four, the count is a compile-time bound of
// the kernel, which then loads several queries' inputs at once; beyond that a query's samples are
// processed in chunks.
inline int samples_bound(int levels, int points) {
  const int lp = levels * points;
  return lp <= 2 ? 2 : lp <= 4 ? 4 : 0;
}

msda::LevelDesc level_desc(const Shape& s, int l, int lds, int band_rows, int band_first) {
  msda::LevelDesc d{};
  d.h = s.h[l];
  d.w = s.w[l];
  d.fh = static_cast<float>(s.h[l]);
  d.fw = static_cast<float>(s.w[l]);
  d.small = static_cast<int64_t>(s.h[l]) * s.w[l] * s.dim < (int64_t{1} << 24) ? 1 : 0;
  d.start = static_cast<int>(s.start[l]);
  d.lds = lds;
  d.band_rows = band_rows;
  d.band_first = band_first;
  return d;
}

// The reference sampler a level reproduces (msda_fwd_sampler, msda_bwd_sampler): the forward's bf16
// rounding points and the Pallas kernel's pixel coordinates (enum msda_sampler in msda.h).
int check_sampler(int sampler) {
  if (sampler < MSDA_SAMPLER_HIP || sampler > MSDA_SAMPLER_PALLAS) return fail(MSDA_ERR_INVALID_ARGUMENT, "unknown sampler code %d", sampler);
  return MSDA_OK;
}

void apply_sampler(const Shape& s, int sampler, int value_dtype, msda::LevelDesc* lv) {
  const bool bf16 = value_dtype == MSDA_DTYPE_BF16;
  for (int l = 0; l < s.levels; ++l) {
    int sm = sampler;
    if (sm == MSDA_SAMPLER_AUTO)  // ops.py:277-279 with _MATMUL_SAMPLER_MAX_LEVEL = 4096 (ops.py:42)
      sm = static_cast<int64_t>(s.h[l]) * s.w[l] <= 4096 ? MSDA_SAMPLER_MATMUL : MSDA_SAMPLER_GATHER;
    lv[l].pallas_xy = sm == MSDA_SAMPLER_PALLAS ? 1 : 0;
    lv[l].rmode = !bf16                             ? msda::kRoundNone
                  : sm == MSDA_SAMPLER_GATHER       ? msda::kRoundGather
                  : sm == MSDA_SAMPLER_GATHER_F32   ? msda::kRoundGatherF32
                  : sm == MSDA_SAMPLER_MATMUL       ? msda::kRoundMatmul
                                                    : msda::kRoundNone;
  }
}

// ------------------------------------------------------------------------------------------
// planning of the forward kernel

struct SamplePlan {
  int grid, threads, lds;
};

// Each level whose slice still fits one head's LDS budget is staged (packed in level order); the
// rest are gathered through L2. Head groups: a workgroup serves `hg` heads of one batch entry, so
// the lanes of one query touch contiguous runs of its [H, ...] rows; hg is the largest power of
// two <= the cap that divides n_heads and keeps the group's slices within the LDS. The cap is 4
// for slices of 1024 queries or more and 1 below: with few queries per slice, one head per
// workgroup spreads the staging over more CUs and lets more workgroups share one (measured on
// MI355X, forward: config 0 3.7 against 5.3 us, config 1 5.6 against 6.0, config 3 10.1 against
// 10.5, config 4 15.3 against 16.7), while at 3900 queries four heads per workgroup fetch the
// location and weight rows and write the output rows as whole runs (14.2 against 17.0 us). A
// workgroup that fills a CU's LDS gets 1024 threads. Then one resident wave of workgroups: fewer,
// longer workgroups amortise the value staging.
int plan_sample(const Shape& s, int vbytes, const DevInfo& dev, const char* prefix, int shift, msda::SampleParams* p,
                SamplePlan* out, int hg_max = 1 << 30) {
  auto knob = [&](const char* name, int dflt) {
    std::string key = std::string(prefix) + name;
    return env_int(key.c_str(), dflt);
  };
  const int budget = std::min(dev.lds_bytes, knob("_LDS_BUDGET", dev.lds_bytes));
  int head_lds = 0;  // elements
  bool all_staged = true;
  for (int l = 0; l < s.levels; ++l) {
    const int64_t bytes = static_cast<int64_t>(s.h[l]) * s.w[l] * s.dim * vbytes;
    p->lv[l] = level_desc(s, l, -1, 0, 0);
    if (static_cast<int64_t>(head_lds) * vbytes + bytes <= budget) {
      p->lv[l].lds = head_lds;
      head_lds += static_cast<int>(bytes / vbytes);
    } else {
      all_staged = false;
    }
  }
  const int64_t head_bytes = align16(static_cast<int64_t>(head_lds) * vbytes);
  int hg = 1;
  const int hg_cap = std::min(hg_max, std::max(1, knob("_HEADS", s.queries >= 1024 ? 4 : 1)));
  const int group_budget = std::min(budget, knob("_GROUP_LDS", dev.lds_bytes));
  while (hg * 2 <= hg_cap && s.heads % (hg * 2) == 0 && (hg * 2) * head_bytes <= group_budget) hg *= 2;
  // With every level staged a head's region is its whole value slice; regions stay 16-byte aligned.
  const int head_stride = all_staged ? static_cast<int>(s.len_value * s.dim) : static_cast<int>(head_bytes / vbytes);
  p->head_lds = head_stride;
  p->all_staged = all_staged ? 1 : 0;
  p->hg = hg;
  p->lpq_shift = shift;
  const int lds = align16(static_cast<int64_t>(hg) * head_stride * vbytes);
  if (all_staged && (static_cast<int64_t>(s.len_value) * s.dim * vbytes) % 16 != 0) p->vec16 = 0;

  const int per_cu = lds > 0 ? std::max(1, dev.lds_bytes / lds) : 8;
  int threads = knob("_THREADS", per_cu >= 4 ? 256 : per_cu >= 2 ? 512 : 1024);
  threads = std::max(64, std::min(msda::kSampleMaxThreads, (threads / 64) * 64));
  const int tpq = hg << shift;  // threads per query
  if (tpq > threads) threads = std::min(msda::kSampleMaxThreads, ((tpq + 63) / 64) * 64);
  if (tpq > threads) return fail(MSDA_ERR_UNSUPPORTED, "head group of %d heads x %d lanes exceeds a workgroup", hg, 1 << shift);
  const int qpp = threads / tpq;
  const int64_t units = static_cast<int64_t>(s.batch) * (s.heads / hg);
  const int target = knob("_TARGET_WGS", dev.cus * std::min(per_cu, 8));
  const int max_blocks = std::max(1, (s.queries + qpp - 1) / qpp);
  {
    const int nqb = static_cast<int>(std::min<int64_t>(max_blocks, std::max<int64_t>(1, (target + units - 1) / units)));
    const int per = (s.queries + nqb - 1) / nqb;
    p->qblock = std::max(qpp, ((per + qpp - 1) / qpp) * qpp);
  }
  p->nqb = std::max(1, (s.queries + p->qblock - 1) / p->qblock);
  const int64_t grid = units * p->nqb;
  if (grid > 0x7fffffff) return fail(MSDA_ERR_UNSUPPORTED, "grid too large");
  out->grid = static_cast<int>(grid);
  out->threads = threads;
  out->lds = align16(lds);
  if (out->lds > dev.lds_bytes) return fail(MSDA_ERR_UNSUPPORTED, "forward needs %d bytes of LDS", out->lds);
  return MSDA_OK;
}

// 16-byte staging / flushing is allowed when every level's rows start and end on 16 bytes.
bool rows_16b(const Shape& s, int vbytes, const void* a, const void* b) {
  if (!aligned(a, 16) || (b != nullptr && !aligned(b, 16))) return false;
  if ((s.len_value * s.dim * vbytes) % 16 != 0) return false;
  for (int l = 0; l < s.levels; ++l) {
    if ((s.start[l] * s.dim * vbytes) % 16 != 0) return false;
    if ((static_cast<int64_t>(s.w[l]) * s.dim * vbytes) % 16 != 0) return false;
  }
  return true;
}


// ------------------------------------------------------------------------------------------
// planning of the backward kernel (bwd_band_kernel)

// LDS of one workgroup of the backward kernel for a band of `rows` rows of a level `w` wide: the
// staged value rows (the band and one halo row), the f64 accumulator of the band, the list of the
// pass's points (`cap` 32-bit entries) and its counter, and the two grad_output row buffers (`gbuf`
// bytes each).
struct BandLayout {
  int acc, list, cnt, gbuf, total;
};

BandLayout band_layout(int rows, int w, int dim, int vbytes, int cap, int gbuf) {
  BandLayout b;
  const int64_t row = static_cast<int64_t>(w) * dim;
  int64_t o = align16(row * (rows + 1) * vbytes);
  b.acc = static_cast<int>(o);
  o += align16((row * rows + 2 * dim) * 8);  // the band's cells and a guard cell on each side
  b.list = static_cast<int>(o);
  o += align16(static_cast<int64_t>(cap) * 4);
  b.cnt = static_cast<int>(o);
  o += 16;
  b.gbuf = gbuf > 0 ? static_cast<int>(o) : -1;
  o += 2 * static_cast<int64_t>(gbuf);
  b.total = o > (int64_t{1} << 30) ? (1 << 30) : static_cast<int>(o);
  return b;
}

struct BandPlan {
  int ch, lps_shift, threads, qpass, cap, lds, nwork;
  int nqb, qblock;  // query blocks per (slice, item); nqb > 1 needs the partial-sum workspace
  int rows[msda::kMaxLevels], bands[msda::kMaxLevels];
  BandLayout layout;  // every workgroup gets the largest level's layout
};

// Bytes of the backward's workspace for a plan: the query blocks' partial grad_value sums.
// f32 partial sums of one query block: every grad_value element, rounded up to whole quads
int64_t part_block_stride(const Shape& s) { return (static_cast<int64_t>(s.batch) * s.heads * s.len_value * s.dim + 3) / 4 * 4; }

int64_t band_workspace(const Shape& s, const BandPlan& bp) {
  return bp.nqb > 1 ? static_cast<int64_t>(bp.nqb) * part_block_stride(s) * 4 : 0;
}

// The second kernel of a split backward: grad_value = sum of the blocks' partials, in block order;
// with rpart, also the fused backward's reference-point gradient (the heads' partials in order).
int launch_partial_sums(const Shape& s, int value_dtype, const float* part, int nqb, void* grad_value, const DevInfo& dev,
                        hipStream_t st, const float* rpart = nullptr, float* dref = nullptr, int ref_dim = 0) {
  const int64_t n = static_cast<int64_t>(s.batch) * s.heads * s.len_value * s.dim;
  const int64_t quads = n / 4;
  // a resident wave of workgroups, each thread four quads per pass
  const int64_t per_wg = std::max(64, env_int("MSDA_PART_SUM_QUADS", 256));
  const int grid = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>((quads + per_wg - 1) / per_wg, static_cast<int64_t>(dev.cus) * 8)));
  const int vec = aligned(grad_value, value_dtype == MSDA_DTYPE_BF16 ? 8 : 16) ? 1 : 0;
  const int64_t stride = part_block_stride(s);
  const int64_t nref = static_cast<int64_t>(s.batch) * s.queries * ref_dim;
  return value_dtype == MSDA_DTYPE_BF16
             ? msda_host::launch_part_sum<msda::bf16_t>(part, nqb, n, stride, grad_value, vec, grid, st, rpart, dref, s.heads, nref)
             : msda_host::launch_part_sum<float>(part, nqb, n, stride, grad_value, vec, grid, st, rpart, dref, s.heads, nref);
}

// Two kinds of plan.
// * Every level fits the LDS whole (its value rows and f64 accumulator): one band per level, and the
//   slice's queries are split into blocks until the grid fills the CUs (as many workgroups per CU as
//   the LDS holds). Blocks write partial grad_value sums that a second kernel adds in block order.
//   This depends on the shape and the device only (so does the workspace size).
// * Otherwise every level is cut into bands of whole image rows that fit the LDS share of `per_cu`
//   workgroups per CU; then bands are added, to the level with the fewest (each level holds the same
//   number of samples, Q * P per slice), until the grid has `per_cu` workgroups per CU. Each band
//   scans its level's locations and lists the points whose corner rows meet it (the points of at
//   most `qpass` queries per pass).
// Workgroup size: up to 1024 threads per CU in all (the kernel's register budget allows 16 waves).
int plan_band(const Shape& s, int vbytes, int ch, const DevInfo& dev, BandPlan* bp) {
  bp->ch = ch;
  bp->lps_shift = lpq_shift_for(s.dim, ch);
  const int lps = 1 << bp->lps_shift;
  const int64_t N = static_cast<int64_t>(s.batch) * s.heads;
  // whole levels
  int whole_lds = 0;
  bool all_whole = true;
  for (int l = 0; l < s.levels; ++l) {
    const BandLayout lay = band_layout(s.h[l], s.w[l], s.dim, vbytes, 0, 0);
    whole_lds = std::max(whole_lds, lay.total);
    if (lay.total > dev.lds_bytes) all_whole = false;
  }
  int per_cu;
  if (all_whole && env_int("MSDA_BWD_FORCE_BANDS", 0) == 0) {
    per_cu = std::max(1, dev.lds_bytes / whole_lds);
    bp->cap = 0;
    bp->qpass = std::max(1, s.queries);
    for (int l = 0; l < s.levels; ++l) bp->bands[l] = 1;
    const int64_t units = N * s.levels;
    int nqb = static_cast<int>(std::max<int64_t>(1, (static_cast<int64_t>(per_cu) * dev.cus + units - 1) / units));
    nqb = std::min(nqb, std::max(1, s.queries / 256));  // blocks of at least 256 queries
    bp->nqb = std::max(1, nqb);
  } else {
    // one workgroup per CU: measured faster than two at the two-level shape (47.9 vs 53.7 us), its
    // fixed phases (staging, scan, barriers, write-out) amortised over bands twice as tall
    per_cu = std::max(1, env_int("MSDA_BWD_WGS_PER_CU", 1));
    bp->nqb = 1;
    // the point list: one 32-bit entry per point of a pass (query offset << 16 | point)
    if (s.points >= 65536) return fail(MSDA_ERR_UNSUPPORTED, "n_points %d: at most 65535 with banded levels", s.points);
    const int max_cap = std::max(64, std::min(8192, env_int("MSDA_BWD_LIST", 8192)));
    bp->qpass = std::max(1, std::min(s.queries, std::max(1, max_cap / s.points)));
    // A level whose single image row would not fit beside a full list gets a shorter list (more
    // scan passes per band) rather than a refusal; shapes that fit keep the full list.
    for (;;) {
      bool fits = true;
      for (int l = 0; l < s.levels; ++l)
        if (band_layout(1, s.w[l], s.dim, vbytes, bp->qpass * s.points, 0).total > dev.lds_bytes) fits = false;
      if (fits || bp->qpass == 1) break;
      bp->qpass = (bp->qpass + 1) / 2;
    }
    bp->cap = bp->qpass * s.points;
    const int budget = dev.lds_bytes / per_cu - 512;
    int64_t nb_total = 0;
    for (int l = 0; l < s.levels; ++l) {
      int rows = s.h[l];
      while (rows > 1 && band_layout(rows, s.w[l], s.dim, vbytes, bp->cap, 0).total > budget) --rows;
      if (band_layout(rows, s.w[l], s.dim, vbytes, bp->cap, 0).total > dev.lds_bytes)
        return fail(MSDA_ERR_UNSUPPORTED, "level %d (width %d, head_dim %d) does not fit in LDS", l, s.w[l], s.dim);
      bp->bands[l] = (s.h[l] + rows - 1) / rows;
      nb_total += bp->bands[l];
    }
    const int forced = env_int("MSDA_BWD_BANDS", 0);
    const int64_t target = std::max(1, env_int("MSDA_BWD_TARGET_WGS", per_cu * dev.cus));
    if (forced > 0) {
      for (int l = 0; l < s.levels; ++l) bp->bands[l] = std::max(bp->bands[l], std::min(forced, s.h[l]));
    } else {
      while (N * nb_total < target) {
        int best = -1;
        for (int l = 0; l < s.levels; ++l)
          if (bp->bands[l] < s.h[l] && (best < 0 || bp->bands[l] < bp->bands[best])) best = l;
        if (best < 0) break;
        ++bp->bands[best];
        ++nb_total;
      }
    }
  }
  bp->qblock = std::max(1, (s.queries + bp->nqb - 1) / bp->nqb);
  // Enough threads for one pass over the block's queries, in whole groups of four waves (one per
  // SIMD; config 3: 768 rather than 640 threads, 38.2 against 39.1 us).
  int threads = env_int("MSDA_BWD_THREADS", 0);
  if (threads <= 0) threads = std::min(1024 / per_cu, std::max(256, ((std::min(s.queries, bp->qblock) * lps + 255) / 256) * 256));
  threads = std::max(64, std::min(msda::kBandMaxThreads, (threads / 64) * 64));
  if (lps > threads) return fail(MSDA_ERR_UNSUPPORTED, "head_dim %d too large", s.dim);
  bp->threads = threads;
  // one layout for all levels: the list after the largest value and accumulator regions
  int vmax = 0, amax = 0;
  bp->nwork = 0;
  for (int l = 0; l < s.levels; ++l) {
    bp->rows[l] = (s.h[l] + bp->bands[l] - 1) / bp->bands[l];
    bp->bands[l] = (s.h[l] + bp->rows[l] - 1) / bp->rows[l];
    bp->nwork += bp->bands[l];
    const int64_t row = static_cast<int64_t>(s.w[l]) * s.dim;
    vmax = std::max(vmax, align16(row * std::min(bp->rows[l] + 1, s.h[l]) * vbytes));
    amax = std::max(amax, align16((row * bp->rows[l] + 2 * s.dim) * 8));
  }
  bp->layout.acc = vmax;
  bp->layout.list = vmax + amax;
  bp->layout.cnt = bp->layout.list + align16(static_cast<int64_t>(bp->cap) * 4);
  bp->layout.gbuf = -1;
  bp->layout.total = bp->layout.cnt + 16;
  bp->lds = bp->layout.total;
  if (bp->lds > dev.lds_bytes) return fail(MSDA_ERR_UNSUPPORTED, "backward needs %d bytes of LDS", bp->lds);
  if (N * bp->nwork * bp->nqb > 0x7fffffff) return fail(MSDA_ERR_UNSUPPORTED, "backward grid too large");
  return MSDA_OK;
}

// The MSDeformAttn prologue and epilogue inside the band kernel (one whole level): `loc` / `attn`
// are then the sampling offsets and attention logits, `grad_loc` / `grad_attn` their gradients.
struct BandFusedArgs {
  const float* ref;
  int ref_dim;
  float inv_points, fpoints;
  float* dref_part;  // [H][B * Q][ref_dim] per-head partials (workspace), or null
  float* dref;       // grad_reference_points: the partials summed over heads, or null
};

int bwd_band_impl(const Shape& s, int ch, const void* value, int value_dtype, const float* loc, const float* attn,
                  const void* grad_output, int grad_output_dtype, void* grad_value, float* grad_loc, float* grad_attn, void* workspace,
                  int64_t workspace_bytes, const DevInfo& dev, hipStream_t st, const BandFusedArgs* fa = nullptr,
                  int sampler = MSDA_SAMPLER_HIP) {
  const int vbytes = value_dtype == MSDA_DTYPE_BF16 ? 2 : 4;
  BandPlan bp;
  int rc = plan_band(s, vbytes, ch, dev, &bp);
  if (rc != MSDA_OK) return rc;
  const bool partial = bp.nqb > 1 && grad_value != nullptr;
  if (partial) {
    const int64_t need = band_workspace(s, bp);
    if (workspace == nullptr || workspace_bytes < need)
      return fail(MSDA_ERR_INVALID_ARGUMENT, "workspace of %lld bytes needed, got %lld (see the workspace size query)",
                  static_cast<long long>(need), static_cast<long long>(workspace == nullptr ? 0 : workspace_bytes));
    if (!aligned(workspace, 16)) return fail(MSDA_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  }
  msda::BandParams p{};
  p.value = value;
  p.loc = loc;
  p.attn = attn;
  p.gout = grad_output;
  p.gout_bf16 = grad_output_dtype == MSDA_DTYPE_BF16;
  p.dvalue = grad_value;
  p.dloc = grad_loc;
  p.dattn = grad_attn;
  p.heads = s.heads;
  p.dim = s.dim;
  p.queries = s.queries;
  p.levels = s.levels;
  p.points = s.points;
  p.len_value = s.len_value;
  p.nwork = bp.nwork;
  p.nqb = bp.nqb;
  p.qblock = bp.qblock;
  p.part = partial ? static_cast<float*>(workspace) : nullptr;
  p.part_stride = part_block_stride(s);
  p.qpass = bp.qpass;
  p.lps_shift = bp.lps_shift;
  p.vec16 = rows_16b(s, vbytes, value, grad_value) ? 1 : 0;
  p.lds_acc = bp.layout.acc + s.dim * 8;  // after the leading guard cell
  // Whole levels whose block gives the waves fewer than two chunks of queries each: one item per
  // point (with one per query, waves get one chunk of queries or none, and the phase lasts a whole
  // chunk's chain of points).
  p.point_items = (fa == nullptr && static_cast<int64_t>(bp.qblock) * (1 << bp.lps_shift) < 2 * static_cast<int64_t>(bp.threads) &&
                   env_int("MSDA_BWD_POINT_ITEMS", 1) != 0)
                      ? 1
                      : 0;
  p.lds_list = bp.layout.list;
  p.lds_cnt = bp.layout.cnt;
  int first = 0;
  for (int l = 0; l < s.levels; ++l) {
    p.lv[l] = level_desc(s, l, 0, bp.rows[l], first);
    first += bp.bands[l];
  }
  apply_sampler(s, sampler, value_dtype, p.lv);
  const int grid = static_cast<int>(static_cast<int64_t>(s.batch) * s.heads * bp.nwork * p.nqb);
  if (fa != nullptr) {
    p.ref = fa->ref;
    p.ref_dim = fa->ref_dim;
    p.inv_points = fa->inv_points;
    p.fpoints = fa->fpoints;
    p.dref_part = fa->dref_part;
    p.bq_total = static_cast<int64_t>(s.batch) * s.queries;
  }
  rc = value_dtype == MSDA_DTYPE_BF16 ? msda_host::dispatch_bwd_band<msda::bf16_t>(ch, p, grid, bp.threads, bp.lds, st, fa != nullptr)
                                      : msda_host::dispatch_bwd_band<float>(ch, p, grid, bp.threads, bp.lds, st, fa != nullptr);
  if (rc != MSDA_OK) return rc;
  const bool ref_sum = fa != nullptr && fa->dref_part != nullptr && fa->dref != nullptr;
  if (partial)
    return launch_partial_sums(s, value_dtype, p.part, p.nqb, grad_value, dev, st, ref_sum ? fa->dref_part : nullptr,
                               ref_sum ? fa->dref : nullptr, ref_sum ? fa->ref_dim : 0);
  if (!ref_sum) return MSDA_OK;
  const int64_t nref = static_cast<int64_t>(s.batch) * s.queries * fa->ref_dim;
  const int rgrid = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>((nref + 255) / 256, static_cast<int64_t>(dev.cus) * 4)));
  hipLaunchKernelGGL(msda::ref_head_sum_kernel, dim3(rgrid), dim3(256), 0, st, fa->dref_part, fa->dref, s.heads, nref);
  return msda_host::check_launch("msda fused backward (reference points)");
}

// ------------------------------------------------------------------------------------------
// planning of the sorted-gather backward (bwd_gather_kernel)

struct GatherPlan {
  int threads, qblock, nqb, lds;
  int g, wt, key, cnt, scan, val;  // LDS byte offsets (val -1: value rows read from global memory)
};

// LDS of a workgroup holding `qb` queries with `nt` threads: grad_output rows in f32 (the area also
// holds one partial row per thread after the gather), a weight / dot slot per (sample, corner),
// the sorted entries (u16, padded to whole rows of `nt`), the cell counters of the largest level
// plus one, one scan slot per wave, and optionally the largest level's value rows.
void gather_layout(const Shape& s, int qb, int nt, int vbytes, bool stage, GatherPlan* gp) {
  int cmax = 0;
  for (int l = 0; l < s.levels; ++l) cmax = std::max(cmax, s.h[l] * s.w[l]);
  const int64_t ns = static_cast<int64_t>(qb) * s.points;
  int64_t o = 0;
  gp->g = 0;
  o += align16(static_cast<int64_t>(std::max(qb, nt)) * (s.dim + 4) * 4);  // rows padded by 16 bytes
  gp->wt = static_cast<int>(o);
  o += align16(ns * 16);
  gp->key = static_cast<int>(o);
  o += align16((ns * 4 + nt) * 2);
  gp->cnt = static_cast<int>(o);
  o += align16((static_cast<int64_t>(cmax) + 1) * 4);
  gp->scan = static_cast<int>(o);
  o += 64;
  gp->val = -1;
  if (stage) {
    gp->val = static_cast<int>(o);
    o += align16(static_cast<int64_t>(cmax) * s.dim * vbytes);
  }
  gp->lds = o > (int64_t{1} << 30) ? (1 << 30) : static_cast<int>(o);
}

int gather_threads(int qb, int points, int max_threads) {
  // every thread holds at most kGatherSpt samples through the sort; about 12 entries per thread
  const int64_t ns = static_cast<int64_t>(qb) * points;
  const int64_t need = (ns + msda::kGatherSpt - 1) / msda::kGatherSpt;
  const int64_t want = (ns * 4 + 11) / 12;
  int64_t t = std::max(need, std::min<int64_t>(want, max_threads));
  t = std::max<int64_t>(64, ((t + 63) / 64) * 64);
  const int forced = env_int("MSDA_BWD_GATHER_THREADS", 0);
  if (forced > 0) t = std::max<int64_t>(t, ((forced + 63) / 64) * 64);
  return static_cast<int>(std::min<int64_t>(t, max_threads));
}

// Whether the sorted gather takes this shape: head_dim 16 or 32, every level under 2^15 cells,
// and at least one query block that fits the LDS.
bool gather_eligible(const Shape& s) {
  // off by default: measured on MI355X slower than the band kernel at every benchmarked shape
  // (one workgroup per CU, so its barrier-separated phases do not overlap; nano_groupdetr
  // config: 73 us against 37 us)
  if (env_int("MSDA_BWD_GATHER", 0) == 0) return false;
  if (s.dim != 16 && s.dim != 32) return false;
  for (int l = 0; l < s.levels; ++l)
    if (static_cast<int64_t>(s.h[l]) * s.w[l] >= (int64_t{1} << msda::kGatherCellBits)) return false;
  return true;
}

// Query blocks: as many queries per workgroup as `per_cu` workgroups per CU leave LDS for (and the
// threads can hold), then more blocks while the grid has fewer workgroups than per_cu * CUs. Blocks
// of one (slice, level) write f32 partial rows that a second kernel adds.
int plan_gather_with(const Shape& s, int vbytes, const DevInfo& dev, bool stage, GatherPlan* gp) {
  const int max_threads = s.dim == 16 ? 1024 : 512;
  const int per_cu = std::max(1, env_int("MSDA_BWD_GATHER_WGS_PER_CU", 1));
  const int budget = dev.lds_bytes / per_cu;
  auto fits = [&](int qb) {
    GatherPlan t;
    gather_layout(s, qb, gather_threads(qb, s.points, max_threads), vbytes, stage, &t);
    return t.lds <= budget && static_cast<int64_t>(qb) * s.points <= static_cast<int64_t>(max_threads) * msda::kGatherSpt &&
           static_cast<int64_t>(qb) * s.points * 4 < 65536;
  };
  int qmax = std::min(s.queries, max_threads * msda::kGatherSpt / std::max(1, s.points));
  while (qmax > 1 && !fits(qmax)) qmax = std::max(1, qmax * 15 / 16);
  if (!fits(qmax)) return fail(MSDA_ERR_UNSUPPORTED, "sorted-gather backward does not fit in LDS");
  const int64_t units = static_cast<int64_t>(s.batch) * s.heads * s.levels;
  int nqb = (s.queries + qmax - 1) / qmax;
  const int forced = env_int("MSDA_BWD_GATHER_QB", 0);
  if (forced > 0) {
    nqb = std::max(nqb, (s.queries + forced - 1) / forced);
  } else {
    const int64_t target = static_cast<int64_t>(per_cu) * dev.cus;
    while (units * nqb < target && (s.queries + nqb) / (nqb + 1) >= 64) ++nqb;
  }
  gp->nqb = nqb;
  gp->qblock = (s.queries + nqb - 1) / nqb;
  gp->threads = gather_threads(gp->qblock, s.points, max_threads);
  gather_layout(s, gp->qblock, gp->threads, vbytes, stage, gp);
  if (gp->lds > dev.lds_bytes) return fail(MSDA_ERR_UNSUPPORTED, "sorted-gather backward needs %d bytes of LDS", gp->lds);
  if (units * nqb > 0x7fffffff) return fail(MSDA_ERR_UNSUPPORTED, "backward grid too large");
  return MSDA_OK;
}

bool gather_aligned(const void* value, const void* grad_value, const void* grad_output, int gbytes) {
  return aligned(value, 16) && aligned(grad_value, 16) && aligned(grad_output, 4 * static_cast<size_t>(gbytes));
}

// The level's value rows are staged in LDS (the corner dots then read LDS instead of L2) when that
// costs at most one more query block than reading them from global memory.
int plan_gather(const Shape& s, int vbytes, const DevInfo& dev, GatherPlan* gp) {
  const int stage = env_int("MSDA_BWD_GATHER_STAGE", -1);
  if (stage >= 0) return plan_gather_with(s, vbytes, dev, stage != 0, gp);
  int rc = plan_gather_with(s, vbytes, dev, false, gp);
  if (rc != MSDA_OK) return rc;
  GatherPlan st;
  if (plan_gather_with(s, vbytes, dev, true, &st) == MSDA_OK && st.nqb <= gp->nqb + 1) *gp = st;
  g_last_error.clear();
  return MSDA_OK;
}

int64_t gather_workspace(const Shape& s, const GatherPlan& gp) {
  return gp.nqb > 1 ? static_cast<int64_t>(gp.nqb) * part_block_stride(s) * 4 : 0;
}

int bwd_gather_impl(const Shape& s, const void* value, int value_dtype, const float* loc, const float* attn, const void* grad_output,
                    int grad_output_dtype, void* grad_value, float* grad_loc, float* grad_attn, void* workspace,
                    int64_t workspace_bytes, const DevInfo& dev, hipStream_t st, int sampler = MSDA_SAMPLER_HIP) {
  const int vbytes = value_dtype == MSDA_DTYPE_BF16 ? 2 : 4;
  GatherPlan gp;
  int rc = plan_gather(s, vbytes, dev, &gp);
  if (rc != MSDA_OK) return rc;
  const bool partial = gp.nqb > 1 && grad_value != nullptr;
  if (partial) {
    const int64_t need = gather_workspace(s, gp);
    if (workspace == nullptr || workspace_bytes < need)
      return fail(MSDA_ERR_INVALID_ARGUMENT, "workspace of %lld bytes needed, got %lld (see the workspace size query)",
                  static_cast<long long>(need), static_cast<long long>(workspace == nullptr ? 0 : workspace_bytes));
    if (!aligned(workspace, 16)) return fail(MSDA_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  }
  const int gbytes = grad_output_dtype == MSDA_DTYPE_BF16 ? 2 : 4;
  // rows are moved 16 bytes (value, grad_value, f32 partials) or 8 bytes (bf16 grad_output) at a time
  if (!gather_aligned(value, grad_value, grad_output, gbytes))
    return fail(MSDA_ERR_UNSUPPORTED, "sorted-gather backward needs 16-byte aligned value rows");
  msda::GatherParams p{};
  p.value = value;
  p.loc = loc;
  p.attn = attn;
  p.gout = grad_output;
  p.dvalue = grad_value;
  p.dloc = grad_loc;
  p.dattn = grad_attn;
  p.part = partial ? static_cast<float*>(workspace) : nullptr;
  p.part_stride = part_block_stride(s);
  p.heads = s.heads;
  p.queries = s.queries;
  p.levels = s.levels;
  p.points = s.points;
  p.len_value = s.len_value;
  p.nqb = gp.nqb;
  p.qblock = gp.qblock;
  p.p_shift = (s.points & (s.points - 1)) == 0 ? __builtin_ctz(static_cast<unsigned>(s.points)) : -1;
  p.lds_g = gp.g;
  p.lds_wt = gp.wt;
  p.lds_key = gp.key;
  p.lds_cnt = gp.cnt;
  p.lds_scan = gp.scan;
  p.lds_val = gp.val;
  for (int l = 0; l < s.levels; ++l) p.lv[l] = level_desc(s, l, 0, 1, 0);
  apply_sampler(s, sampler, value_dtype, p.lv);
  const int grid = static_cast<int>(static_cast<int64_t>(s.batch) * s.heads * s.levels * gp.nqb);
  const bool gb = grad_output_dtype == MSDA_DTYPE_BF16;
  rc = value_dtype == MSDA_DTYPE_BF16 ? msda_host::dispatch_bwd_gather<msda::bf16_t>(s.dim, gb, p, grid, gp.threads, gp.lds, st)
                                      : msda_host::dispatch_bwd_gather<float>(s.dim, gb, p, grid, gp.threads, gp.lds, st);
  if (rc != MSDA_OK || !partial) return rc;
  return launch_partial_sums(s, value_dtype, p.part, p.nqb, grad_value, dev, st);
}


}  // namespace

namespace msda_host {
bool env_flag(const char* name) { return env_int(name, 0) != 0; }
int knob(const char* name, int dflt) { return env_int(name, dflt); }

int device_attrs(int* lds_bytes, int* cus) {
  DevInfo d;
  const int rc = device_info(&d);
  if (rc != MSDA_OK) return rc;
  *lds_bytes = d.lds_bytes;
  *cus = d.cus;
  return MSDA_OK;
}
}  // namespace msda_host


namespace {

// What the fused-prologue entry points add (msda_fused_fwd / msda_fused_bwd): the reference
// points, and the reference-point gradient the backward returns.
struct Fused {
  const float* ref;
  int ref_dim;
  float* dref;
};

int check_fused(const Fused& fz, int len_query) {
  if (fz.ref_dim != 2 && fz.ref_dim != 4) return fail(MSDA_ERR_INVALID_ARGUMENT, "ref_dim must be 2 or 4, got %d", fz.ref_dim);
  if (len_query > 0 && fz.ref == nullptr) return fail(MSDA_ERR_INVALID_ARGUMENT, "reference_points is NULL");
  if (!aligned(fz.ref, 4 * static_cast<size_t>(fz.ref_dim)))
    return fail(MSDA_ERR_INVALID_ARGUMENT, "reference_points must be %d-byte aligned", 4 * fz.ref_dim);
  if (!aligned(fz.dref, 4)) return fail(MSDA_ERR_INVALID_ARGUMENT, "grad_reference_points must be 4-byte aligned");
  return MSDA_OK;
}

void fill_fused(msda::SampleParams* p, const Fused* fz, int n_points) {
  if (fz == nullptr) return;
  p->ref = fz->ref;
  p->ref_dim = fz->ref_dim;
  p->fpoints = static_cast<float>(n_points);
  p->inv_points = (n_points & (n_points - 1)) == 0 ? 1.0f / static_cast<float>(n_points) : 0.0f;
}

int fwd_impl(const void* value, int value_dtype, const float* loc, const float* attn, void* output, int output_dtype, int batch,
             int n_heads, int head_dim, int len_query, int n_levels, int n_points, const int32_t* spatial_shapes,
             const int32_t* level_start_index, int64_t len_value, void* stream, const Fused* fz, int sampler = MSDA_SAMPLER_HIP) {
  g_last_error.clear();
  Shape s;
  int rc = validate(&s, batch, n_heads, head_dim, len_query, n_levels, n_points, spatial_shapes, level_start_index, len_value);
  if (rc != MSDA_OK) return rc;
  if ((rc = check_dtype(value_dtype, "value")) != MSDA_OK) return rc;
  if ((rc = check_dtype(output_dtype, "output")) != MSDA_OK) return rc;
  if ((rc = check_sampler(sampler)) != MSDA_OK) return rc;
  if (fz != nullptr && (rc = check_fused(*fz, batch == 0 ? 0 : len_query)) != MSDA_OK) return rc;
  if (batch == 0 || len_query == 0) return MSDA_OK;
  if (value == nullptr || loc == nullptr || attn == nullptr || output == nullptr)
    return fail(MSDA_ERR_INVALID_ARGUMENT, "%s: NULL tensor pointer", fz ? "msda_fused_fwd" : "msda_fwd");
  if (!aligned(loc, 8) || !aligned(attn, 4))
    return fail(MSDA_ERR_INVALID_ARGUMENT, "%s must be 8-byte aligned and %s 4-byte aligned", fz ? "sampling_offsets" : "sampling_locations",
                fz ? "attention_logits" : "attention_weights");
  const int vbytes = value_dtype == MSDA_DTYPE_BF16 ? 2 : 4;
  const int obytes = output_dtype == MSDA_DTYPE_BF16 ? 2 : 4;
  if (!aligned(value, vbytes) || !aligned(output, obytes)) return fail(MSDA_ERR_INVALID_ARGUMENT, "value/output not aligned to their element size");
  const int vec = pick_vec(head_dim, env_int("MSDA_FWD_MAX_VEC", 8), {{value, vbytes}, {output, obytes}});
  const int ns = env_int("MSDA_FWD_GROUPED", 1) ? samples_bound(n_levels, n_points) : 0;
  const int shift = lpq_shift_for(head_dim, vec);
  if (shift > 6) return fail(MSDA_ERR_UNSUPPORTED, "head_dim %d too large (max %d for this dtype)", head_dim, 64 * vec);

  DevInfo dev;
  if ((rc = device_info(&dev)) != MSDA_OK) return rc;

  msda::SampleParams p{};
  p.value = value;
  p.loc = loc;
  p.attn = attn;
  p.out = output;
  p.out_bf16 = output_dtype == MSDA_DTYPE_BF16;
  p.heads = n_heads;
  p.dim = head_dim;
  p.queries = len_query;
  p.levels = n_levels;
  p.points = n_points;
  p.len_value = len_value;
  p.vec16 = rows_16b(s, vbytes, value, nullptr);
  p.rheads = n_heads;
  p.vstride = head_dim;
  p.cs_shift = 0;
  fill_fused(&p, fz, n_points);
  SamplePlan plan;
  if ((rc = plan_sample(s, vbytes, dev, "MSDA_FWD", shift, &p, &plan)) != MSDA_OK) return rc;
  // A level too large for the LDS can be staged by splitting each head's channels over 2 or 4
  // workgroups (one head each) when every level then fits, each part a whole number of 16-byte
  // chunks per cell. Staging reads every cell of the level, gathering only what the samples touch,
  // so the split pays with many queries per slice. Measured on MI355X (forward through a HIP graph,
  // gathered against split): f32 at 3900 queries 78.1 -> 70.1 us (64 x 64 and 32 x 32 levels,
  // 16 heads x 16), 40.7 -> 39.0 (40 x 40 and 20 x 20, 8 x 32), 12.9 -> 11.6 (48 x 48, 8 x 32),
  // at 1200 queries 40.8 -> 30.2 and 21.4 -> 21.2, at 300 queries 14.9 -> 14.7 and 8.8 -> 10.5;
  // bf16 slower at every count (80 x 80 and 20 x 20, 16 x 16: 300 queries 10.5 -> 11.5, 3900
  // queries 63.9 -> 72.9, eager). So: f32 value maps with at least 1024 queries, unless the knob
  // MSDA_FWD_SPLIT says otherwise (0 never, 1 whenever it fits).
  int vec_used = vec, shift_used = shift;
  const int split_knob = env_int("MSDA_FWD_SPLIT", -1);
  const bool split = split_knob > 0 || (split_knob < 0 && vbytes == 4 && len_query >= 1024);
  if (!p.all_staged && aligned(value, 16) && split) {
    for (int cs = 1; cs <= 2; ++cs) {
      const int part = head_dim >> cs;
      if (head_dim % (1 << cs) != 0 || (part * vbytes) % 16 != 0) break;
      Shape s2 = s;
      s2.heads = n_heads << cs;
      s2.dim = part;
      msda::SampleParams p2 = p;
      p2.heads = s2.heads;
      p2.dim = part;
      p2.cs_shift = cs;
      p2.vec16 = 1;
      const int vec2 = pick_vec(part, env_int("MSDA_FWD_MAX_VEC", 8), {{value, vbytes}, {output, obytes}});
      const int shift2 = lpq_shift_for(part, vec2);
      SamplePlan plan2;
      if (plan_sample(s2, vbytes, dev, "MSDA_FWD", shift2, &p2, &plan2, 1) != MSDA_OK) {
        g_last_error.clear();
        continue;
      }
      if (!p2.all_staged) continue;
      s = s2;
      p = p2;
      plan = plan2;
      vec_used = vec2;
      shift_used = shift2;
      break;
    }
  }
  apply_sampler(s, sampler, value_dtype, p.lv);
  bool rounded = false;
  for (int l = 0; l < n_levels; ++l) rounded = rounded || p.lv[l].rmode != msda::kRoundNone;
  // one level, two points, two lanes per (query, head), every level staged: the two lanes split the
  // samples' coordinate work (fwd_pair; f32 interpolation only)
  p.pair_share = (n_levels == 1 && n_points == 2 && shift_used == 1 && p.all_staged && ns == 2 && !rounded && env_int("MSDA_FWD_PAIR", 1)) ? 1 : 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool fused = fz != nullptr;
  if (value_dtype == MSDA_DTYPE_BF16)
    return msda_host::dispatch_fwd<msda::bf16_t>(vec_used, ns, fused, p, plan.grid, plan.threads, plan.lds, st);
  return msda_host::dispatch_fwd<float>(vec_used, ns, fused, p, plan.grid, plan.threads, plan.lds, st);
}

// ------------------------------------------------------------------------------------------
// the fused-prologue backward: prologue kernel, the core's band kernel, epilogue kernel

// Workspace of msda_fused_bwd: the rows' locations and weights formed by the prologue, the
// locations' gradient when grad_sampling_offsets is not requested but the reference points' is,
// and the core's partial sums.
struct FusedLayout {
  int64_t loc, attn, dloc, band, total;
};

FusedLayout fused_layout(const Shape& s, int64_t band_bytes) {
  const int64_t samples = static_cast<int64_t>(s.batch) * s.queries * s.heads * s.levels * s.points;
  FusedLayout f;
  f.loc = 0;
  f.attn = align16(samples * 8);
  f.dloc = f.attn + align16(samples * 4);
  f.band = f.dloc + align16(samples * 8);
  f.total = f.band + band_bytes;
  return f;
}

int fused_bwd_impl(const Shape& s, int ch, const void* value, int value_dtype, const float* offsets, const float* logits,
                   const void* grad_output, int grad_output_dtype, void* grad_value, float* grad_offsets, float* grad_logits,
                   const Fused& fz, void* workspace, int64_t workspace_bytes, const DevInfo& dev, hipStream_t st) {
  const int vbytes = value_dtype == MSDA_DTYPE_BF16 ? 2 : 4;
  if (s.queries == 0)  // grad_value is zero; nothing else has elements
    return bwd_band_impl(s, ch, value, value_dtype, nullptr, nullptr, grad_output, grad_output_dtype, grad_value, nullptr, nullptr,
                         nullptr, 0, dev, st);
  BandPlan bp;
  int rc = plan_band(s, vbytes, ch, dev, &bp);
  if (rc != MSDA_OK) return rc;
  const FusedLayout lay = fused_layout(s, band_workspace(s, bp));
  if (workspace == nullptr || workspace_bytes < lay.total)
    return fail(MSDA_ERR_INVALID_ARGUMENT, "workspace of %lld bytes needed, got %lld (see the workspace size query)",
                static_cast<long long>(lay.total), static_cast<long long>(workspace == nullptr ? 0 : workspace_bytes));
  if (!aligned(workspace, 16)) return fail(MSDA_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  char* ws = static_cast<char*>(workspace);
  const float inv_points = (s.points & (s.points - 1)) == 0 ? 1.0f / static_cast<float>(s.points) : 0.0f;
  // One level that fits the LDS whole, 2 or 4 points, head_dim 16 or 32: the band kernel applies
  // the prologue and epilogue per (query, head) row itself (no row kernels, no location / weight
  // round trip through memory); the reference-point partials of the heads go to the locations'
  // region of the workspace (H * B * Q * ref_dim floats <= B * Q * H * P * 2).
  if (s.levels == 1 && bp.nwork == 1 && (s.points == 2 || s.points == 4) && ch == 8 && (s.dim == 16 || s.dim == 32) &&
      aligned(offsets, 16) && aligned(logits, s.points == 4 ? 16 : 8) && aligned(fz.ref, fz.ref_dim * 4) &&
      env_int("MSDA_FUSED_IN_KERNEL", 1) != 0) {
    float* dref_part = fz.dref != nullptr ? reinterpret_cast<float*>(ws + lay.loc) : nullptr;
    const BandFusedArgs fa{fz.ref, fz.ref_dim, inv_points, static_cast<float>(s.points), dref_part, fz.dref};
    return bwd_band_impl(s, ch, value, value_dtype, offsets, logits, grad_output, grad_output_dtype, grad_value, grad_offsets,
                         grad_logits, ws + lay.band, workspace_bytes - lay.band, dev, st, &fa);
  }
  msda::FusedRowParams fp{};
  fp.ref = fz.ref;
  fp.off = offsets;
  fp.logits = logits;
  fp.loc = reinterpret_cast<float*>(ws + lay.loc);
  fp.attn = reinterpret_cast<float*>(ws + lay.attn);
  fp.ref_dim = fz.ref_dim;
  fp.heads = s.heads;
  fp.levels = s.levels;
  fp.points = s.points;
  fp.bq_total = static_cast<int64_t>(s.batch) * s.queries;
  fp.fpoints = static_cast<float>(s.points);
  fp.inv_points = inv_points;
  for (int l = 0; l < s.levels; ++l) {
    fp.fw[l] = static_cast<float>(s.w[l]);
    fp.fh[l] = static_cast<float>(s.h[l]);
  }
  const int64_t rows = fp.bq_total * s.heads;
  // Rows of at most 32 samples over at most 4 levels, a (b, q) group of heads x samples within 256
  // threads and fewer than 2^31 samples: the kernels with one thread per sample.
  const int lp = s.levels * s.points;
  const int64_t nsamp = rows * lp;
  const int nb = (s.levels <= 4 && lp <= 32 && s.heads * lp <= 256 && nsamp < (int64_t{1} << 31) &&
                  env_int("MSDA_FUSED_PER_SAMPLE", 1) != 0)
                     ? (lp <= 8 ? 8 : lp <= 16 ? 16 : 32)
                     : 0;
  const dim3 pgrid(static_cast<unsigned>((nsamp + 255) / 256));
  if (nb == 8)
    hipLaunchKernelGGL(msda::fused_prologue_samples_kernel<8>, pgrid, dim3(256), 0, st, fp);
  else if (nb == 16)
    hipLaunchKernelGGL(msda::fused_prologue_samples_kernel<16>, pgrid, dim3(256), 0, st, fp);
  else if (nb == 32)
    hipLaunchKernelGGL(msda::fused_prologue_samples_kernel<32>, pgrid, dim3(256), 0, st, fp);
  else
    hipLaunchKernelGGL(msda::fused_prologue_kernel, dim3(static_cast<unsigned>((rows + 255) / 256)), dim3(256), 0, st, fp);
  if ((rc = msda_host::check_launch("msda fused backward (prologue)")) != MSDA_OK) return rc;
  float* dloc = grad_offsets != nullptr ? grad_offsets : (fz.dref != nullptr ? reinterpret_cast<float*>(ws + lay.dloc) : nullptr);
  rc = bwd_band_impl(s, ch, value, value_dtype, fp.loc, fp.attn, grad_output, grad_output_dtype, grad_value, dloc, grad_logits,
                     ws + lay.band, workspace_bytes - lay.band, dev, st);
  if (rc != MSDA_OK) return rc;
  if (dloc == nullptr && grad_logits == nullptr) return MSDA_OK;
  fp.dloc = dloc;
  fp.doff = grad_offsets;
  fp.dlogits = grad_logits;
  fp.dref = fz.dref;
  int hp_shift = 0;
  while ((1 << hp_shift) < s.heads) ++hp_shift;
  const int64_t per_block = 256 >> hp_shift;
  if (nb != 0) {
    const int G = 256 / (s.heads * lp), hp = 1 << hp_shift;
    const dim3 sgrid(static_cast<unsigned>((fp.bq_total + G - 1) / G));
    const size_t lds = static_cast<size_t>(G) * (s.heads * lp + s.levels * hp) * sizeof(float4);
    if (nb == 8)
      hipLaunchKernelGGL(msda::fused_epilogue_samples_kernel<8>, sgrid, dim3(256), lds, st, fp, G, hp);
    else if (nb == 16)
      hipLaunchKernelGGL(msda::fused_epilogue_samples_kernel<16>, sgrid, dim3(256), lds, st, fp, G, hp);
    else
      hipLaunchKernelGGL(msda::fused_epilogue_samples_kernel<32>, sgrid, dim3(256), lds, st, fp, G, hp);
  } else {
    hipLaunchKernelGGL(msda::fused_epilogue_kernel, dim3(static_cast<unsigned>((fp.bq_total + per_block - 1) / per_block)),
                       dim3(256), 0, st, fp, hp_shift);
  }
  return msda_host::check_launch("msda fused backward (epilogue)");
}

int64_t workspace_impl(int batch, int n_heads, int head_dim, int len_query, int n_levels, int n_points, const int32_t* spatial_shapes,
                       const int32_t* level_start_index, int64_t len_value, int ref_dim) {
  g_last_error.clear();
  Shape s;
  int rc = validate(&s, batch, n_heads, head_dim, len_query, n_levels, n_points, spatial_shapes, level_start_index, len_value);
  if (rc != MSDA_OK) return rc;
  if (ref_dim != 0 && ref_dim != 2 && ref_dim != 4) return fail(MSDA_ERR_INVALID_ARGUMENT, "ref_dim must be 2 or 4, got %d", ref_dim);
  if (batch == 0 || len_query == 0) return 0;
  DevInfo dev;
  if ((rc = device_info(&dev)) != MSDA_OK) return rc;
  // The plan depends on the value dtype, which the query does not name: the larger need of the
  // dtypes whose plan fits (a wide level can fit the LDS in bf16 but not in f32); an error only if
  // neither fits. For the core op either backward kernel may run (the sorted gather needs aligned
  // rows), so also the larger of the two kernels' needs.
  int64_t need = 0;
  int planned = 0, err = MSDA_OK;
  std::string msg;
  for (int vbytes : {2, 4}) {
    BandPlan bp;
    if ((rc = plan_band(s, vbytes, 16, dev, &bp)) != MSDA_OK) {
      err = rc;
      msg = g_last_error;
      continue;
    }
    ++planned;
    if (ref_dim != 0) {
      need = std::max(need, fused_layout(s, band_workspace(s, bp)).total);
      continue;
    }
    need = std::max(need, band_workspace(s, bp));
    GatherPlan gp;
    if (gather_eligible(s) && plan_gather(s, vbytes, dev, &gp) == MSDA_OK) need = std::max(need, gather_workspace(s, gp));
  }
  if (planned == 0) {
    g_last_error = msg;
    return err;
  }
  g_last_error.clear();
  return need;
}

int bwd_impl(const void* value, int value_dtype, const float* loc, const float* attn, const void* grad_output, int grad_output_dtype,
             void* grad_value, float* grad_loc, float* grad_attn, int batch, int n_heads, int head_dim, int len_query, int n_levels,
             int n_points, const int32_t* spatial_shapes, const int32_t* level_start_index, int64_t len_value, void* workspace,
             int64_t workspace_bytes, void* stream, const Fused* fz, int sampler = MSDA_SAMPLER_HIP) {
  g_last_error.clear();
  Shape s;
  int rc = validate(&s, batch, n_heads, head_dim, len_query, n_levels, n_points, spatial_shapes, level_start_index, len_value);
  if (rc != MSDA_OK) return rc;
  if ((rc = check_sampler(sampler)) != MSDA_OK) return rc;
  if ((rc = check_dtype(value_dtype, "value")) != MSDA_OK) return rc;
  if ((rc = check_dtype(grad_output_dtype, "grad_output")) != MSDA_OK) return rc;
  const char* name = fz ? "msda_fused_bwd" : "msda_bwd";
  if (fz != nullptr && (rc = check_fused(*fz, batch == 0 ? 0 : len_query)) != MSDA_OK) return rc;
  if (batch == 0) return MSDA_OK;
  const bool want_dref = fz != nullptr && fz->dref != nullptr && len_query > 0;
  if (grad_value == nullptr && grad_loc == nullptr && grad_attn == nullptr && !want_dref) return MSDA_OK;
  if (value == nullptr) return fail(MSDA_ERR_INVALID_ARGUMENT, "%s: value is NULL", name);
  if (len_query > 0 && (loc == nullptr || attn == nullptr || grad_output == nullptr))
    return fail(MSDA_ERR_INVALID_ARGUMENT, "%s: NULL tensor pointer", name);
  if (!aligned(loc, 8) || !aligned(attn, 4) || !aligned(grad_loc, 8) || !aligned(grad_attn, 4))
    return fail(MSDA_ERR_INVALID_ARGUMENT, "location tensors must be 8-byte aligned and weight tensors 4-byte aligned");
  const int vbytes = value_dtype == MSDA_DTYPE_BF16 ? 2 : 4;
  const int gbytes = grad_output_dtype == MSDA_DTYPE_BF16 ? 2 : 4;
  if (!aligned(value, vbytes) || !aligned(grad_value, vbytes) || !aligned(grad_output, gbytes))
    return fail(MSDA_ERR_INVALID_ARGUMENT, "value/grad_value/grad_output not aligned to their element size");
  for (int l = 0; l < n_levels; ++l)
    if (s.h[l] > 32000 || s.w[l] > 32000)
      return fail(MSDA_ERR_UNSUPPORTED, "level %d (%d x %d) exceeds 32000 rows or columns", l, s.h[l], s.w[l]);
  if (static_cast<int64_t>(len_query) * n_heads * head_dim >= (int64_t{1} << 30))
    return fail(MSDA_ERR_UNSUPPORTED, "len_query * n_heads * head_dim reaches 2^30");
  // a workgroup addresses one batch entry's sample rows with 32-bit offsets (24-bit multiplies)
  if (static_cast<int64_t>(len_query) * n_heads * n_levels * n_points >= (int64_t{1} << 24) ||
      static_cast<int64_t>(n_heads) * head_dim * 4 >= (int64_t{1} << 24))
    return fail(MSDA_ERR_UNSUPPORTED, "len_query * n_heads * n_levels * n_points reaches 2^24");
  if (fz != nullptr && n_heads > 64) return fail(MSDA_ERR_UNSUPPORTED, "msda_fused_bwd supports at most 64 heads, got %d", n_heads);
  // the fused backward keeps the prologue's locations and weights in the workspace
  if (fz != nullptr && len_query > 0 && workspace == nullptr)
    return fail(MSDA_ERR_INVALID_ARGUMENT, "msda_fused_bwd: workspace is NULL (see the workspace size query)");
  // 8-channel lanes: measured on MI355X faster than 16 at head_dim 16 (nano 12.1 vs 13.4 us,
  // nano_groupdetr 36.9 vs 43.0, two_level 58.5 vs 82.6)
  const int ch = pick_vec(head_dim, env_int("MSDA_BWD_MAX_VEC", 8), {{value, vbytes}, {grad_output, gbytes}});
  if (lpq_shift_for(head_dim, ch) > 6) return fail(MSDA_ERR_UNSUPPORTED, "head_dim %d too large (max %d)", head_dim, 64 * ch);
  DevInfo dev;
  if ((rc = device_info(&dev)) != MSDA_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (fz != nullptr)
    return fused_bwd_impl(s, ch, value, value_dtype, loc, attn, grad_output, grad_output_dtype, grad_value, grad_loc, grad_attn, *fz,
                          workspace, workspace_bytes, dev, st);
  GatherPlan gp;
  if (len_query > 0 && gather_eligible(s) && gather_aligned(value, grad_value, grad_output, gbytes) &&
      plan_gather(s, vbytes, dev, &gp) == MSDA_OK)
    return bwd_gather_impl(s, value, value_dtype, loc, attn, grad_output, grad_output_dtype, grad_value, grad_loc, grad_attn,
                           workspace, workspace_bytes, dev, st, sampler);
  g_last_error.clear();
  return bwd_band_impl(s, ch, value, value_dtype, loc, attn, grad_output, grad_output_dtype, grad_value, grad_loc, grad_attn,
                       workspace, workspace_bytes, dev, st, nullptr, sampler);
}

}  // namespace

extern "C" {

const char* msda_version(void) { return "msda-gfx950 0.3.0"; }

const char* msda_last_error(void) { return g_last_error.c_str(); }

int msda_set_tuning(const char* name, const char* value) {
  g_last_error.clear();
  if (name == nullptr || std::string(name).rfind("MSDA_", 0) != 0)
    return fail(MSDA_ERR_INVALID_ARGUMENT, "tuning knob names start with MSDA_");
  std::lock_guard<std::mutex> lock(g_knob_mu);
  if (value == nullptr) {
    g_knob_set.erase(name);
  } else {
    const bool set = *value != 0;
    g_knob_set[name] = std::make_pair(set, set ? std::atoi(value) : 0);
  }
  return MSDA_OK;
}

int msda_fwd(const void* value, int value_dtype, const float* sampling_locations, const float* attention_weights,
             void* output, int output_dtype, int batch, int n_heads, int head_dim, int len_query, int n_levels,
             int n_points, const int32_t* spatial_shapes, const int32_t* level_start_index, int64_t len_value,
             void* stream) {
  return fwd_impl(value, value_dtype, sampling_locations, attention_weights, output, output_dtype, batch, n_heads, head_dim, len_query,
                  n_levels, n_points, spatial_shapes, level_start_index, len_value, stream, nullptr);
}

int msda_fwd_sampler(const void* value, int value_dtype, const float* sampling_locations, const float* attention_weights,
                     void* output, int output_dtype, int sampler, int batch, int n_heads, int head_dim, int len_query, int n_levels,
                     int n_points, const int32_t* spatial_shapes, const int32_t* level_start_index, int64_t len_value,
                     void* stream) {
  return fwd_impl(value, value_dtype, sampling_locations, attention_weights, output, output_dtype, batch, n_heads, head_dim, len_query,
                  n_levels, n_points, spatial_shapes, level_start_index, len_value, stream, nullptr, sampler);
}

int64_t msda_bwd_workspace_size(int batch, int n_heads, int head_dim, int len_query, int n_levels, int n_points,
                                const int32_t* spatial_shapes, const int32_t* level_start_index, int64_t len_value) {
  return workspace_impl(batch, n_heads, head_dim, len_query, n_levels, n_points, spatial_shapes, level_start_index, len_value, 0);
}

int msda_bwd(const void* value, int value_dtype, const float* sampling_locations, const float* attention_weights,
             const void* grad_output, int grad_output_dtype, void* grad_value, float* grad_sampling_locations,
             float* grad_attention_weights, int batch, int n_heads, int head_dim, int len_query, int n_levels,
             int n_points, const int32_t* spatial_shapes, const int32_t* level_start_index, int64_t len_value,
             void* workspace, int64_t workspace_bytes, void* stream) {
  return bwd_impl(value, value_dtype, sampling_locations, attention_weights, grad_output, grad_output_dtype, grad_value,
                  grad_sampling_locations, grad_attention_weights, batch, n_heads, head_dim, len_query, n_levels, n_points,
                  spatial_shapes, level_start_index, len_value, workspace, workspace_bytes, stream, nullptr);
}

int msda_bwd_sampler(const void* value, int value_dtype, const float* sampling_locations, const float* attention_weights,
                     const void* grad_output, int grad_output_dtype, void* grad_value, float* grad_sampling_locations,
                     float* grad_attention_weights, int sampler, int batch, int n_heads, int head_dim, int len_query, int n_levels,
                     int n_points, const int32_t* spatial_shapes, const int32_t* level_start_index, int64_t len_value,
                     void* workspace, int64_t workspace_bytes, void* stream) {
  return bwd_impl(value, value_dtype, sampling_locations, attention_weights, grad_output, grad_output_dtype, grad_value,
                  grad_sampling_locations, grad_attention_weights, batch, n_heads, head_dim, len_query, n_levels, n_points,
                  spatial_shapes, level_start_index, len_value, workspace, workspace_bytes, stream, nullptr, sampler);
}

int msda_bwd_noalloc(const void* value, int value_dtype, const float* sampling_locations, const float* attention_weights,
                     const void* grad_output, int grad_output_dtype, void* grad_value, float* grad_sampling_locations,
                     float* grad_attention_weights, int batch, int n_heads, int head_dim, int len_query, int n_levels,
                     int n_points, const int32_t* spatial_shapes, const int32_t* level_start_index, int64_t len_value,
                     void* stream) {
  const int64_t need = workspace_impl(batch, n_heads, head_dim, len_query, n_levels, n_points, spatial_shapes, level_start_index,
                                      len_value, 0);
  if (need < 0) return static_cast<int>(need);
  if (need > kNoAllocScratchBytes)
    return fail(MSDA_ERR_UNSUPPORTED, "msda_bwd_noalloc: this shape needs %lld bytes of scratch, the library holds %lld",
                static_cast<long long>(need), static_cast<long long>(kNoAllocScratchBytes));
  void* ws = nullptr;
  if (need > 0) {
    const int rc = noalloc_scratch(&ws);
    if (rc != MSDA_OK) return rc;
  }
  return bwd_impl(value, value_dtype, sampling_locations, attention_weights, grad_output, grad_output_dtype, grad_value,
                  grad_sampling_locations, grad_attention_weights, batch, n_heads, head_dim, len_query, n_levels, n_points,
                  spatial_shapes, level_start_index, len_value, ws, need > 0 ? kNoAllocScratchBytes : 0, stream, nullptr);
}

int msda_fused_fwd(const void* value, int value_dtype, const float* reference_points, int ref_dim, const float* sampling_offsets,
                   const float* attention_logits, void* output, int output_dtype, int batch, int n_heads, int head_dim,
                   int len_query, int n_levels, int n_points, const int32_t* spatial_shapes, const int32_t* level_start_index,
                   int64_t len_value, void* stream) {
  const Fused fz{reference_points, ref_dim, nullptr};
  return fwd_impl(value, value_dtype, sampling_offsets, attention_logits, output, output_dtype, batch, n_heads, head_dim, len_query,
                  n_levels, n_points, spatial_shapes, level_start_index, len_value, stream, &fz);
}

int64_t msda_fused_bwd_workspace_size(int batch, int n_heads, int head_dim, int len_query, int n_levels, int n_points, int ref_dim,
                                      const int32_t* spatial_shapes, const int32_t* level_start_index, int64_t len_value) {
  if (ref_dim != 2 && ref_dim != 4) {
    g_last_error.clear();
    return fail(MSDA_ERR_INVALID_ARGUMENT, "ref_dim must be 2 or 4, got %d", ref_dim);
  }
  return workspace_impl(batch, n_heads, head_dim, len_query, n_levels, n_points, spatial_shapes, level_start_index, len_value, ref_dim);
}

int msda_fused_bwd(const void* value, int value_dtype, const float* reference_points, int ref_dim, const float* sampling_offsets,
                   const float* attention_logits, const void* grad_output, int grad_output_dtype, void* grad_value,
                   float* grad_sampling_offsets, float* grad_attention_logits, float* grad_reference_points, int batch, int n_heads,
                   int head_dim, int len_query, int n_levels, int n_points, const int32_t* spatial_shapes,
                   const int32_t* level_start_index, int64_t len_value, void* workspace, int64_t workspace_bytes, void* stream) {
  const Fused fz{reference_points, ref_dim, grad_reference_points};
  return bwd_impl(value, value_dtype, sampling_offsets, attention_logits, grad_output, grad_output_dtype, grad_value,
                  grad_sampling_offsets, grad_attention_logits, batch, n_heads, head_dim, len_query, n_levels, n_points, spatial_shapes,
                  level_start_index, len_value, workspace, workspace_bytes, stream, &fz);
}

}  // extern "C"

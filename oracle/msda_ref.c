/*
 * msda_ref.c — C restatement of RF-DETR-JAX's deformable-attention gather path, in f32.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ as a second oracle at full benchmark sizes and by
 * bench.py as the CPU baseline ("port"). Nothing in the product library links or calls it.
 *
 * Follows, in single precision like the reference's f32 run:
 *   coordinates   src/rfdetr_jax/models/ops.py:270 (grid = 2*loc - 1) and ops.py:83-84
 *                 (ix = ((grid + 1) * W - 1) / 2), one rounding per operation (no FMA contraction:
 *                 this file is compiled with -ffp-contract=off);
 *   floor, masks, clipped corners, weights   ops.py:85-128 (corner order (x0,y0),(x1,y0),(x0,y1),(x1,y1));
 *   corner sum    ops.py:133-134; point-weighted sum over level-major points   ops.py:285-289;
 *   output layout [B, Q, H*D]   ops.py:290-292.
 * The backward pass is the VJP JAX autodiff takes of those lines: dA = <g, sample>,
 * dloc = A * size * <g, d sample / d pixel>, and dV scatter-added at the clipped corner indices
 * with the masked weights (the transpose of the take_along_axis at ops.py:120).
 *
 * Work is split over the batch*heads slices with OpenMP; each slice writes disjoint outputs.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct {
  int32_t idx[4];  /* clipped flat corner index within the level */
  float w[4];      /* masked corner weights (x0y0, x1y0, x0y1, x1y1) */
  float m[4];      /* in-bounds masks */
  float fx, fy;    /* fractional parts */
} corners_t;

static float pixel(float loc, int size) {
  float grid = 2.0f * loc - 1.0f;
  return ((grid + 1.0f) * (float)size - 1.0f) / 2.0f;
}

static int32_t sat_int(float v) {
  if (v != v) return 0; /* NaN -> 0, XLA convert semantics */
  if (v <= -2147483648.0f) return INT32_MIN;
  if (v >= 2147483647.0f) return INT32_MAX;
  return (int32_t)v;
}

static int32_t clip(int64_t v, int32_t hi) { return v < 0 ? 0 : (v > hi ? hi : (int32_t)v); }

static void corners(float lx, float ly, int h, int w, corners_t* c) {
  float ix = pixel(lx, w), iy = pixel(ly, h);
  float ix0 = floorf(ix), iy0 = floorf(iy);
  float fx = ix - ix0, fy = iy - iy0;
  float gx = 1.0f - fx, gy = 1.0f - fy;
  int64_t x0 = sat_int(ix0), y0 = sat_int(iy0), x1 = x0 + 1, y1 = y0 + 1;
  int inx0 = x0 >= 0 && x0 < w, inx1 = x1 >= 0 && x1 < w;
  int iny0 = y0 >= 0 && y0 < h, iny1 = y1 >= 0 && y1 < h;
  int32_t cx0 = clip(x0, w - 1), cx1 = clip(x1, w - 1), cy0 = clip(y0, h - 1), cy1 = clip(y1, h - 1);
  c->idx[0] = cy0 * w + cx0;
  c->idx[1] = cy0 * w + cx1;
  c->idx[2] = cy1 * w + cx0;
  c->idx[3] = cy1 * w + cx1;
  c->m[0] = (float)(inx0 && iny0);
  c->m[1] = (float)(inx1 && iny0);
  c->m[2] = (float)(inx0 && iny1);
  c->m[3] = (float)(inx1 && iny1);
  c->w[0] = gx * gy * c->m[0];
  c->w[1] = fx * gy * c->m[1];
  c->w[2] = gx * fy * c->m[2];
  c->w[3] = fx * fy * c->m[3];
  c->fx = fx;
  c->fy = fy;
}

static void set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
}

int msda_oracle_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* out[B,Q,H*D] = sum_{l,p} A * bilinear(value[b*H+h], l, loc). shapes: [L][2] = (H_l, W_l). */
int msda_oracle_fwd(const float* value, const float* loc, const float* attn, float* out,
                    int B, int H, int D, int Q, int L, int P, const int32_t* shapes, int64_t S,
                    int threads) {
  int64_t starts[64];
  if (L > 64 || D > 1024) return -1;
  int64_t acc = 0;
  for (int l = 0; l < L; ++l) { starts[l] = acc; acc += (int64_t)shapes[2 * l] * shapes[2 * l + 1]; }
  if (acc != S) return -1;
  set_threads(threads);
  const int64_t N = (int64_t)B * H;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t n = 0; n < N; ++n) {
    const int b = (int)(n / H), h = (int)(n % H);
    const float* vs = value + n * S * D;
    float sample[1024];
    float total[1024];
    for (int q = 0; q < Q; ++q) {
      const int64_t bqh = ((int64_t)b * Q + q) * H + h;
      for (int d = 0; d < D; ++d) total[d] = 0.0f;
      for (int l = 0; l < L; ++l) {
        const int hl = shapes[2 * l], wl = shapes[2 * l + 1];
        const float* vl = vs + starts[l] * D;
        for (int p = 0; p < P; ++p) {
          const int64_t s = bqh * L * P + (int64_t)l * P + p;
          corners_t c;
          corners(loc[2 * s], loc[2 * s + 1], hl, wl, &c);
          for (int d = 0; d < D; ++d) {
            sample[d] = vl[(int64_t)c.idx[0] * D + d] * c.w[0] + vl[(int64_t)c.idx[1] * D + d] * c.w[1] +
                        vl[(int64_t)c.idx[2] * D + d] * c.w[2] + vl[(int64_t)c.idx[3] * D + d] * c.w[3];
          }
          const float a = attn[s];
          for (int d = 0; d < D; ++d) total[d] += a * sample[d];
        }
      }
      memcpy(out + bqh * D, total, sizeof(float) * (size_t)D);
    }
  }
  return 0;
}

/* Gradients of msda_oracle_fwd for cotangent gout[B,Q,H*D]; dvalue is overwritten. */
int msda_oracle_bwd(const float* value, const float* loc, const float* attn, const float* gout,
                    float* dvalue, float* dloc, float* dattn,
                    int B, int H, int D, int Q, int L, int P, const int32_t* shapes, int64_t S,
                    int threads) {
  int64_t starts[64];
  if (L > 64 || D > 1024) return -1;
  int64_t acc = 0;
  for (int l = 0; l < L; ++l) { starts[l] = acc; acc += (int64_t)shapes[2 * l] * shapes[2 * l + 1]; }
  if (acc != S) return -1;
  set_threads(threads);
  const int64_t N = (int64_t)B * H;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t n = 0; n < N; ++n) {
    const int b = (int)(n / H), h = (int)(n % H);
    const float* vs = value + n * S * D;
    float* dvs = dvalue + n * S * D;
    memset(dvs, 0, sizeof(float) * (size_t)(S * D));
    for (int q = 0; q < Q; ++q) {
      const int64_t bqh = ((int64_t)b * Q + q) * H + h;
      const float* g = gout + bqh * D;
      for (int l = 0; l < L; ++l) {
        const int hl = shapes[2 * l], wl = shapes[2 * l + 1];
        const float* vl = vs + starts[l] * D;
        float* dvl = dvs + starts[l] * D;
        for (int p = 0; p < P; ++p) {
          const int64_t s = bqh * L * P + (int64_t)l * P + p;
          corners_t c;
          corners(loc[2 * s], loc[2 * s + 1], hl, wl, &c);
          const float a = attn[s];
          const float gx = 1.0f - c.fx, gy = 1.0f - c.fy;
          float da = 0.0f, dx = 0.0f, dy = 0.0f;
          for (int d = 0; d < D; ++d) {
            const float v00 = vl[(int64_t)c.idx[0] * D + d] * c.m[0];
            const float v10 = vl[(int64_t)c.idx[1] * D + d] * c.m[1];
            const float v01 = vl[(int64_t)c.idx[2] * D + d] * c.m[2];
            const float v11 = vl[(int64_t)c.idx[3] * D + d] * c.m[3];
            const float smp = vl[(int64_t)c.idx[0] * D + d] * c.w[0] + vl[(int64_t)c.idx[1] * D + d] * c.w[1] +
                              vl[(int64_t)c.idx[2] * D + d] * c.w[2] + vl[(int64_t)c.idx[3] * D + d] * c.w[3];
            da += g[d] * smp;
            dx += g[d] * (gy * (v10 - v00) + c.fy * (v11 - v01));
            dy += g[d] * (gx * (v01 - v00) + c.fx * (v11 - v10));
          }
          dattn[s] = da;
          dloc[2 * s] = a * (float)wl * dx;
          dloc[2 * s + 1] = a * (float)hl * dy;
          for (int k = 0; k < 4; ++k) {
            const float aw = a * c.w[k];
            float* row = dvl + (int64_t)c.idx[k] * D;
            for (int d = 0; d < D; ++d) row[d] += aw * g[d];
          }
        }
      }
    }
  }
  return 0;
}

/*
 * vrs_oracle.c -- CPU restatement of the vision-rs YOLO26 inference hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * path: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  The product library never links or calls it.
 *
 * Layout convention: NCHW float32, exactly as the reference's tensors and
 * fixtures (the fixture generators under tests/fixtures save NCHW row-major f32).
 * Each function cites the reference file:line whose semantics it restates.
 *
 * Parity pins (what checks each function; see tests/test_oracle_golden.py):
 *   orc_conv2d            conv_grouped/{depthwise,g4}, conv_yolo26, c3k2, c2psa,
 *                         sppf, detect_yolo26 fixtures + torch F.conv2d
 *   orc_bn_fold/affine    c3k2/c2psa/sppf/detect fixtures (eval-mode BN)
 *   orc_bn_train          conv_yolo26 fixture (train-mode BN, batch statistics)
 *   orc_maxpool2d         sppf fixture + torch F.max_pool2d (edges)
 *   orc_upsample_nearest  concat_upsample fixture
 *   orc_silu/orc_sigmoid  silu_4d / sigmoid_4d fixtures
 *   orc_psa_attention     c2psa fixture + torch softmax(QK^T)V restatement
 *   orc_detect_decode_grid detect_decode fixture (A13 layout)
 *   orc_detect_postprocess closed-form decode + brute-force argmax/sort checks
 *   orc_detect_unletterbox closed forms (square image: divide by the size;
 *                         2:1 image: known scale and padding)
 *   orc_letterbox         torch F.interpolate(bilinear, antialias=True) on the
 *                         float stage (same triangle filter, PIL formulation),
 *                         closed forms (identity, 2x [1,3,3,1]/8, a half-way
 *                         rounding case), geometry of the reference
 *   orc_msda              torch F.grid_sample (bilinear, zeros, align_corners=False)
 *                         + brute-force tiny cases
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Compiler and flags this library was built with (reported beside the CPU
 * baseline's timings). */
#ifndef ORC_FLAGS
#define ORC_FLAGS "(flags not recorded)"
#endif
const char* orc_build_info(void) {
#if defined(__clang__)
  return "clang " __clang_version__ "; " ORC_FLAGS;
#elif defined(__GNUC__)
  return "gcc " __VERSION__ "; " ORC_FLAGS;
#else
  return "unknown compiler; " ORC_FLAGS;
#endif
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* Conv2d, grouped, zero padding, optional bias.                              */
/* Semantics: teeny-kernels Conv2dForward as called at                       */
/*   tests/test_conv_grouped_cuda.rs:79-113 (args x,w,y,B,Cin,Cout,Hin,Win,  */
/*   Hout,Wout) and the layer constructors blocks/conv.rs:31-99 (pad = k/2). */
/* y[b,co,oy,ox] = bias[co] + sum_{ci in group, ky, kx}                       */
/*     w[co, ci_local, ky, kx] * x[b, ci, oy*s+ky-p, ox*s+kx-p]              */
/* Implemented as im2col + blocked SGEMM so the CPU baseline is not naive.   */
/* ------------------------------------------------------------------------ */

#define GEMM_CO 8
#define GEMM_P 256

/* out[co][p] (+)= W[co][k] * col[k][p], co in [0,CO), p in [0,P) */
static void sgemm_rows(const float* W, int K, const float* col, int P, float* out, int CO) {
  float acc[GEMM_CO][GEMM_P];
  for (int co0 = 0; co0 < CO; co0 += GEMM_CO) {
    int nco = CO - co0 < GEMM_CO ? CO - co0 : GEMM_CO;
    for (int p0 = 0; p0 < P; p0 += GEMM_P) {
      int np = P - p0 < GEMM_P ? P - p0 : GEMM_P;
      for (int r = 0; r < GEMM_CO; ++r)
        for (int p = 0; p < GEMM_P; ++p) acc[r][p] = 0.f;
      for (int k = 0; k < K; ++k) {
        const float* ck = col + (size_t)k * P + p0;
        for (int r = 0; r < nco; ++r) {
          const float a = W[(size_t)(co0 + r) * K + k];
          float* ar = acc[r];
          for (int p = 0; p < np; ++p) ar[p] += a * ck[p];
        }
      }
      for (int r = 0; r < nco; ++r)
        memcpy(out + (size_t)(co0 + r) * P + p0, acc[r], sizeof(float) * np);
    }
  }
}

void orc_conv2d(const float* x, int B, int Cin, int H, int W,
                const float* w, int Cout, int kh, int kw, int stride, int pad, int groups,
                const float* bias, float* y) {
  const int Ho = (H + 2 * pad - kh) / stride + 1;
  const int Wo = (W + 2 * pad - kw) / stride + 1;
  const int cig = Cin / groups, cog = Cout / groups;
  const int K = cig * kh * kw;
  const int P = Ho * Wo;
  const int direct = (kh == 1 && kw == 1 && stride == 1 && pad == 0);
  /* Parallel over (batch, group, output-channel block); each task builds the
   * im2col panel it needs (cheap relative to the GEMM for every YOLO26 shape). */
  const int cob = 64;
  const int ncob = (cog + cob - 1) / cob;
  const long ntask = (long)B * groups * ncob;
#pragma omp parallel
  {
    float* col = direct ? NULL : (float*)malloc(sizeof(float) * (size_t)K * P);
#pragma omp for schedule(dynamic, 1)
    for (long t = 0; t < ntask; ++t) {
      const int b = (int)(t / ((long)groups * ncob));
      const int g = (int)((t / ncob) % groups);
      const int cb = (int)(t % ncob);
      const float* xg = x + ((size_t)b * Cin + (size_t)g * cig) * H * W;
      const float* panel;
      if (direct) {
        panel = xg;
      } else {
        for (int ci = 0; ci < cig; ++ci)
          for (int ky = 0; ky < kh; ++ky)
            for (int kx = 0; kx < kw; ++kx) {
              float* dst = col + ((size_t)(ci * kh + ky) * kw + kx) * P;
              for (int oy = 0; oy < Ho; ++oy) {
                const int iy = oy * stride + ky - pad;
                for (int ox = 0; ox < Wo; ++ox) {
                  const int ix = ox * stride + kx - pad;
                  dst[oy * Wo + ox] = (iy >= 0 && iy < H && ix >= 0 && ix < W)
                                          ? xg[((size_t)ci * H + iy) * W + ix] : 0.f;
                }
              }
            }
        panel = col;
      }
      const int co0 = g * cog + cb * cob;
      const int nco = (cog - cb * cob) < cob ? (cog - cb * cob) : cob;
      float* yo = y + ((size_t)b * Cout + co0) * P;
      sgemm_rows(w + (size_t)co0 * K, K, panel, P, yo, nco);
      if (bias)
        for (int r = 0; r < nco; ++r)
          for (int p = 0; p < P; ++p) yo[(size_t)r * P + p] += bias[co0 + r];
    }
    free(col);
  }
}

/* ------------------------------------------------------------------------ */
/* BatchNorm folding: examples/yolo26.rs:3437-3495                            */
/*   bn_scale[c] = gamma[c] / sqrt(var[c] + eps); bn_shift[c] = beta - scale*mean */
/* ------------------------------------------------------------------------ */
void orc_bn_fold(const float* gamma, const float* beta, const float* mean, const float* var,
                 float eps, int C, float* scale, float* shift) {
  for (int c = 0; c < C; ++c) {
    const float s = gamma[c] / sqrtf(var[c] + eps);
    scale[c] = s;
    shift[c] = beta[c] - s * mean[c];
  }
}

/* y = act(scale[c]*y + shift[c]); act 0 = none, 1 = SiLU (blocks/conv.rs:31-46) */
void orc_affine_act(float* y, int B, int C, int HW, const float* scale, const float* shift, int act) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int c = 0; c < C; ++c) {
      float* p = y + ((size_t)b * C + c) * HW;
      const float s = scale ? scale[c] : 1.f, t = shift ? shift[c] : 0.f;
      for (int i = 0; i < HW; ++i) {
        float v = s * p[i] + t;
        if (act == 1) v = v / (1.f + expf(-v));
        p[i] = v;
      }
    }
}

/* Training-mode BN with batch statistics (biased variance), as the
 * conv_yolo26 fixture uses (tests/fixtures/conv_yolo26/generate.py:37-38). */
void orc_bn_train(float* y, int B, int C, int HW, const float* gamma, const float* beta, float eps) {
  for (int c = 0; c < C; ++c) {
    double s = 0, s2 = 0;
    for (int b = 0; b < B; ++b)
      for (int i = 0; i < HW; ++i) {
        const double v = y[((size_t)b * C + c) * HW + i];
        s += v; s2 += v * v;
      }
    const double n = (double)B * HW;
    const double mean = s / n, var = s2 / n - mean * mean;
    const float rstd = (float)(1.0 / sqrt(var + eps));
    for (int b = 0; b < B; ++b)
      for (int i = 0; i < HW; ++i) {
        float* p = &y[((size_t)b * C + c) * HW + i];
        *p = (float)((*p - mean) * rstd) * gamma[c] + beta[c];
      }
  }
}

/* SiLU forward x*sigmoid(x) (teeny-kernels SiluForward, tests/test_c2psa_cuda.rs:327-331) */
void orc_silu(const float* x, float* y, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) y[i] = x[i] / (1.f + expf(-x[i]));
}

void orc_sigmoid(const float* x, float* y, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) y[i] = 1.f / (1.f + expf(-x[i]));
}

/* MaxPool2d, padding acts as -inf (window clipped to the image):
 * teeny-core MaxPool2d::with_padding((5,5),(1,1),(2,2)) at blocks/sppf.rs:48-50. */
void orc_maxpool2d(const float* x, int B, int C, int H, int W, int k, int s, int p, float* y) {
  const int Ho = (H + 2 * p - k) / s + 1, Wo = (W + 2 * p - k) / s + 1;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int c = 0; c < C; ++c) {
      const float* xp = x + ((size_t)b * C + c) * H * W;
      float* yp = y + ((size_t)b * C + c) * Ho * Wo;
      for (int oy = 0; oy < Ho; ++oy)
        for (int ox = 0; ox < Wo; ++ox) {
          float m = -INFINITY;
          for (int ky = 0; ky < k; ++ky) {
            const int iy = oy * s + ky - p;
            if (iy < 0 || iy >= H) continue;
            for (int kx = 0; kx < k; ++kx) {
              const int ix = ox * s + kx - p;
              if (ix < 0 || ix >= W) continue;
              const float v = xp[iy * W + ix];
              if (v > m) m = v;
            }
          }
          yp[oy * Wo + ox] = m;
        }
    }
}

/* Nearest upsample, integer scale (blocks/upsample.rs:23-35): y[oy,ox] = x[oy/sh, ox/sw] */
void orc_upsample_nearest(const float* x, int B, int C, int H, int W, int sh, int sw, float* y) {
  const int Ho = H * sh, Wo = W * sw;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int c = 0; c < C; ++c) {
      const float* xp = x + ((size_t)b * C + c) * H * W;
      float* yp = y + ((size_t)b * C + c) * Ho * Wo;
      for (int oy = 0; oy < Ho; ++oy)
        for (int ox = 0; ox < Wo; ++ox) yp[oy * Wo + ox] = xp[(oy / sh) * W + ox / sw];
    }
}

/* ------------------------------------------------------------------------ */
/* PSA attention core.                                                        */
/* Channel layout of the qkv conv output, per head h (psa.rs:23-32, and the  */
/* ultralytics Attention split restated in tests/fixtures/c2psa_yolo26/      */
/* generate.py:1-36): channels [h*(2kd+vd) + 0:kd] = q, [+kd:2kd] = k,       */
/* [+2kd : 2kd+vd] = v.  Softmax scale kd^-0.5 (psa.rs:986), online softmax  */
/* equivalent to the exact softmax (flash_attn2.rs:53-121).                  */
/* out[b, h*vd + d, n] = sum_j softmax_j(q_n . k_j * scale) v[d, j]          */
/* ------------------------------------------------------------------------ */
void orc_psa_attention(const float* qkv, int B, int heads, int kd, int vd, int N, float* out) {
  const int cq = heads * (2 * kd + vd);
  const int c = heads * vd;
  const float scale = 1.f / sqrtf((float)kd);
#pragma omp parallel
  {
    float* srow = (float*)malloc(sizeof(float) * N);
#pragma omp for collapse(2) schedule(dynamic, 1)
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < heads; ++h) {
        const float* base = qkv + ((size_t)b * cq + (size_t)h * (2 * kd + vd)) * N;
        const float* q = base;
        const float* k = base + (size_t)kd * N;
        const float* v = base + (size_t)2 * kd * N;
        float* o = out + ((size_t)b * c + (size_t)h * vd) * N;
        for (int n = 0; n < N; ++n) {
          float m = -INFINITY;
          for (int j = 0; j < N; ++j) {
            float s = 0.f;
            for (int d = 0; d < kd; ++d) s += q[(size_t)d * N + n] * k[(size_t)d * N + j];
            s *= scale;
            srow[j] = s;
            if (s > m) m = s;
          }
          double l = 0.0;
          for (int j = 0; j < N; ++j) { srow[j] = expf(srow[j] - m); l += srow[j]; }
          const float inv = (float)(1.0 / l);
          for (int d = 0; d < vd; ++d) {
            double acc = 0.0;
            const float* vr = v + (size_t)d * N;
            for (int j = 0; j < N; ++j) acc += (double)srow[j] * vr[j];
            o[(size_t)d * N + n] = (float)acc * inv;
          }
        }
      }
    free(srow);
  }
}

/* ------------------------------------------------------------------------ */
/* Detect decode, grid-unit anchors, [B,4,A] layout:                          */
/* kernels/detect_decode.rs:36-86.  x1 = ax - l, x2 = ax + r, ...;            */
/* cx = (x1+x2)*0.5*s, cy likewise, w = (x2-x1)*s, h = (y2-y1)*s.            */
/* ------------------------------------------------------------------------ */
void orc_detect_decode_grid(const float* boxes, const float* ax, const float* ay, const float* st,
                            int B, int A, float* out) {
  for (int b = 0; b < B; ++b)
    for (int a = 0; a < A; ++a) {
      const float* bb = boxes + (size_t)b * 4 * A;
      float* o = out + (size_t)b * 4 * A;
      const float x1 = ax[a] - bb[a], y1 = ay[a] - bb[A + a];
      const float x2 = ax[a] + bb[2 * A + a], y2 = ay[a] + bb[3 * A + a];
      o[a] = (x1 + x2) * 0.5f * st[a];
      o[A + a] = (y1 + y2) * 0.5f * st[a];
      o[2 * A + a] = (x2 - x1) * st[a];
      o[3 * A + a] = (y2 - y1) * st[a];
    }
}

/* ------------------------------------------------------------------------ */
/* Detect post-process on the raw head outputs (A12).                         */
/* Layout: boxes[b] = per scale block [4][A_s]; scores[b] = per scale block   */
/* [nc][A_s] (blocks/detect.rs:62-80; offsets examples/yolo26.rs:1423-1447).  */
/* Per anchor (examples/yolo26.rs:1488-1529):                                 */
/*   anchor centre (gx+0.5)*s (loss/anchor.rs:47-66)                          */
/*   xywh = (cx + s*(r-l)*0.5, cy + s*(b-t)*0.5, s*(l+r), s*(t+b))            */
/*   score/class = max_by over c of sigmoid(logit_c): on ties (and NaN, which  */
/*     compares Equal) the LAST class wins                                     */
/*   keep score >= thr; stable sort by score descending (anchor order kept    */
/*     among equal scores); keep the first max_det.                            */
/* Outputs per image: count[b], and max_det rows of score, class, anchor,     */
/* xywh[4].                                                                    */
/* ------------------------------------------------------------------------ */
typedef struct { float score; int cls; int anchor; } orc_cand;

static int orc_cand_cmp(const void* pa, const void* pb) {
  const orc_cand* a = (const orc_cand*)pa;
  const orc_cand* b = (const orc_cand*)pb;
  if (a->score > b->score) return -1;
  if (a->score < b->score) return 1;
  return (a->anchor > b->anchor) - (a->anchor < b->anchor);
}

void orc_detect_postprocess(const float* boxes, const float* scores, int B, int nc,
                            int img_h, int img_w, const int* strides, int nscales,
                            float thr, int max_det,
                            int* count, float* out_score, int* out_cls, int* out_anchor,
                            float* out_xywh) {
  int a_s[8], fw[8], a_base[9];
  a_base[0] = 0;
  for (int s = 0; s < nscales; ++s) {
    fw[s] = img_w / strides[s];
    a_s[s] = (img_h / strides[s]) * fw[s];
    a_base[s + 1] = a_base[s] + a_s[s];
  }
  const int A = a_base[nscales];
#pragma omp parallel for schedule(dynamic, 1)
  for (int b = 0; b < B; ++b) {
    const float* bx = boxes + (size_t)b * 4 * A;
    const float* sc = scores + (size_t)b * nc * A;
    orc_cand* cands = (orc_cand*)malloc(sizeof(orc_cand) * (size_t)A);
    float* xywh = (float*)malloc(sizeof(float) * 4 * (size_t)A);
    int n = 0;
    for (int s = 0; s < nscales; ++s) {
      const float* bb = bx + (size_t)4 * a_base[s];
      const float* ss = sc + (size_t)nc * a_base[s];
      const float st = (float)strides[s];
      for (int j = 0; j < a_s[s]; ++j) {
        const int ai = a_base[s] + j;
        const float l = bb[j], t = bb[a_s[s] + j], r = bb[2 * a_s[s] + j], bo = bb[3 * a_s[s] + j];
        const float cx = ((float)(j % fw[s]) + 0.5f) * st;
        const float cy = ((float)(j / fw[s]) + 0.5f) * st;
        xywh[4 * ai + 0] = cx + st * (r - l) * 0.5f;
        xywh[4 * ai + 1] = cy + st * (bo - t) * 0.5f;
        xywh[4 * ai + 2] = st * (l + r);
        xywh[4 * ai + 3] = st * (t + bo);
        float best = 1.f / (1.f + expf(-ss[j]));
        int bc = 0;
        for (int c = 1; c < nc; ++c) {
          const float v = 1.f / (1.f + expf(-ss[(size_t)c * a_s[s] + j]));
          if (!(best > v)) { best = v; bc = c; }  /* Rust max_by: keep old only if Greater */
        }
        if (best >= thr) { cands[n].score = best; cands[n].cls = bc; cands[n].anchor = ai; ++n; }
      }
    }
    qsort(cands, (size_t)n, sizeof(orc_cand), orc_cand_cmp);
    const int keep = n < max_det ? n : max_det;
    count[b] = keep;
    for (int i = 0; i < max_det; ++i) {
      const size_t o = (size_t)b * max_det + i;
      if (i < keep) {
        out_score[o] = cands[i].score;
        out_cls[o] = cands[i].cls;
        out_anchor[o] = cands[i].anchor;
        for (int q = 0; q < 4; ++q) out_xywh[4 * o + q] = xywh[4 * cands[i].anchor + q];
      } else {
        out_score[o] = 0.f; out_cls[o] = -1; out_anchor[o] = -1;
        for (int q = 0; q < 4; ++q) out_xywh[4 * o + q] = 0.f;
      }
    }
    free(cands);
    free(xywh);
  }
}

/* ------------------------------------------------------------------------ */
/* Multi-scale deformable attention (no reference function; BASELINE config  */
/* 4 + the published Deformable-DETR formulation).                           */
/* value [B, S, heads, Dh]; shapes [L][2] = (H_l, W_l); starts[L];            */
/* ref [B, Q, 2] (x, y) in [0,1]; off [B, Q, heads, L, P, 2];                 */
/* attw [B, Q, heads, L, P] (already softmaxed); out [B, Q, heads*Dh].        */
/* loc = ref + off; bilinear sample at (loc_x*W_l - 0.5, loc_y*H_l - 0.5),    */
/* zero outside (grid_sample bilinear, zeros, align_corners=False).           */
/* ------------------------------------------------------------------------ */
void orc_msda(const float* value, int B, int S, int heads, int Dh, int L, const int* shapes,
              const int* starts, const float* ref, const float* off, const float* attw,
              int Q, int P, float* out) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int q = 0; q < Q; ++q) {
      const float rx = ref[((size_t)b * Q + q) * 2 + 0];
      const float ry = ref[((size_t)b * Q + q) * 2 + 1];
      for (int h = 0; h < heads; ++h) {
        double acc[256];
        for (int d = 0; d < Dh; ++d) acc[d] = 0.0;
        for (int l = 0; l < L; ++l) {
          const int Hl = shapes[2 * l], Wl = shapes[2 * l + 1];
          for (int p = 0; p < P; ++p) {
            const size_t oi = ((((size_t)b * Q + q) * heads + h) * L + l) * P + p;
            const float lx = rx + off[2 * oi + 0];
            const float ly = ry + off[2 * oi + 1];
            const float a = attw[oi];
            const float ix = lx * (float)Wl - 0.5f;
            const float iy = ly * (float)Hl - 0.5f;
            const float fx0 = floorf(ix), fy0 = floorf(iy);
            const int x0 = (int)fx0, y0 = (int)fy0;
            const float wx1 = ix - fx0, wy1 = iy - fy0;
            const float wx0 = 1.f - wx1, wy0 = 1.f - wy1;
            const int xs[2] = {x0, x0 + 1}, ys[2] = {y0, y0 + 1};
            const float wxs[2] = {wx0, wx1}, wys[2] = {wy0, wy1};
            for (int cy = 0; cy < 2; ++cy)
              for (int cx = 0; cx < 2; ++cx) {
                const int xx = xs[cx], yy = ys[cy];
                if (xx < 0 || xx >= Wl || yy < 0 || yy >= Hl) continue;
                const float wgt = wxs[cx] * wys[cy] * a;
                const float* v = value + (((size_t)b * S + starts[l] + (size_t)yy * Wl + xx) * heads + h) * Dh;
                for (int d = 0; d < Dh; ++d) acc[d] += (double)wgt * v[d];
              }
          }
        }
        float* o = out + ((size_t)b * Q + q) * heads * Dh + (size_t)h * Dh;
        for (int d = 0; d < Dh; ++d) o[d] = (float)acc[d];
      }
    }
}

/* Elementwise add (teeny-kernels ElemwiseAddForward, tests/test_c2psa_cuda.rs:350-356) */
void orc_add(const float* a, const float* b, float* y, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) y[i] = a[i] + b[i];
}

/* Un-letterbox (examples/yolo26.rs:1531-1547), float32 throughout:
 * lb_scale = img / max(w, h); new = round(o * lb_scale) (f32::round: half away
 * from zero); pad = (img - new) / 2 in integers; scale_o = o * lb_scale;
 * cx_n = (cx - pad_x) / scale_x, cy_n likewise, w_n = w / scale_x,
 * h_n = h / scale_y.  Slots past count[b] are zero. */
void orc_detect_unletterbox(int B, int max_det, int img_size, const int* orig_wh, const int* count,
                            const float* xywh, float* out) {
  for (int b = 0; b < B; ++b) {
    const int ow = orig_wh[2 * b], oh = orig_wh[2 * b + 1];
    const float s = (float)img_size / (float)(ow > oh ? ow : oh);
    const int nw = (int)roundf((float)ow * s), nh = (int)roundf((float)oh * s);
    const float px = (float)(img_size > nw ? (img_size - nw) / 2 : 0);
    const float py = (float)(img_size > nh ? (img_size - nh) / 2 : 0);
    const float sx = (float)ow * s, sy = (float)oh * s;
    for (int k = 0; k < max_det; ++k) {
      const float* d = xywh + ((size_t)b * max_det + k) * 4;
      float* o = out + ((size_t)b * max_det + k) * 4;
      if (k >= count[b]) {
        o[0] = o[1] = o[2] = o[3] = 0.f;
        continue;
      }
      o[0] = (d[0] - px) / sx;
      o[1] = (d[1] - py) / sy;
      o[2] = d[2] / sx;
      o[3] = d[3] / sy;
    }
  }
}

/* Letterbox, preprocess_image_raw (examples/yolo26.rs:1229-1253): scale =
 * img / max(w, h) in f64, new = round(dim * scale) (half away from zero),
 * image::imageops::resize(img, new_w, new_h, FilterType::Triangle), centred at
 * ((img - new_w) / 2, (img - new_h) / 2) on a 114/255 canvas, NCHW u8 / 255.
 * The resize is the image crate's (0.25.10, Cargo.lock:2807-2810; the crate is
 * not vendored), restated from its published imageops::sample:
 *   resize: same size -> copy; else tmp = vertical_sample(img, new_h) (float32
 *     buffer [new_h][w]), out = horizontal_sample(tmp, new_w);
 *   each pass, per output index o: ratio = src / dst (f32), sratio = max(ratio,
 *     1), support = 1 * sratio (triangle support 1), centre = (o + 0.5) *
 *     ratio, left = clamp(floor(centre - support), 0, src - 1), right =
 *     clamp(ceil(centre + support), left + 1, src), weights w_i =
 *     tri((i - (centre - 0.5)) / sratio) for i in [left, right), each divided
 *     by their running float32 sum; t = sum_i p_i * w_i in order;
 *   horizontal_sample clamps t to [0, 255] and rounds half away from zero.
 * Separate multiplies and adds (no FMA), as Rust evaluates them.
 * resized (optional): the [new_h][new_w][3] float32 values before rounding. */
static float orc_tri(float x) {
  const float a = fabsf(x);
  return a < 1.0f ? 1.0f - a : 0.0f;
}
static int orc_resample_weights(int o, int src, int dst, float* w, int* first) {
  const float ratio = (float)src / (float)dst;
  const float sratio = ratio < 1.0f ? 1.0f : ratio;
  const float support = 1.0f * sratio;
  const float centre = ((float)o + 0.5f) * ratio;
  long left = (long)floorf(centre - support);
  left = left < 0 ? 0 : (left > src - 1 ? src - 1 : left);
  long right = (long)ceilf(centre + support);
  right = right < left + 1 ? left + 1 : (right > src ? src : right);
  const float c = centre - 0.5f;
  float sum = 0.0f;
  for (long i = left; i < right; ++i) {
    w[i - left] = orc_tri(((float)i - c) / sratio);
    sum += w[i - left];
  }
  for (long i = left; i < right; ++i) w[i - left] /= sum;
  *first = (int)left;
  return (int)(right - left);
}
void orc_letterbox(const uint8_t* rgb, int w, int h, int img_size, float* out, float* resized, int* new_wh) {
  const double scale = (double)img_size / (double)(w > h ? w : h);
  const int nw = (int)round((double)w * scale), nh = (int)round((double)h * scale);
  const int pad_x = (img_size - nw) / 2, pad_y = (img_size - nh) / 2;
  new_wh[0] = nw;
  new_wh[1] = nh;
  float* res = (float*)malloc(sizeof(float) * 3 * ((size_t)nw * nh + 1));
  if (nw == w && nh == h) {
    for (long i = 0; i < (long)w * h * 3; ++i) res[i] = (float)rgb[i];
  } else {
    const int maxt = 2 * (w > h ? w : h) + 4;
    float* wts = (float*)malloc(sizeof(float) * maxt);
    float* tmp = (float*)malloc(sizeof(float) * 3 * ((size_t)nh * w + 1));
    for (int oy = 0; oy < nh; ++oy) {  /* vertical_sample */
      int top;
      const int n = orc_resample_weights(oy, h, nh, wts, &top);
      for (int x = 0; x < w; ++x) {
        float t[3] = {0.0f, 0.0f, 0.0f};
        for (int j = 0; j < n; ++j)
          for (int c = 0; c < 3; ++c) t[c] += (float)rgb[((size_t)(top + j) * w + x) * 3 + c] * wts[j];
        for (int c = 0; c < 3; ++c) tmp[((size_t)oy * w + x) * 3 + c] = t[c];
      }
    }
    for (int ox = 0; ox < nw; ++ox) {  /* horizontal_sample */
      int left;
      const int n = orc_resample_weights(ox, w, nw, wts, &left);
      for (int y = 0; y < nh; ++y) {
        float t[3] = {0.0f, 0.0f, 0.0f};
        for (int i = 0; i < n; ++i)
          for (int c = 0; c < 3; ++c) t[c] += tmp[((size_t)y * w + left + i) * 3 + c] * wts[i];
        for (int c = 0; c < 3; ++c) res[((size_t)y * nw + ox) * 3 + c] = t[c];
      }
    }
    free(tmp);
    free(wts);
  }
  if (resized) memcpy(resized, res, sizeof(float) * 3 * (size_t)nw * nh);
  const float pad = 114.0f / 255.0f;
  const size_t plane = (size_t)img_size * img_size;
  for (size_t i = 0; i < 3 * plane; ++i) out[i] = pad;
  for (int y = 0; y < nh; ++y)
    for (int x = 0; x < nw; ++x)
      for (int c = 0; c < 3; ++c) {
        float v = res[((size_t)y * nw + x) * 3 + c];
        v = v < 0.0f ? 0.0f : (v > 255.0f ? 255.0f : v);
        const uint8_t u = (uint8_t)roundf(v);
        out[c * plane + (size_t)(pad_y + y) * img_size + pad_x + x] = (float)u / 255.0f;
      }
  free(res);
}

// Detect-head post-processing on gfx950.
//
// Stage 1 (one thread per anchor): LTRB -> xywh decode, sigmoid per class,
// argmax, threshold -- the host loops of examples/yolo26.rs:1488-1528 with
// the anchor grid of loss/anchor.rs:47-66.  The argmax follows Rust's
// Iterator::max_by with partial_cmp().unwrap_or(Equal): the running best is
// kept only if it compares Greater, so the last of equal maxima wins and a
// NaN compares Equal.  A kept anchor gets the unique 64-bit key
// (score_bits << 32) | (0xffffffff - anchor): ordering keys descending is the
// stable descending sort of examples/yolo26.rs:1529 (equal scores keep
// ascending anchor order); sigmoid scores are non-negative so their IEEE bits
// order like the values.
//
// Stage 2 (one workgroup per image): exact top-k (k = min(count, max_det)).
// With at most TOPK_MAX kept anchors every key is gathered into LDS and
// bitonic-sorted.  Otherwise a most-significant-digit radix select raises a
// threshold 8 bits at a time and stops as soon as the keys at or above it
// fit the LDS buffer (at the latest after the 8th digit, when the threshold
// is the k-th largest key itself); those keys are gathered and sorted.
#include "common.h"

extern "C" __global__ __launch_bounds__(256) void vrs_detect_stage1(vrs_det1_args a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.B * a.A) return;
  const int b = (int)(i / a.A), ai = (int)(i - (int64_t)b * a.A);
  int s = 0;
  while (s + 1 < a.nscales && ai >= a.a_base[s + 1]) ++s;
  const int as = (s + 1 < a.nscales ? a.a_base[s + 1] : a.A) - a.a_base[s];
  const int j = ai - a.a_base[s];
  const float st = a.stride[s];
  const float* bb = a.boxes + (int64_t)b * 4 * a.A + 4 * (int64_t)a.a_base[s];
  const float l = bb[j], t = bb[as + j], r = bb[2 * as + j], bo = bb[3 * as + j];
  const float cx = ((float)(j % a.fw[s]) + 0.5f) * st;
  const float cy = ((float)(j / a.fw[s]) + 0.5f) * st;
  float* xy = a.xywh + i * 4;
  xy[0] = cx + st * (r - l) * 0.5f;
  xy[1] = cy + st * (bo - t) * 0.5f;
  xy[2] = st * (l + r);
  xy[3] = st * (t + bo);

  const float* sc = a.scores + (int64_t)b * a.nc * a.A + (int64_t)a.nc * a.a_base[s] + j;
  float best = 1.0f / (1.0f + expf(-sc[0]));
  int bc = 0;
  for (int c = 1; c < a.nc; ++c) {
    const float v = 1.0f / (1.0f + expf(-sc[(int64_t)c * as]));
    if (!(best > v)) { best = v; bc = c; }
  }
  a.cls[i] = bc;
  a.keys[i] = (best >= a.thr) ? (((uint64_t)__float_as_uint(best)) << 32) | (uint64_t)(0xffffffffu - (uint32_t)ai)
                              : 0ull;
}

namespace {
constexpr int TOPK_MAX = 1024;
}

extern "C" __global__ __launch_bounds__(1024) void vrs_detect_stage2(vrs_det2_args a) {
  __shared__ uint32_t hist[256];
  __shared__ uint64_t sel[TOPK_MAX];
  __shared__ uint32_t s_count, s_nsel, s_digit, s_krem, s_ntop;
  const int b = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
  const uint64_t* keys = a.keys + (int64_t)b * a.A;

  if (tid == 0) { s_count = 0; s_nsel = 0; }
  __syncthreads();
  uint32_t local = 0;
  for (int i = tid; i < a.A; i += nt) local += keys[i] != 0ull;
  atomicAdd(&s_count, local);
  __syncthreads();
  const uint32_t count = s_count;
  const uint32_t k = count < (uint32_t)a.max_det ? count : (uint32_t)a.max_det;

  // gather threshold: every nonzero key when they all fit the buffer
  uint64_t thr_key = 1ull;
  if (count > (uint32_t)TOPK_MAX && k > 0) {
    uint64_t prefix = 0, pmask = 0;
    if (tid == 0) s_krem = k;
    for (int shift = 56; shift >= 0; shift -= 8) {
      for (int i = tid; i < 256; i += nt) hist[i] = 0;
      __syncthreads();
      for (int i = tid; i < a.A; i += nt) {
        const uint64_t key = keys[i];
        if (key != 0ull && (key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        uint32_t cum = 0, krem = s_krem;
        int d = 255;
        for (; d > 0; --d) {
          if (cum + hist[d] >= krem) break;
          cum += hist[d];
        }
        s_digit = (uint32_t)d;
        s_krem = krem - cum;
        // keys whose digits so far are >= the new prefix: above it at the
        // earlier digits (k - krem), in the higher bins of this one (cum),
        // and in bin d
        s_ntop = (k - krem) + cum + hist[d];
      }
      __syncthreads();
      prefix |= ((uint64_t)s_digit) << shift;
      pmask |= 255ull << shift;
      const bool fits = s_ntop <= (uint32_t)TOPK_MAX;
      __syncthreads();
      if (fits) break;
    }
    // lower bits zero: the keys >= prefix are exactly those counted in s_ntop,
    // and they include the k largest
    thr_key = prefix;
  }

  for (int i = tid; i < TOPK_MAX; i += nt) sel[i] = 0ull;
  __syncthreads();
  if (k > 0)
    for (int i = tid; i < a.A; i += nt) {
      const uint64_t key = keys[i];
      if (key != 0ull && key >= thr_key) {
        const uint32_t slot = atomicAdd(&s_nsel, 1u);
        if (slot < (uint32_t)TOPK_MAX) sel[slot] = key;
      }
    }
  __syncthreads();
  // sort the smallest power of two of slots holding every gathered key
  const uint32_t nsel = s_nsel < (uint32_t)TOPK_MAX ? s_nsel : (uint32_t)TOPK_MAX;
  int P = 2;
  while ((uint32_t)P < nsel) P <<= 1;

  // bitonic sort, descending, over P slots (zeros sink to the end)
  for (int size = 2; size <= P; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < P; i += nt) {
        const int j = i ^ stride;
        if (j > i) {
          const bool desc = (i & size) == 0;
          const uint64_t x = sel[i], y = sel[j];
          if (desc ? (x < y) : (x > y)) { sel[i] = y; sel[j] = x; }
        }
      }
      __syncthreads();
    }

  if (tid == 0) a.count[b] = (int32_t)k;
  for (int i = tid; i < a.max_det; i += nt) {
    const int64_t o = (int64_t)b * a.max_det + i;
    if ((uint32_t)i < k) {
      const uint64_t key = sel[i];
      const int anchor = (int)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
      a.out_score[o] = __uint_as_float((uint32_t)(key >> 32));
      a.out_anchor[o] = anchor;
      a.out_cls[o] = a.cls[(int64_t)b * a.A + anchor];
      const float* xy = a.xywh + ((int64_t)b * a.A + anchor) * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) a.out_xywh[o * 4 + q] = xy[q];
    } else {
      a.out_score[o] = 0.f;
      a.out_anchor[o] = -1;
      a.out_cls[o] = -1;
#pragma unroll
      for (int q = 0; q < 4; ++q) a.out_xywh[o * 4 + q] = 0.f;
    }
  }
}

// Letterbox pixels -> [cx, cy, w, h] normalised to the original image, the
// reference's un-letterbox (examples/yolo26.rs:1531-1547) in the same float32
// operations: s = img / max(ow, oh); new = round(o * s) (half away from
// zero); pad = (img - new) / 2 in integers; divide by o * s.  One thread per
// detection slot; slots past count[b] are zeroed.
extern "C" __global__ __launch_bounds__(256) void vrs_detect_unletterbox(vrs_unlb_args a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.B * a.max_det) return;
  const int b = (int)(i / a.max_det), k = (int)(i - (int64_t)b * a.max_det);
  float* o = a.out + i * 4;
  if (k >= a.count[b]) {
    o[0] = o[1] = o[2] = o[3] = 0.f;
    return;
  }
  const int ow = a.orig_wh[2 * b], oh = a.orig_wh[2 * b + 1];
  const float s = (float)a.img_size / (float)(ow > oh ? ow : oh);
  const int nw = (int)roundf((float)ow * s), nh = (int)roundf((float)oh * s);
  const float px = (float)(a.img_size > nw ? (a.img_size - nw) / 2 : 0);
  const float py = (float)(a.img_size > nh ? (a.img_size - nh) / 2 : 0);
  const float sx = (float)ow * s, sy = (float)oh * s;
  const float* d = a.xywh + i * 4;
  o[0] = (d[0] - px) / sx;
  o[1] = (d[1] - py) / sy;
  o[2] = d[2] / sx;
  o[3] = d[3] / sy;
}

// ---- letterbox preprocessing (examples/yolo26.rs:1229-1253) ---------------
// preprocess_image_raw resizes with image 0.25.10 imageops::resize(...,
// FilterType::Triangle): a vertical pass over the source columns into float32
// (weights normalised per output row), then a horizontal pass over that
// buffer (normalised per output column), clamped to [0, 255] and rounded half
// away from zero to u8; the canvas holds u8 / 255 inside the resized region
// and 114 / 255 elsewhere.  Per axis, output index o of a dst-long axis from a
// src-long one: ratio = src / dst, sr = max(ratio, 1), centre = (o + 0.5) *
// ratio, taps i in [clamp(floor(centre - sr), 0, src - 1), clamp(ceil(centre
// + sr), lo + 1, src)), weight tri((i - (centre - 0.5)) / sr) / sum, tri(x) =
// max(0, 1 - |x|).  The kernel fuses both passes per output pixel with the
// same float32 operations in the same order (vertical sum over a column's
// taps, then the horizontal sum over columns), so it reproduces the two-pass
// result bit for bit; contraction into FMA is off as in the reference.
namespace {
__device__ inline float lb_tri(float x) {
  const float a = fabsf(x);
  return a < 1.0f ? 1.0f - a : 0.0f;
}
// Window [lo, lo + n) of output index o along a dst-long axis from a
// src-long one, with its normalised weights written to w[0..n) (n <= cap; the
// host's ratio bounds keep the true window within cap).  One division per tap
// for the weight and one for the normalisation, as the reference does them.
__device__ inline int lb_window(int o, int src, int dst, int cap, float* w, int& lo) {
#pragma clang fp contract(off)
  const float ratio = (float)src / (float)dst;
  const float sr = ratio < 1.0f ? 1.0f : ratio;  // support 1 x sratio
  const float centre = ((float)o + 0.5f) * ratio;
  int l = (int)floorf(centre - sr);
  l = l < 0 ? 0 : (l > src - 1 ? src - 1 : l);
  int h = (int)ceilf(centre + sr);
  h = h < l + 1 ? l + 1 : (h > src ? src : h);
  if (h - l > cap) h = l + cap;
  const float c = centre - 0.5f;
  float sum = 0.0f;
  for (int i = l; i < h; ++i) {
    const float v = lb_tri(((float)i - c) / sr);
    w[i - l] = v;
    sum += v;
  }
  for (int i = 0; i < h - l; ++i) w[i] = w[i] / sum;
  lo = l;
  return h - l;
}
__device__ inline float lb_quant(float v) {  // clamp, round half away from zero, / 255
  v = v < 0.0f ? 0.0f : (v > 255.0f ? 255.0f : v);
  return roundf(v) / 255.0f;
}
constexpr int LB_TW = 64, LB_TH = 4, LB_LD = VRS_LB_MAX_TAPS + 1;  // odd row pitch: no bank conflicts
}  // namespace

// One workgroup per 64 x 4 tile of one image's canvas (grid.y = image).  The
// 64 column and 4 row windows of the tile are computed once into LDS; each
// thread then sums its pixel's window from the RGB8 source (all three
// channels per tap) and writes the three NCHW planes.
extern "C" __global__ __launch_bounds__(256) void vrs_letterbox_f32(vrs_lb_args a) {
#pragma clang fp contract(off)
  __shared__ float wcol[LB_TW * LB_LD];
  __shared__ float wrow[LB_TH * LB_LD];
  __shared__ int gcol[LB_TW][2], grow[LB_TH][2];
  const vrs_lb_image im = a.img[blockIdx.y];
  const int tiles_x = (a.S + LB_TW - 1) / LB_TW;
  const int x0 = (int)(blockIdx.x % tiles_x) * LB_TW, y0 = (int)(blockIdx.x / tiles_x) * LB_TH;
  const int tx = threadIdx.x % LB_TW, ty = threadIdx.x / LB_TW;
  // does the tile meet the resized region? (uniform over the workgroup)
  const bool inside = x0 < im.px + im.nw && x0 + LB_TW > im.px && y0 < im.py + im.nh && y0 + LB_TH > im.py;
  if (inside) {
    const int t = threadIdx.x;
    if (t < LB_TW) {
      const int p = x0 + t - im.px;
      if (p >= 0 && p < im.nw) {
        int lo;
        const int n = lb_window(p, im.w, im.nw, VRS_LB_MAX_TAPS, wcol + t * LB_LD, lo);
        gcol[t][0] = lo;
        gcol[t][1] = lo + n;
      }
    } else if (t < LB_TW + LB_TH) {
      const int r = t - LB_TW, p = y0 + r - im.py;
      if (p >= 0 && p < im.nh) {
        int lo;
        const int n = lb_window(p, im.h, im.nh, VRS_LB_MAX_TAPS, wrow + r * LB_LD, lo);
        grow[r][0] = lo;
        grow[r][1] = lo + n;
      }
    }
    __syncthreads();
  }
  const int ox = x0 + tx, oy = y0 + ty;
  if (ox >= a.S || oy >= a.S) return;
  const int64_t plane = (int64_t)a.S * a.S;
  float* o = a.out + (int64_t)im.slot * 3 * plane + (int64_t)oy * a.S + ox;
  const int px = ox - im.px, py = oy - im.py;
  if (!inside || px < 0 || px >= im.nw || py < 0 || py >= im.nh) {
    o[0] = a.pad;
    o[plane] = a.pad;
    o[2 * plane] = a.pad;
    return;
  }
  const int lo = gcol[tx][0], hi = gcol[tx][1], top = grow[ty][0], bot = grow[ty][1];
  const int64_t row = (int64_t)im.w * 3;
  const uint8_t* src = a.rgb + im.off + (int64_t)top * row;
  const float* wy = wrow + ty * LB_LD;
  const float* wx = wcol + tx * LB_LD;
  float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f;
  const int n = bot - top;
  for (int i = lo; i < hi; ++i) {
    const uint8_t* p = src + (int64_t)i * 3;
    float t0 = 0.0f, t1 = 0.0f, t2 = 0.0f;
    for (int j0 = 0; j0 < n; j0 += 8) {   // 8 taps' bytes in flight, then the sums in order
      uint8_t q[8][3];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j0 + j < n) {
          const uint8_t* pj = p + (int64_t)(j0 + j) * row;
          q[j][0] = pj[0];
          q[j][1] = pj[1];
          q[j][2] = pj[2];
        }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j0 + j < n) {
          const float w = wy[j0 + j];
          t0 += (float)q[j][0] * w;
          t1 += (float)q[j][1] * w;
          t2 += (float)q[j][2] * w;
        }
    }
    const float w = wx[i - lo];
    s0 += t0 * w;
    s1 += t1 * w;
    s2 += t2 * w;
  }
  o[0] = lb_quant(s0);
  o[plane] = lb_quant(s1);
  o[2 * plane] = lb_quant(s2);
}

// Staged variants for images shrunk at most 2x (vrs_letterbox_f32_s2), 4x
// (_s4) or VRS_LB_STAGED_RATIO = 8x (_s8) per axis: one workgroup per 64 x 4
// tile (32 x 4 for _s8).  After the
// windows, the source patch the tile reads (rows spanned by its 4 row windows
// x columns spanned by its 64 column windows) is copied into LDS with aligned
// dword loads, all in flight together; the vertical pass then runs once per
// (tile row, source column) from LDS into a float32 buffer, and the
// horizontal pass reads that buffer -- the same float32 operations in the same
// order as the direct kernel and the two-pass reference.  The patch is copied
// in 16-byte loads so that a workgroup keeps its whole patch in flight at
// once (the kernel is bound by loads in flight, not by bandwidth).
namespace {
// R: the largest shrink factor per axis the instance accepts; LDS is sized
// for it, so the small-ratio instance fits twice as many workgroups per CU
template <int R, int LBS_TW>
__device__ __forceinline__ void lb_staged(const vrs_lb_args& a) {
#pragma clang fp contract(off)
  constexpr int LBS_TH = 4, NT = LBS_TW * LBS_TH, LBS_TAPS = 2 * R + 2, LBS_LD = LBS_TAPS + 1;
  // source columns / rows a tile touches: (n - 1) * ratio + 2 * ratio + 2, +2 slack
  constexpr int LBS_CMAX = (LBS_TW - 1) * R + 2 * R + 4;
  constexpr int LBS_RMAX = (LBS_TH - 1) * R + 2 * R + 4;
  constexpr int LBS_PW = (LBS_CMAX * 3 + 15 + 15) / 16;   // 16-byte chunks per patch row (15-byte lead-in)
  constexpr int LBS_VREG = 4;                               // chunks in flight per thread and round
  __shared__ float wcol[LBS_TW * LBS_LD];
  __shared__ float wrow[LBS_TH * LBS_LD];
  __shared__ int gcol[LBS_TW][2], grow[LBS_TH][2];
  __shared__ u32x4_t patch[LBS_RMAX * LBS_PW];
  __shared__ int plead[LBS_RMAX];
  __shared__ float vbuf[LBS_TH * LBS_CMAX * 3];
  const vrs_lb_image im = a.img[blockIdx.y];
  const int tiles_x = (a.S + LBS_TW - 1) / LBS_TW;
  const int x0 = (int)(blockIdx.x % tiles_x) * LBS_TW, y0 = (int)(blockIdx.x / tiles_x) * LBS_TH;
  const int64_t plane = (int64_t)a.S * a.S;
  float* ob = a.out + (int64_t)im.slot * 3 * plane;
  const int t = threadIdx.x;
  const int tx = t % LBS_TW, ty = t / LBS_TW;
  const int ox = x0 + tx, oy = y0 + ty;
  // in-image columns [cf, cl] and rows [rf, rl] of the tile (uniform)
  const int cf = max(im.px - x0, 0), cl = min(im.px + im.nw - x0, LBS_TW) - 1;
  const int rf = max(im.py - y0, 0), rl = min(im.py + im.nh - y0, LBS_TH) - 1;
  if (cf > cl || rf > rl) {   // all padding
    if (ox < a.S && oy < a.S) {
      float* o = ob + (int64_t)oy * a.S + ox;
      o[0] = a.pad;
      o[plane] = a.pad;
      o[2 * plane] = a.pad;
    }
    return;
  }
  if (t < LBS_TW) {
    if (t >= cf && t <= cl) {
      int lo;
      const int n = lb_window(x0 + t - im.px, im.w, im.nw, LBS_TAPS, wcol + t * LBS_LD, lo);
      gcol[t][0] = lo;
      gcol[t][1] = lo + n;
    }
  } else if (t < LBS_TW + LBS_TH) {
    const int r = t - LBS_TW;
    if (r >= rf && r <= rl) {
      int lo;
      const int n = lb_window(y0 + r - im.py, im.h, im.nh, LBS_TAPS, wrow + r * LBS_LD, lo);
      grow[r][0] = lo;
      grow[r][1] = lo + n;
    }
  }
  __syncthreads();
  // window bounds are non-decreasing along an axis: the patch is source rows
  // [top of the first row window, bottom of the last) x columns [lo of the
  // first column window, hi of the last)
  const int c_lo = gcol[cf][0];
  const int ncol = min(gcol[cl][1] - c_lo, LBS_CMAX);   // <= LBS_CMAX and LBS_RMAX by the ratio bound
  const int ytop = grow[rf][0];
  const int nrow = min(grow[rl][1] - ytop, LBS_RMAX);
  // patch row i holds the source bytes [s_i, s_i + 3*ncol) of image row
  // ytop + i (s_i = off + ((ytop + i)*w + c_lo)*3), copied as the 16-byte
  // aligned chunks that cover them; the bytes start at plead[i] = address of
  // s_i mod 16.  Chunks straddling the image's first or last byte (only
  // those) are assembled from byte loads.
  const unsigned char* img0 = a.rgb + im.off;
  const unsigned char* img1 = img0 + (int64_t)im.w * im.h * 3;
  const int nq = (3 * ncol + 15 + 15) / 16;   // chunks per row copy (<= LBS_PW)
  const int total = nrow * nq;
  if (t < nrow)
    plead[t] = (int)(reinterpret_cast<uintptr_t>(img0 + ((int64_t)(ytop + t) * im.w + c_lo) * 3) & 15);
  for (int base = t; base < total; base += NT * LBS_VREG) {
    u32x4_t v[LBS_VREG];
#pragma unroll
    for (int u = 0; u < LBS_VREG; ++u) {
      const int idx = base + u * NT;
      if (idx < total) {
        const int i = idx / nq, d = idx - (idx / nq) * nq;
        const unsigned char* row_p = img0 + ((int64_t)(ytop + i) * im.w + c_lo) * 3;
        const unsigned char* q = reinterpret_cast<const unsigned char*>(
            (reinterpret_cast<uintptr_t>(row_p) & ~(uintptr_t)15) + 16 * (uintptr_t)d);
        if (q >= img0 && q + 16 <= img1) {
          v[u] = *reinterpret_cast<const u32x4_t*>(q);
        } else {
          uint32_t wv[4] = {0, 0, 0, 0};
          for (int k = 0; k < 16; ++k)
            if (q + k >= img0 && q + k < img1) wv[k / 4] |= (uint32_t)q[k] << (8 * (k % 4));
          v[u] = (u32x4_t){wv[0], wv[1], wv[2], wv[3]};
        }
      }
    }
#pragma unroll
    for (int u = 0; u < LBS_VREG; ++u) {
      const int idx = base + u * NT;
      if (idx < total) patch[(idx / nq) * LBS_PW + idx % nq] = v[u];
    }
  }
  __syncthreads();
  // vertical pass: one (tile row, patch column) per thread and step; the row
  // loop is uniform over the workgroup
  const unsigned char* pb = reinterpret_cast<const unsigned char*>(patch);
  for (int r = rf; r <= rl; ++r) {
    const int top = grow[r][0], n = grow[r][1] - top;
    const float* wy = wrow + r * LBS_LD;
    for (int x = t; x < ncol; x += NT) {
      float t0 = 0.0f, t1 = 0.0f, t2 = 0.0f;
      for (int j = 0; j < n; ++j) {
        const int i = top - ytop + j;
        const unsigned char* q = pb + i * LBS_PW * 16 + plead[i] + x * 3;
        const float w = wy[j];
        t0 += (float)q[0] * w;
        t1 += (float)q[1] * w;
        t2 += (float)q[2] * w;
      }
      float* vv = vbuf + (r * LBS_CMAX + x) * 3;
      vv[0] = t0;
      vv[1] = t1;
      vv[2] = t2;
    }
  }
  __syncthreads();
  // horizontal pass, one pixel per thread
  if (ox >= a.S || oy >= a.S) return;
  float* o = ob + (int64_t)oy * a.S + ox;
  if (tx < cf || tx > cl || ty < rf || ty > rl) {
    o[0] = a.pad;
    o[plane] = a.pad;
    o[2 * plane] = a.pad;
    return;
  }
  const int lo = gcol[tx][0], n = min(gcol[tx][1], c_lo + ncol) - lo;
  const float* vv = vbuf + (ty * LBS_CMAX + lo - c_lo) * 3;
  const float* wx = wcol + tx * LBS_LD;
  float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f;
  for (int i = 0; i < n; ++i) {
    const float w = wx[i];
    s0 += vv[3 * i] * w;
    s1 += vv[3 * i + 1] * w;
    s2 += vv[3 * i + 2] * w;
  }
  o[0] = lb_quant(s0);
  o[plane] = lb_quant(s1);
  o[2 * plane] = lb_quant(s2);
}
}  // namespace

extern "C" __global__ __launch_bounds__(256) void vrs_letterbox_f32_s2(vrs_lb_args a) { lb_staged<2, 64>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_letterbox_f32_s4(vrs_lb_args a) { lb_staged<4, 64>(a); }
// 32 x 4 tiles (128 threads) keep the patch of an 8x shrink within 40 KB of LDS
extern "C" __global__ __launch_bounds__(128) void vrs_letterbox_f32_s8(vrs_lb_args a) {
  lb_staged<VRS_LB_STAGED_RATIO, 32>(a);
}

// Grid-unit decode on [B,4,A] rows l,t,r,b (kernels/detect_decode.rs:36-86):
// cx = (ax - l + ax + r) * 0.5 * s, cy likewise, w = (r + l) * s, h = (b + t) * s.
extern "C" __global__ __launch_bounds__(256) void vrs_detect_decode_grid(vrs_dec_args a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.B * a.A) return;
  const int b = (int)(i / a.A), ai = (int)(i - (int64_t)b * a.A);
  const float* bx = a.boxes + (int64_t)b * 4 * a.A;
  float* o = a.out + (int64_t)b * 4 * a.A;
  const float x1 = a.ax[ai] - bx[ai], y1 = a.ay[ai] - bx[a.A + ai];
  const float x2 = a.ax[ai] + bx[2 * a.A + ai], y2 = a.ay[ai] + bx[3 * a.A + ai];
  const float s = a.st[ai];
  o[ai] = (x1 + x2) * 0.5f * s;
  o[a.A + ai] = (y1 + y2) * 0.5f * s;
  o[2 * a.A + ai] = (x2 - x1) * s;
  o[3 * a.A + ai] = (y2 - y1) * s;
}

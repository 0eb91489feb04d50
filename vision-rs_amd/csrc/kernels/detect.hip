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
// Stage 2 (one workgroup per image): exact top-k.  A most-significant-digit
// radix select over the keys finds the k-th largest key (k = min(count,
// max_det)); the keys >= it are gathered into LDS and bitonic-sorted.
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
  __shared__ uint32_t s_count, s_nsel, s_digit, s_krem;
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

  uint64_t prefix = 0, pmask = 0;
  if (tid == 0) s_krem = k;
  for (int shift = 56; shift >= 0 && k > 0; shift -= 8) {
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
    }
    __syncthreads();
    prefix |= ((uint64_t)s_digit) << shift;
    pmask |= 255ull << shift;
    __syncthreads();
  }
  const uint64_t kth = prefix;  // exact k-th largest key (keys are unique)

  for (int i = tid; i < TOPK_MAX; i += nt) sel[i] = 0ull;
  __syncthreads();
  if (k > 0)
    for (int i = tid; i < a.A; i += nt) {
      const uint64_t key = keys[i];
      if (key != 0ull && key >= kth) {
        const uint32_t slot = atomicAdd(&s_nsel, 1u);
        if (slot < (uint32_t)TOPK_MAX) sel[slot] = key;
      }
    }
  __syncthreads();

  // bitonic sort, descending, over TOPK_MAX slots (zeros sink to the end)
  for (int size = 2; size <= TOPK_MAX; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < TOPK_MAX; i += nt) {
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
struct LbAxis {
  int lo, hi;
  float c, sr, sum;
};
__device__ inline LbAxis lb_axis(int o, int src, int dst) {
#pragma clang fp contract(off)
  LbAxis ax;
  const float ratio = (float)src / (float)dst;
  ax.sr = ratio < 1.0f ? 1.0f : ratio;  // support 1 x sratio
  const float centre = ((float)o + 0.5f) * ratio;
  int lo = (int)floorf(centre - ax.sr);
  lo = lo < 0 ? 0 : (lo > src - 1 ? src - 1 : lo);
  int hi = (int)ceilf(centre + ax.sr);
  hi = hi < lo + 1 ? lo + 1 : (hi > src ? src : hi);
  // the host bounds ratio so that a window has at most VRS_LB_MAX_TAPS taps
  if (hi - lo > VRS_LB_MAX_TAPS) hi = lo + VRS_LB_MAX_TAPS;
  ax.lo = lo;
  ax.hi = hi;
  ax.c = centre - 0.5f;
  float sum = 0.0f;
  for (int i = lo; i < hi; ++i) sum += lb_tri(((float)i - ax.c) / ax.sr);
  ax.sum = sum;
  return ax;
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
        const LbAxis ax = lb_axis(p, im.w, im.nw);
        gcol[t][0] = ax.lo;
        gcol[t][1] = ax.hi;
        for (int i = ax.lo; i < ax.hi; ++i) wcol[t * LB_LD + i - ax.lo] = lb_tri(((float)i - ax.c) / ax.sr) / ax.sum;
      }
    } else if (t < LB_TW + LB_TH) {
      const int r = t - LB_TW, p = y0 + r - im.py;
      if (p >= 0 && p < im.nh) {
        const LbAxis ax = lb_axis(p, im.h, im.nh);
        grow[r][0] = ax.lo;
        grow[r][1] = ax.hi;
        for (int i = ax.lo; i < ax.hi; ++i) wrow[r * LB_LD + i - ax.lo] = lb_tri(((float)i - ax.c) / ax.sr) / ax.sum;
      }
    }
    __syncthreads();
  }
  const int ox = x0 + tx, oy = y0 + ty;
  if (ox >= a.S || oy >= a.S) return;
  const int64_t plane = (int64_t)a.S * a.S;
  float* o = a.out + (int64_t)blockIdx.y * 3 * plane + (int64_t)oy * a.S + ox;
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
  for (int i = lo; i < hi; ++i) {
    const uint8_t* p = src + (int64_t)i * 3;
    float t0 = 0.0f, t1 = 0.0f, t2 = 0.0f;
    for (int j = 0; j < bot - top; ++j, p += row) {
      const float w = wy[j];
      t0 += (float)p[0] * w;
      t1 += (float)p[1] * w;
      t2 += (float)p[2] * w;
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

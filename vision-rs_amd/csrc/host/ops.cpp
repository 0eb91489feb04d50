// Single-op C-ABI entry points (include/vrs.h): each validates, prepares the
// launch(es) and runs them on the caller's stream.
#include <cmath>
#include <cstring>

#include "vrs_internal.h"
#include <algorithm>

using namespace vrs;

namespace {

int run_all(const std::vector<Launch>& ls, void* stream) {
  for (const auto& l : ls) {
    int rc = run(l, static_cast<hipStream_t>(stream));
    if (rc) return rc;
  }
  return VRS_OK;
}

uint16_t host_f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

}  // namespace

namespace vrs {
uint8_t f32_to_e4m3(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80);
  if (std::isnan(v)) return (uint8_t)(sign | 0x7f);
  float a = std::fabs(v);
  if (a >= 448.f) return (uint8_t)(sign | 0x7e);               // saturate at 448 = 1.75 * 2^8
  if (a < 0.015625f) {                                          // below 2^-6: subnormal, step 2^-9
    const int q = (int)std::nearbyint(a * 512.f);               // 0..8; 8 is the smallest normal
    return (uint8_t)(sign | q);
  }
  int e2;
  const float f = std::frexp(a, &e2);                           // a = f * 2^e2, f in [0.5, 1)
  int e = e2 - 1;                                               // a = (1 + m) * 2^e
  int q = (int)std::nearbyint((f * 2.f - 1.f) * 8.f);           // 3 mantissa bits, ties to even
  if (q == 8) { q = 0; ++e; }
  return (uint8_t)(sign | ((e + 7) << 3) | q);
}
}  // namespace vrs

extern "C" {

int vrs_conv2d(vrs_ctx* ctx, const vrs_conv_desc* d, const vrs_nhwc* x, const void* w, const float* scale,
               const float* shift, const vrs_nhwc* res, const vrs_nhwc* y, void* stream) {
  if (!ctx || !d || !x || !y) return fail(VRS_EINVAL, "vrs_conv2d: null argument");
  ConvSpec cs;
  cs.k = d->k; cs.stride = d->stride; cs.act = d->act; cs.dtype = d->dtype; cs.tile = d->tile;
  cs.in_scale = d->in_scale;
  cs.x_f8 = d->x_e4m3 != 0;
  cs.y_f8 = d->y_e4m3 != 0;
  cs.res_f8 = d->res_e4m3 != 0;
  cs.out_step = d->out_step;
  cs.res_step = d->res_step;
  if (d->groups < 1) return fail(VRS_EINVAL, "vrs_conv2d: groups=%d", d->groups);
  if ((cs.x_f8 || cs.y_f8 || cs.res_f8) && (d->groups != 1 || d->dtype != VRS_FP8))
    return fail(VRS_EINVAL, "vrs_conv2d: e4m3 activations are for dense VRS_FP8 convs");
  if (d->groups > 1 && d->groups == x->c && d->groups == y->c) cs.depthwise = true;
  else cs.groups = d->groups;
  if (d->act != VRS_ACT_NONE && d->act != VRS_ACT_SILU) return fail(VRS_EINVAL, "vrs_conv2d: act %d", d->act);
  std::vector<Launch> ls;
  int rc = prep_conv(ctx, cs, *x, w, scale, shift, res, *y, ls);
  return rc ? rc : run_all(ls, stream);
}

int64_t vrs_pack_conv_weight(const float* w, int32_t cout, int32_t cin_g, int32_t k, int32_t groups, int32_t cin_pad,
                             int32_t dtype, void* out) {
  if (cout <= 0 || cin_g <= 0 || k <= 0 || groups <= 0) return fail(VRS_EINVAL, "pack_conv_weight: bad dims");
  if (dtype != VRS_BF16 && dtype != VRS_F32) return fail(VRS_EUNSUPPORTED, "pack_conv_weight: dtype");
  if (cout % groups) return fail(VRS_EINVAL, "pack_conv_weight: Cout %d not divisible by groups %d", cout, groups);
  // other groups > 1: the dense layout over each output channel's cin_g inputs
  // (OIHW already holds cin_g input channels per output channel)
  const bool depthwise = groups > 1 && groups == cout && cin_g == 1;
  if (groups > 1 && !depthwise && cin_pad != cin_g)
    return fail(VRS_EINVAL, "pack_conv_weight: grouped weights take no channel padding");
  if (depthwise) {
    const int64_t n = (int64_t)cout * k * k;
    const int64_t bytes = n * (int64_t)elt_size(dtype);
    if (!out) return bytes;
    if (!w) return fail(VRS_EINVAL, "pack_conv_weight: null weight");
    for (int c = 0; c < cout; ++c)  // [C][1][k][k] -> tap-major [k*k][C]
      for (int t = 0; t < k * k; ++t) {
        const float v = w[(int64_t)c * k * k + t];
        const int64_t o = (int64_t)t * cout + c;
        if (dtype == VRS_F32) static_cast<float*>(out)[o] = v;
        else static_cast<uint16_t*>(out)[o] = host_f2bf(v);
      }
    return bytes;
  }
  if (cin_pad < cin_g) return fail(VRS_EINVAL, "pack_conv_weight: cin_pad < cin");
  const int64_t n = (int64_t)cout * k * k * cin_pad;
  const int64_t bytes = n * (int64_t)elt_size(dtype);
  if (!out) return bytes;
  if (!w) return fail(VRS_EINVAL, "pack_conv_weight: null weight");
  for (int co = 0; co < cout; ++co)
    for (int ky = 0; ky < k; ++ky)
      for (int kx = 0; kx < k; ++kx)
        for (int ci = 0; ci < cin_pad; ++ci) {
          const float v = ci < cin_g ? w[(((int64_t)co * cin_g + ci) * k + ky) * k + kx] : 0.f;
          const int64_t o = (((int64_t)co * k + ky) * k + kx) * cin_pad + ci;
          if (dtype == VRS_F32) static_cast<float*>(out)[o] = v;
          else static_cast<uint16_t*>(out)[o] = host_f2bf(v);
        }
  return bytes;
}

int64_t vrs_pack_conv_weight_fp8(const float* w, int32_t cout, int32_t cin, int32_t k, int32_t cin_pad,
                                 uint8_t* out, float* out_scale) {
  if (cout <= 0 || cin <= 0 || k <= 0 || cin_pad < cin) return fail(VRS_EINVAL, "pack_conv_weight_fp8: shape");
  const int64_t bytes = (int64_t)cout * k * k * cin_pad;
  if (!out) return bytes;
  if (!w || !out_scale) return fail(VRS_EINVAL, "pack_conv_weight_fp8: null argument");
  const int64_t per = (int64_t)cin * k * k;
  for (int co = 0; co < cout; ++co) {
    float amax = 0.f;
    for (int64_t i = 0; i < per; ++i) amax = std::max(amax, std::fabs(w[co * per + i]));
    const float sc = amax > 0.f ? amax / 448.f : 1.f;
    out_scale[co] = sc;
    for (int ky = 0; ky < k; ++ky)
      for (int kx = 0; kx < k; ++kx)
        for (int ci = 0; ci < cin_pad; ++ci) {
          const int64_t o = (((int64_t)co * k + ky) * k + kx) * cin_pad + ci;
          out[o] = ci < cin ? f32_to_e4m3(w[((int64_t)(co * cin + ci) * k + ky) * k + kx] / sc) : 0;
        }
  }
  return bytes;
}

int64_t vrs_pack_stem_weight(const float* w, int32_t cout, int32_t dtype, void* out) {
  if (cout < 1 || cout > 128) return fail(VRS_EINVAL, "pack_stem_weight: cout %d (1..128)", cout);
  if (dtype != VRS_BF16 && dtype != VRS_F32) return fail(VRS_EUNSUPPORTED, "pack_stem_weight: dtype");
  const int cpad = (cout + 31) / 32 * 32;
  const int64_t bytes = (int64_t)cpad * 32 * (int64_t)elt_size(dtype);
  if (!out) return bytes;
  if (!w) return fail(VRS_EINVAL, "pack_stem_weight: null weights");
  for (int co = 0; co < cpad; ++co)
    for (int k = 0; k < 32; ++k) {
      // k = c*9 + ky*3 + kx is exactly the OIHW offset within one output channel
      const float v = (co < cout && k < 27) ? w[co * 27 + k] : 0.f;
      const int64_t o = (int64_t)co * 32 + k;
      if (dtype == VRS_F32) static_cast<float*>(out)[o] = v;
      else static_cast<uint16_t*>(out)[o] = host_f2bf(v);
    }
  return bytes;
}

int vrs_conv_stem(vrs_ctx* ctx, const vrs_conv_desc* d, const float* x, int32_t n, int32_t c, int32_t h, int32_t w,
                  const void* wp, const float* scale, const float* shift, const vrs_nhwc* y, void* stream) {
  if (!ctx || !d || !x || !y) return fail(VRS_EINVAL, "vrs_conv_stem: null argument");
  if (c != 3 || d->k != 3 || d->stride != 2 || d->groups != 1)
    return fail(VRS_EUNSUPPORTED, "vrs_conv_stem: 3 channels, 3x3, stride 2 only");
  if (d->act != VRS_ACT_NONE && d->act != VRS_ACT_SILU) return fail(VRS_EINVAL, "vrs_conv_stem: act %d", d->act);
  std::vector<Launch> ls;
  int rc = prep_stem(ctx, d->act, d->dtype, x, n, h, w, wp, scale, shift, y->c, *y, ls);
  return rc ? rc : run_all(ls, stream);
}

int vrs_conv_stem_pair(vrs_ctx* ctx, const vrs_conv_desc* d0, const vrs_conv_desc* d1, const float* x, int32_t n,
                       int32_t c, int32_t h, int32_t w, const void* w0, const float* scale0, const float* shift0,
                       const void* w1, const float* scale1, const float* shift1, const vrs_nhwc* y, void* stream) {
  if (!ctx || !d0 || !d1 || !x || !y) return fail(VRS_EINVAL, "vrs_conv_stem_pair: null argument");
  if (c != 3 || d0->k != 3 || d0->stride != 2 || d0->groups != 1 || d1->k != 3 || d1->stride != 2 || d1->groups != 1)
    return fail(VRS_EUNSUPPORTED, "vrs_conv_stem_pair: two 3x3 stride-2 dense convs on a 3-channel image only");
  if (d0->dtype != d1->dtype) return fail(VRS_EINVAL, "vrs_conv_stem_pair: the two layers' dtypes differ");
  int rc = stem_pair_check(d0->dtype, d0->act, d1->act, h, w);
  if (rc) return rc;
  std::vector<Launch> ls;
  rc = prep_stem_pair(ctx, x, n, h, w, w0, scale0, shift0, w1, scale1, shift1, *y, ls);
  return rc ? rc : run_all(ls, stream);
}

int vrs_conv_bottleneck_pair(vrs_ctx* ctx, const vrs_conv_desc* d1, const vrs_conv_desc* d2, const vrs_nhwc* x,
                             const void* w1, const float* scale1, const float* shift1, int32_t c_hidden,
                             const void* w2, const float* scale2, const float* shift2, const vrs_nhwc* res,
                             const vrs_nhwc* y, void* stream) {
  if (!ctx || !d1 || !d2 || !x || !y) return fail(VRS_EINVAL, "vrs_conv_bottleneck_pair: null argument");
  if (d1->k != 3 || d1->stride != 1 || d1->groups != 1 || d2->k != 3 || d2->stride != 1 || d2->groups != 1)
    return fail(VRS_EUNSUPPORTED, "vrs_conv_bottleneck_pair: two 3x3 stride-1 dense convs only");
  if (d1->dtype != d2->dtype) return fail(VRS_EINVAL, "vrs_conv_bottleneck_pair: the two convs' dtypes differ");
  if (d1->x_e4m3 || d1->y_e4m3 || d1->res_e4m3 || d2->x_e4m3 || d2->y_e4m3 || d2->res_e4m3)
    return fail(VRS_EINVAL, "vrs_conv_bottleneck_pair: e4m3 activations need the fp8 convs");
  int rc = bpair_check(d1->dtype, d1->act, d2->act, x->c, c_hidden, y->c);
  if (rc) return rc;
  std::vector<Launch> ls;
  rc = prep_bpair(ctx, *x, w1, scale1, shift1, c_hidden, w2, scale2, shift2, res, *y, ls);
  return rc ? rc : run_all(ls, stream);
}

int vrs_conv_pointwise_pair(vrs_ctx* ctx, const vrs_conv_desc* d1, const vrs_conv_desc* d2, const vrs_nhwc* x,
                            const void* w1, const float* scale1, const float* shift1, int32_t c_mid, const void* w2,
                            const float* scale2, const float* shift2, int32_t nc, float* y, int64_t sb, int64_t sp,
                            int64_t sc, void* stream) {
  if (!ctx || !d1 || !d2 || !x || !y) return fail(VRS_EINVAL, "vrs_conv_pointwise_pair: null argument");
  if (d1->k != 1 || d1->stride != 1 || d1->groups != 1 || d2->k != 1 || d2->stride != 1 || d2->groups != 1)
    return fail(VRS_EUNSUPPORTED, "vrs_conv_pointwise_pair: two 1x1 stride-1 dense convs only");
  if (d1->dtype != d2->dtype) return fail(VRS_EINVAL, "vrs_conv_pointwise_pair: the two convs' dtypes differ");
  if (d1->x_e4m3 || d1->y_e4m3 || d1->res_e4m3 || d2->x_e4m3 || d2->y_e4m3 || d2->res_e4m3)
    return fail(VRS_EINVAL, "vrs_conv_pointwise_pair: e4m3 activations need the fp8 convs");
  int rc = pwpair_check(d1->dtype, d1->act, d2->act, x->c, c_mid, nc);
  if (rc) return rc;
  std::vector<Launch> ls;
  rc = prep_pwpair(ctx, *x, w1, scale1, shift1, c_mid, w2, scale2, shift2, nc, y, sb, sp, sc, ls);
  return rc ? rc : run_all(ls, stream);
}

int vrs_bn_fold(const float* gamma, const float* beta, const float* mean, const float* var, float eps, int32_t c,
                float* scale, float* shift) {
  if (!gamma || !beta || !mean || !var || !scale || !shift || c <= 0) return fail(VRS_EINVAL, "vrs_bn_fold: bad args");
  for (int i = 0; i < c; ++i) {
    const float s = gamma[i] / std::sqrt(var[i] + eps);
    scale[i] = s;
    shift[i] = beta[i] - s * mean[i];
  }
  return VRS_OK;
}

int vrs_pack_input(vrs_ctx* ctx, const float* x, int32_t n, int32_t c, int32_t h, int32_t w, const vrs_nhwc* y,
                   int32_t dtype, void* stream) {
  if (!ctx || !y) return fail(VRS_EINVAL, "vrs_pack_input: null argument");
  std::vector<Launch> ls;
  int rc = prep_pack_input(ctx, x, n, c, h, w, *y, dtype, ls);
  return rc ? rc : run_all(ls, stream);
}

int vrs_unpack_output(vrs_ctx* ctx, const vrs_nhwc* x, int32_t dtype, float* y, void* stream) {
  if (!ctx || !x) return fail(VRS_EINVAL, "vrs_unpack_output: null argument");
  std::vector<Launch> ls;
  int rc = prep_unpack(ctx, *x, dtype, y, ls);
  return rc ? rc : run_all(ls, stream);
}

int vrs_sppf_pool(vrs_ctx* ctx, const vrs_nhwc* buf, int32_t dtype, void* stream) {
  if (!ctx || !buf) return fail(VRS_EINVAL, "vrs_sppf_pool: null argument");
  std::vector<Launch> ls;
  int rc = prep_pool(ctx, *buf, dtype, ls);
  return rc ? rc : run_all(ls, stream);
}

int vrs_upsample2x(vrs_ctx* ctx, const vrs_nhwc* x, const vrs_nhwc* y, int32_t dtype, void* stream) {
  if (!ctx || !x || !y) return fail(VRS_EINVAL, "vrs_upsample2x: null argument");
  std::vector<Launch> ls;
  int rc = prep_up(ctx, *x, *y, dtype, ls);
  return rc ? rc : run_all(ls, stream);
}

int vrs_psa_attention(vrs_ctx* ctx, const vrs_psa_desc* d, const vrs_nhwc* qkv, const void* pe_w,
                      const float* pe_scale, const float* pe_shift, const vrs_nhwc* out, void* stream) {
  if (!ctx || !d || !qkv || !out) return fail(VRS_EINVAL, "vrs_psa_attention: null argument");
  if (d->key_dim != 32 || d->head_dim != 64)
    return fail(VRS_EUNSUPPORTED, "vrs_psa_attention: key_dim %d head_dim %d (32/64 only)", d->key_dim, d->head_dim);
  std::vector<Launch> ls;
  int rc = prep_attn(ctx, d->heads, d->dtype, *qkv, pe_w, pe_scale, pe_shift, *out, ls);
  return rc ? rc : run_all(ls, stream);
}

}  // extern "C"

namespace vrs {

int64_t det_anchors(const vrs_detect_desc* d) {
  int64_t a = 0;
  for (int s = 0; s < d->nscales; ++s) a += (int64_t)(d->img_h / d->strides[s]) * (d->img_w / d->strides[s]);
  return a;
}

int det_check(const vrs_detect_desc* d) {
  if (!d) return fail(VRS_EINVAL, "detect: null descriptor");
  if (d->n <= 0 || d->nc <= 0 || d->nscales < 1 || d->nscales > 4 || d->img_h <= 0 || d->img_w <= 0)
    return fail(VRS_EBADSHAPE, "detect: bad descriptor");
  for (int s = 0; s < d->nscales; ++s)
    if (d->strides[s] <= 0 || d->img_h % d->strides[s] || d->img_w % d->strides[s])
      return fail(VRS_EBADSHAPE, "detect: image %dx%d not divisible by stride %d", d->img_h, d->img_w, d->strides[s]);
  if (d->max_det < 1 || d->max_det > 1024) return fail(VRS_EUNSUPPORTED, "detect: max_det %d (1..1024)", d->max_det);
  if (det_anchors(d) >= (1ll << 31) / 80) return fail(VRS_EBADSHAPE, "detect: too many anchors");
  return VRS_OK;
}

}  // namespace vrs

extern "C" {

size_t vrs_detect_workspace_size(const vrs_detect_desc* d) {
  if (det_check(d)) return 0;
  return (size_t)d->n * det_anchors(d) * (8 + 4 + 16);
}

int vrs_detect_postprocess(vrs_ctx* ctx, const vrs_detect_desc* d, const float* boxes, const float* scores,
                           void* ws, size_t ws_bytes, int32_t* count, float* score, int32_t* cls, int32_t* anchor,
                           float* xywh, void* stream) {
  if (!ctx) return fail(VRS_EINVAL, "vrs_detect_postprocess: null ctx");
  int rc = det_check(d);
  if (rc) return rc;
  if (!boxes || !scores || !ws || !count || !score || !cls || !anchor || !xywh)
    return fail(VRS_EINVAL, "vrs_detect_postprocess: null buffer");
  const int64_t A = det_anchors(d);
  if (ws_bytes < (size_t)d->n * A * 28) return fail(VRS_EINVAL, "vrs_detect_postprocess: workspace too small");
  if (reinterpret_cast<uintptr_t>(ws) % 16) return fail(VRS_EINVAL, "vrs_detect_postprocess: workspace alignment");
  uint64_t* keys = static_cast<uint64_t*>(ws);
  float* xy = reinterpret_cast<float*>(keys + (size_t)d->n * A);
  int32_t* cl = reinterpret_cast<int32_t*>(xy + (size_t)d->n * A * 4);
  vrs_det1_args a1{};
  a1.boxes = boxes; a1.scores = scores; a1.keys = keys; a1.cls = cl; a1.xywh = xy;
  a1.B = d->n; a1.nc = d->nc; a1.A = (int32_t)A; a1.nscales = d->nscales; a1.thr = d->thr;
  int base = 0;
  for (int s = 0; s < d->nscales; ++s) {
    a1.a_base[s] = base;
    a1.fw[s] = d->img_w / d->strides[s];
    a1.stride[s] = (float)d->strides[s];
    base += (d->img_h / d->strides[s]) * a1.fw[s];
  }
  vrs_det2_args a2{keys, cl, xy, count, score, cls, anchor, xywh, d->n, (int32_t)A, d->max_det};
  hipFunction_t f1, f2;
  if ((rc = get_fn(ctx, "vrs_detect_stage1", &f1)) || (rc = get_fn(ctx, "vrs_detect_stage2", &f2))) return rc;
  std::vector<Launch> ls;
  ls.push_back(make_launch("vrs_detect_stage1", f1, dim3((unsigned)((d->n * A + 255) / 256)), dim3(256), 0, a1));
  ls.push_back(make_launch("vrs_detect_stage2", f2, dim3(d->n), dim3(1024), 0, a2));
  return run_all(ls, stream);
}

int vrs_detect_unletterbox(vrs_ctx* ctx, int32_t n, int32_t max_det, int32_t img_size, const int32_t* orig_wh,
                           const int32_t* count, const float* xywh, float* out, void* stream) {
  if (!ctx || !orig_wh || !count || !xywh || !out) return fail(VRS_EINVAL, "vrs_detect_unletterbox: null argument");
  if (n <= 0 || max_det <= 0 || img_size <= 0) return fail(VRS_EBADSHAPE, "vrs_detect_unletterbox: empty shape");
  if ((int64_t)n * max_det >= (1ll << 31)) return fail(VRS_EBADSHAPE, "vrs_detect_unletterbox: too many slots");
  hipFunction_t f;
  int rc = get_fn(ctx, "vrs_detect_unletterbox", &f);
  if (rc) return rc;
  vrs_unlb_args a{orig_wh, count, xywh, out, n, max_det, img_size};
  std::vector<Launch> ls;
  ls.push_back(make_launch("vrs_detect_unletterbox", f, dim3((unsigned)(((int64_t)n * max_det + 255) / 256)),
                           dim3(256), 0, a));
  return run_all(ls, stream);
}

int vrs_letterbox(vrs_ctx* ctx, int32_t n, int32_t img_size, const uint8_t* rgb, int64_t rgb_bytes,
                  const int64_t* offsets, const int32_t* wh, float* out, void* stream) {
  if (!ctx || !rgb || !offsets || !wh || !out) return fail(VRS_EINVAL, "vrs_letterbox: null argument");
  if (n <= 0 || img_size <= 0 || rgb_bytes <= 0) return fail(VRS_EBADSHAPE, "vrs_letterbox: empty shape");
  if (img_size > 16384) return fail(VRS_EBADSHAPE, "vrs_letterbox: img_size %d > 16384", img_size);
  std::vector<vrs_lb_image> ims((size_t)n);
  for (int i = 0; i < n; ++i) {
    const int32_t w = wh[2 * i], h = wh[2 * i + 1];
    const int64_t off = offsets[i];
    if (w <= 0 || h <= 0) return fail(VRS_EBADSHAPE, "vrs_letterbox: image %d is %dx%d", i, w, h);
    if (off < 0 || off > rgb_bytes || (rgb_bytes - off) / 3 / w < h)
      return fail(VRS_EBADSHAPE, "vrs_letterbox: image %d (%dx%d at byte %lld) runs past rgb_bytes", i, w, h,
                  (long long)off);
    // preprocess_image_raw: scale and new size in f64, round half away from
    // zero, integer centring
    const double scale = (double)img_size / (double)(w > h ? w : h);
    const int32_t nw = (int32_t)std::round((double)w * scale), nh = (int32_t)std::round((double)h * scale);
    // bounded filter windows: ratio <= 62 gives at most 2*62 + 2 taps
    if ((nw > 0 && (float)w / (float)nw > 62.0f) || (nh > 0 && (float)h / (float)nh > 62.0f))
      return fail(VRS_EUNSUPPORTED, "vrs_letterbox: image %d (%dx%d) shrinks by more than 62x", i, w, h);
    ims[(size_t)i] = vrs_lb_image{off, w, h, nw, nh, (img_size - nw) / 2, (img_size - nh) / 2, i, 0};
  }
  // per image the staged kernel for shrinks up to 2x, 4x, then
  // VRS_LB_STAGED_RATIO x per axis (the kernels' own float32 ratio), else the
  // direct kernel
  auto kind = [](const vrs_lb_image& im) {
    auto within = [&](float r) {
      return (im.nw == 0 || (float)im.w / (float)im.nw <= r) && (im.nh == 0 || (float)im.h / (float)im.nh <= r);
    };
    return within(2.0f) ? 0 : within(4.0f) ? 1 : within((float)VRS_LB_STAGED_RATIO) ? 2 : 3;
  };
  static const char* names[4] = {"vrs_letterbox_f32_s2", "vrs_letterbox_f32_s4", "vrs_letterbox_f32_s8",
                                 "vrs_letterbox_f32"};
  std::vector<Launch> ls;
  for (int pass = 0; pass < 4; ++pass) {
    std::vector<vrs_lb_image> sel;
    for (const auto& im : ims)
      if (kind(im) == pass) sel.push_back(im);
    if (sel.empty()) continue;
    const char* name = names[pass];
    hipFunction_t f;
    int rc = get_fn(ctx, name, &f);
    if (rc) return rc;
    const int tw = pass == 2 ? 32 : 64;   // tile width; 4 rows
    const unsigned tiles = (unsigned)(((img_size + tw - 1) / tw) * ((img_size + 3) / 4));
    for (size_t b0 = 0; b0 < sel.size(); b0 += VRS_LB_MAX_IMAGES) {
      vrs_lb_args a{};
      a.rgb = rgb;
      a.out = out;
      a.pad = 114.0f / 255.0f;
      a.S = img_size;
      a.count = (int32_t)std::min<size_t>(VRS_LB_MAX_IMAGES, sel.size() - b0);
      for (int k = 0; k < a.count; ++k) a.img[k] = sel[b0 + (size_t)k];
      ls.push_back(make_launch(name, f, dim3(tiles, (unsigned)a.count), dim3(pass == 2 ? 128 : 256), 0, a));
    }
  }
  return run_all(ls, stream);
}

int vrs_detect_decode_grid(vrs_ctx* ctx, const float* boxes, const float* ax, const float* ay, const float* st,
                           int32_t n, int32_t a, float* out, void* stream) {
  if (!ctx || !boxes || !ax || !ay || !st || !out) return fail(VRS_EINVAL, "vrs_detect_decode_grid: null argument");
  if (n <= 0 || a <= 0) return fail(VRS_EBADSHAPE, "vrs_detect_decode_grid: empty");
  hipFunction_t f;
  int rc = get_fn(ctx, "vrs_detect_decode_grid", &f);
  if (rc) return rc;
  vrs_dec_args args{boxes, ax, ay, st, out, n, a};
  std::vector<Launch> ls;
  ls.push_back(make_launch("vrs_detect_decode_grid", f, dim3((unsigned)(((int64_t)n * a + 255) / 256)), dim3(256),
                           0, args));
  return run_all(ls, stream);
}

int vrs_msda(vrs_ctx* ctx, const vrs_msda_desc* d, const float* value, const float* ref, const float* off,
             const float* attw, float* out, void* stream) {
  if (!ctx || !d || !value || !ref || !off || !attw || !out) return fail(VRS_EINVAL, "vrs_msda: null argument");
  if (d->head_dim != 32) return fail(VRS_EUNSUPPORTED, "vrs_msda: head_dim %d (32 only)", d->head_dim);
  if (d->n <= 0 || d->q <= 0 || d->heads <= 0 || d->levels < 1 || d->levels > 8 || d->points < 1)
    return fail(VRS_EBADSHAPE, "vrs_msda: bad descriptor");
  vrs_msda_args a{};
  a.value = value; a.ref = ref; a.off = off; a.attw = attw; a.out = out;
  a.B = d->n; a.Q = d->q; a.heads = d->heads; a.L = d->levels; a.P = d->points;
  int64_t s = 0;
  for (int l = 0; l < d->levels; ++l) {
    if (d->level_h[l] <= 0 || d->level_w[l] <= 0) return fail(VRS_EBADSHAPE, "vrs_msda: level %d empty", l);
    a.lh[l] = d->level_h[l]; a.lw[l] = d->level_w[l]; a.lstart[l] = (int32_t)s;
    s += (int64_t)d->level_h[l] * d->level_w[l];
  }
  if (s >= (1ll << 31)) return fail(VRS_EBADSHAPE, "vrs_msda: too many value rows");
  a.S = (int32_t)s;
  if (reinterpret_cast<uintptr_t>(value) % 16 || reinterpret_cast<uintptr_t>(out) % 16 ||
      reinterpret_cast<uintptr_t>(off) % 8)
    return fail(VRS_EBADSHAPE, "vrs_msda: value/out must be 16-byte and off 8-byte aligned");
  // 8 lanes per (query, head), each owning 4 of the 32 channels.  L = 4,
  // P = 4 with <= 8 heads: one workgroup per query, one wave per level.
  const bool split = d->levels == 4 && d->points == 4 && d->heads <= 8;
  const char* name = split ? "vrs_msda_l4p4s_f32"
                           : (d->levels == 4 && d->points == 4) ? "vrs_msda_l4p4_f32" : "vrs_msda_f32";
  hipFunction_t f;
  int rc = get_fn(ctx, name, &f);
  if (rc) return rc;
  const int64_t threads = (int64_t)d->n * d->q * d->heads * 8;
  const int64_t blocks = split ? (int64_t)d->n * d->q : (threads + 255) / 256;
  if (blocks >= (1ll << 31)) return fail(VRS_EBADSHAPE, "vrs_msda: grid too large");
  std::vector<Launch> ls;
  ls.push_back(make_launch(name, f, dim3((unsigned)blocks), dim3(256), 0, a));
  return run_all(ls, stream);
}

}  // extern "C"

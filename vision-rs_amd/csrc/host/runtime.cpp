// Host runtime: errors, code-object loading, launch preparation.
// Everything here validates on the host before any HIP call and reports
// failures through status codes (include/vrs.h conventions).
#include <dirent.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>

#include "vrs_internal.h"

namespace vrs {

static thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_check(hipError_t e, const char* what) {
  return fail(VRS_EHIP, "%s: %s", what, hipGetErrorString(e));
}

int get_fn(vrs_ctx* ctx, const char* name, hipFunction_t* out) {
  auto it = ctx->fns.find(name);
  if (it != ctx->fns.end()) { *out = it->second; return VRS_OK; }
  for (hipModule_t m : ctx->modules) {
    hipFunction_t f = nullptr;
    if (hipModuleGetFunction(&f, m, name) == hipSuccess && f) {
      ctx->fns[name] = f;
      *out = f;
      return VRS_OK;
    }
    // A miss in this module is expected while probing; do not leave it as the
    // thread's sticky last error (the caller's own HIP checks would see it).
    (void)hipGetLastError();
  }
  return fail(VRS_ENOMODULE, "kernel '%s' not found in the code objects under %s", name, ctx->dir.c_str());
}

int run(const Launch& l, hipStream_t s) {
  void* params[] = {const_cast<uint8_t*>(l.args.data())};
  hipError_t e = hipModuleLaunchKernel(l.fn, l.grid.x, l.grid.y, l.grid.z, l.block.x, l.block.y, l.block.z,
                                       l.shmem, s, params, nullptr);
  if (e != hipSuccess) return fail(VRS_EHIP, "launch %s: %s", l.name.c_str(), hipGetErrorString(e));
  return VRS_OK;
}

static const void* at(const vrs_nhwc& v, int dtype) {
  return static_cast<const char*>(v.data) + (int64_t)v.c_off * elt_size(dtype);
}
// a view of e4m3 bytes (fp8 convs with e4m3 activations in memory)
static const void* at8(const vrs_nhwc& v) { return static_cast<const char*>(v.data) + v.c_off; }

// power of two in [2^-100, 2^100] (an e4m3 activation step)
static bool pow2_step(float s) {
  int e = 0;
  const float m = frexpf(s, &e);
  return s > 0.f && m == 0.5f && s >= 1e-30f && s <= 1e30f;
}

static int check_view(const vrs_nhwc& v, const char* what, int align) {
  if (!v.data) return fail(VRS_EINVAL, "%s: null data", what);
  if (v.n <= 0 || v.h <= 0 || v.w <= 0 || v.c <= 0) return fail(VRS_EBADSHAPE, "%s: empty shape", what);
  if (v.c_off < 0 || v.c_off + v.c > v.pitch)
    return fail(VRS_EBADSHAPE, "%s: channels [%d,%d) exceed pitch %d", what, v.c_off, v.c_off + v.c, v.pitch);
  if (v.c_off % align || v.pitch % align || v.c % align)
    return fail(VRS_EBADSHAPE, "%s: channel offset/pitch/count must be multiples of %d", what, align);
  if (reinterpret_cast<uintptr_t>(v.data) % 16) return fail(VRS_EBADSHAPE, "%s: data not 16-byte aligned", what);
  return VRS_OK;
}

static int check_dtype(int dtype) {
  if (dtype != VRS_BF16 && dtype != VRS_F32) return fail(VRS_EUNSUPPORTED, "dtype %d not supported", dtype);
  return VRS_OK;
}

static inline int out_size(int in, int k, int s) { return (in + 2 * (k / 2) - k) / s + 1; }

// Resident workgroups per CU of a kernel (registers, AGPRs and LDS as the
// runtime's occupancy calculator sees them), 1..8.
static int resident_wgs(hipFunction_t f, int threads = 256) {
  int n = 0;
  if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, threads, 0) != hipSuccess) {
    (void)hipGetLastError();
    n = 1;
  }
  return n < 1 ? 1 : n > 8 ? 8 : n;
}

// Dense-conv tiles.  bf16 has every tile with 32- and (when Cin % 64 == 0)
// 64-deep K steps; the float32 parity path has 128x128, 64x256 and 32x256.
struct TileInfo { int code, bm, bn; const char* tag; bool f32; bool k32; int threads; };
static const TileInfo kTiles[] = {
    {VRS_TILE_128x128, 128, 128, "128x128", true, true, 256}, {VRS_TILE_256x128, 256, 128, "256x128", false, true, 256},
    {VRS_TILE_128x256, 128, 256, "128x256", false, true, 256}, {VRS_TILE_64x256, 64, 256, "64x256", true, true, 256},
    {VRS_TILE_32x256, 32, 256, "32x256", true, true, 256},
    {VRS_TILE_256x256, 256, 256, "256x256", false, false, 512},  // 64-deep K steps only
    {VRS_TILE_64x64, 64, 64, "64x64", false, true, 256},          // bf16, Cin % 32 == 0
};

static const TileInfo* tile_info(int code) {
  for (const auto& t : kTiles)
    if (t.code == (code & 0xff)) return &t;
  return nullptr;
}

// Kernel name for a tile, or an error when the combination is not built.
// up: the fused-upsample instance (_u), built for 128x128, 256x128, 128x256
// and 256x256 in bf16 and 128x128 and 64x256 in float32, aligned and not
// persistent
static int tile_kernel(int code, int cin, int dtype, bool up, char* name, size_t n, int* bm, int* bn, int* threads,
                       bool x8 = false, bool y8 = false) {
  if ((code & 0xff) == VRS_TILE_H3 || (code & 0xff) == VRS_TILE_W1_256 || (code & 0xff) == VRS_TILE_W1_128)
    return fail(VRS_EINVAL, "conv: the halo and weight-stationary tiles are prepared separately");
  const TileInfo* t = tile_info(code);
  if (!t) return fail(VRS_EINVAL, "conv: unknown tile code %d", code);
  if (up) {
    const bool built = dtype != VRS_F32 ? (t->code == VRS_TILE_128x128 || t->code == VRS_TILE_256x128 ||
                                           t->code == VRS_TILE_128x256 || t->code == VRS_TILE_256x256)
                                        : (t->code == VRS_TILE_128x128 || t->code == VRS_TILE_64x256);
    if (!built || (code & VRS_TILE_PERSIST) || cin % 32 != 0)
      return fail(VRS_EUNSUPPORTED, "conv: no fused-upsample kernel for tile %s (dtype %d, Cin %d)", t->tag, dtype, cin);
  }
  const bool k128 = (code & VRS_TILE_K128) != 0;
  if (k128 && dtype != VRS_FP8) return fail(VRS_EUNSUPPORTED, "conv: 128-deep steps are built for fp8 only");
  if (dtype == VRS_FP8) {
    if (cin % 64 != 0) return fail(VRS_EUNSUPPORTED, "conv fp8: needs Cin %% 64 == 0 (Cin=%d)", cin);
    if (t->code == VRS_TILE_32x256 || t->code == VRS_TILE_64x64 || (code & VRS_TILE_PERSIST))
      return fail(VRS_EUNSUPPORTED, "conv fp8: tile %s%s not built", t->tag, (code & VRS_TILE_PERSIST) ? " persistent" : "");
    if (k128 && (cin % 128 != 0 || up || t->code != VRS_TILE_256x256 || !x8))
      return fail(VRS_EUNSUPPORTED, "conv fp8: 128-deep steps need tile 256x256, an e4m3 input, Cin %% 128 == 0 "
                  "and no fused upsample (tile %s, Cin %d)", t->tag, cin);
    snprintf(name, n, "vrs_conv_fp8_%s_k%d_%c%s%s", t->tag, k128 ? 128 : 64, up ? 'u' : 'a', x8 ? "_x8" : "",
             y8 ? "_y8" : "");
    *bm = t->bm;
    *bn = t->bn;
    *threads = t->threads;
    return VRS_OK;
  }
  if (dtype == VRS_F32 && !t->f32) return fail(VRS_EUNSUPPORTED, "conv: tile %s has no float32 build", t->tag);
  const bool g = cin % 32 != 0;
  bool k64 = !(code & VRS_TILE_K32) && dtype == VRS_BF16 && cin % 64 == 0 && t->code != VRS_TILE_32x256;
  if (code & VRS_TILE_PERSIST) {
    if (dtype != VRS_BF16 || g ||
        (t->code != VRS_TILE_128x128 && t->code != VRS_TILE_64x256 && t->code != VRS_TILE_256x256) ||
        (t->code == VRS_TILE_64x256 && k64) || (t->code == VRS_TILE_256x256 && !k64))
      return fail(VRS_EUNSUPPORTED, "conv: persistent tile %s%s not built for this dtype/Cin", t->tag,
                  k64 ? " k64" : "");
    snprintf(name, n, "vrs_conv_bf16_%s_k%d_p", t->tag, k64 ? 64 : 32);
    *bm = t->bm;
    *bn = t->bn;
    *threads = t->threads;
    return VRS_OK;
  }
  if (!t->k32 && (!k64 || g))
    return fail(VRS_EUNSUPPORTED, "conv: tile %s needs Cin %% 64 == 0 and 64-deep steps (Cin=%d)", t->tag, cin);
  if (g && t->code != VRS_TILE_128x128 && t->code != VRS_TILE_64x256 && t->code != VRS_TILE_32x256)
    return fail(VRS_EUNSUPPORTED, "conv: tile %s needs Cin %% 32 == 0 (Cin=%d)", t->tag, cin);
  snprintf(name, n, "vrs_conv_%s_%s_k%d_%c", dsuffix(dtype), t->tag, k64 ? 64 : 32, up ? 'u' : g ? 'g' : 'a');
  *bm = t->bm;
  *bn = t->bn;
  *threads = t->threads;
  return VRS_OK;
}

// Shape heuristic (VRS_TILE_AUTO): the widest tile that still gives the
// 256-CU chip at least two workgroups per CU.
static int auto_tile(int cout, int cin, int64_t M, int dtype, int num_cu) {
  auto blocks = [&](int bm, int bn) { return (int64_t)((cout + bm - 1) / bm) * ((M + bn - 1) / bn); };
  const int64_t want = 2ll * (num_cu > 0 ? num_cu : 256);
  if (cout <= 32) return VRS_TILE_32x256;
  if (cout <= 64) return VRS_TILE_64x256;
  if (dtype == VRS_BF16 && cin % 32 == 0) {
    if (cout <= 128 && blocks(128, 256) >= want) return VRS_TILE_128x256;
    if (cout > 128 && blocks(256, 128) >= want) return VRS_TILE_256x128;
  }
  return VRS_TILE_128x128;
}

// Strip width of the halo-tiled 3x3 kernel for an image width (0: not usable).
// 32 or 16 when they divide the width: a 16-lane group of the MFMA operand
// reads then never spans a strip row (a row change skips the two halo
// columns and puts two lanes of the group on the same LDS banks), and the
// strip's pixel count is a multiple of the 256-pixel run (no padded run) for
// any height.  Else the whole width up to 40 pixels, else 20 when it divides
// the width, else 32.
static int h3_strip_width(int w) {
  if (w < 8) return 0;
  if (w % 32 == 0) return 32;
  if (w % 16 == 0) return 16;
  if (w <= 40) return w;
  if (w % 20 == 0) return 20;
  return 32;
}

// Input widths the fp8 weight-stationary 1x1 kernel is built for.
static bool w1_fp8_cin(int cin) {
  return cin == 128 || cin == 192 || cin == 256 || cin == 384 || cin == 512 || cin == 768;
}

std::vector<int> conv_tile_candidates(int cout, int cin, int dtype, int k, int stride, int w, int64_t m,
                                      int num_cu) {
  std::vector<int> c;
  if (dtype == VRS_BF16 && k == 3 && stride == 1 && cin % 32 == 0 && h3_strip_width(w) > 0) c.push_back(VRS_TILE_H3);
  if (dtype == VRS_BF16 && k == 1 && stride == 1 && cin % 64 == 0 && (cin <= 256 || cin == 384) && w > 0) {
    if (cout > 128 && cin <= 192) c.push_back(VRS_TILE_W1_256);
    c.push_back(VRS_TILE_W1_128);
  }
  if (dtype == VRS_FP8) {
    if (cin % 64) return c;
    c.push_back(VRS_TILE_128x128);
    c.push_back(VRS_TILE_64x256);
    if (cout > 128) c.push_back(VRS_TILE_256x128);
    if (cout <= 128) c.push_back(VRS_TILE_128x256);
    if (cout >= 256) c.push_back(VRS_TILE_256x256);
    // 128-deep steps (e4m3 inputs only: a bf16-input conv fails to prepare it)
    if (cin % 128 == 0 && cout >= 256) c.push_back(VRS_TILE_256x256 | VRS_TILE_K128);
    if (k == 1 && stride == 1 && w > 0 && w1_fp8_cin(cin)) c.push_back(VRS_TILE_W1_128);
    return c;
  }
  const bool g = cin % 32 != 0;
  for (const auto& t : kTiles) {
    if (dtype == VRS_F32 && !t.f32) continue;
    if (g && t.code != VRS_TILE_128x128 && t.code != VRS_TILE_64x256 && t.code != VRS_TILE_32x256) continue;
    if (t.bm >= 2 * 128 && cout <= 128) continue;   // mostly empty rows
    if (t.bm <= 64 && cout > 4 * t.bm) continue;     // too many passes over the input
    if (t.code == VRS_TILE_64x64) {   // only where 128x128 leaves the chip under-filled
      const int64_t b128 = (int64_t)((cout + 127) / 128) * ((m + 127) / 128);
      if (g || (m > 0 && b128 >= 2ll * (num_cu > 0 ? num_cu : 256))) continue;
    }
    if (!t.k32) {  // 64-deep only (256x256), also persistent with an even step count
      if (dtype == VRS_BF16 && cin % 64 == 0 && cout >= t.bm) {
        c.push_back(t.code);
        if ((k * k * cin / 64) % 2 == 0) c.push_back(t.code | VRS_TILE_PERSIST);
      }
      continue;
    }
    c.push_back(t.code);
    if (dtype == VRS_BF16 && cin % 64 == 0 && t.code != VRS_TILE_32x256) c.push_back(t.code | VRS_TILE_K32);
    if (dtype == VRS_BF16 && !g && (t.code == VRS_TILE_128x128 || t.code == VRS_TILE_64x256)) {
      c.push_back(t.code | VRS_TILE_K32 | VRS_TILE_PERSIST);
      if (t.code == VRS_TILE_128x128 && cin % 64 == 0) c.push_back(t.code | VRS_TILE_PERSIST);
    }
  }
  return c;
}

static int prep_dense(vrs_ctx* ctx, const ConvSpec& cs, const vrs_nhwc& x, const void* w, const float* scale,
                      const float* shift, int cout, int ho, int wo, vrs_conv_args& a, std::vector<Launch>& out) {
  int rc;
  const bool f8 = cs.dtype == VRS_FP8;
  if (!f8 && (rc = check_dtype(cs.dtype))) return rc;
  if (!f8 && (cs.x_f8 || cs.y_f8 || cs.res_f8))
    return fail(VRS_EINVAL, "conv: e4m3 activations need the fp8 dtype");
  // bytes per element of the input (and fused-upsample source)
  const int64_t xs = cs.x_f8 ? 1 : (int64_t)elt_size(cs.dtype);
  if (f8) {
    if (!pow2_step(cs.in_scale))
      return fail(VRS_EINVAL, "conv fp8: in_scale %g must be a positive power of two", (double)cs.in_scale);
    if (cs.y_f8 && !pow2_step(cs.out_step))
      return fail(VRS_EINVAL, "conv fp8: out_step %g must be a positive power of two", (double)cs.out_step);
    if (cs.y_f8 && a.stage != 1)
      return fail(VRS_EUNSUPPORTED, "conv fp8: an e4m3 output must be an NHWC view with 16-channel aligned offset, "
                  "pitch and count, under 2 GiB");
    if (cs.res_f8 && a.stage != 1)
      return fail(VRS_EUNSUPPORTED, "conv fp8: an e4m3 residual needs a staged output (16-byte aligned NHWC view)");
    a.out_step = cs.y_f8 ? cs.out_step : 0.f;
    a.in_scale = cs.in_scale;
    // bfloat16 bits of 448 * in_scale (exact: 448 has 3 significant bits)
    uint32_t fb;
    const float lim = 448.f * cs.in_scale;
    memcpy(&fb, &lim, 4);
    const uint32_t hb = fb >> 16;
    a.clamp_bits = hb | (hb << 16);
  }
  if ((rc = check_view(x, "conv input", cs.x_f8 ? 16 : 8))) return rc;
  if (!w || !scale || !shift) return fail(VRS_EINVAL, "conv: null weight/scale/shift");
  if (cs.k < 1 || cs.k > 7 || cs.k % 2 == 0 || cs.stride < 1) return fail(VRS_EBADSHAPE, "conv: k=%d s=%d", cs.k, cs.stride);
  if (ho != out_size(x.h, cs.k, cs.stride) || wo != out_size(x.w, cs.k, cs.stride))
    return fail(VRS_EBADSHAPE, "conv: output %dx%d does not match input %dx%d k=%d s=%d", ho, wo, x.h, x.w, cs.k,
                cs.stride);
  a.x = cs.x_f8 ? at8(x) : at(x, cs.dtype);
  a.w = w;
  a.scale = scale;
  a.shift = shift;
  {  // raw-buffer extents (the kernels use 32-bit byte offsets)
    const int64_t xb = ((int64_t)x.n * x.h * x.w * x.pitch - x.c_off) * xs;
    const int64_t wb = (int64_t)cout * cs.k * cs.k * x.c * (f8 ? 1 : (int64_t)elt_size(cs.dtype));
    if (xb >= (1ll << 31) || wb >= (1ll << 31))
      return fail(VRS_EBADSHAPE, "conv: input buffer (%lld B) or weights (%lld B) exceed 2 GiB", (long long)xb,
                  (long long)wb);
    a.x_bytes = (int32_t)xb;
    a.w_bytes = (int32_t)wb;
  }
  if (cs.up) {  // channels [0, up->c) of the input are up(*cs.up), nearest 2x
    const vrs_nhwc& u = *cs.up;
    if ((rc = check_view(u, "conv upsample source", cs.x_f8 ? 16 : 8))) return rc;
    if (cs.k != 1 || cs.stride != 1 || u.n != x.n || 2 * u.h != x.h || 2 * u.w != x.w || u.c >= x.c || u.c % 64)
      return fail(VRS_EBADSHAPE, "conv: a fused upsample needs a 1x1 stride-1 conv, a half-size source and a "
                  "split at a multiple of 64 channels below Cin (source %dx%dx%d, input %dx%dx%d)", u.h, u.w, u.c,
                  x.h, x.w, x.c);
    const int64_t ub = ((int64_t)u.n * u.h * u.w * u.pitch - u.c_off) * xs;
    if (ub >= (1ll << 31)) return fail(VRS_EBADSHAPE, "conv: upsample source exceeds 2 GiB");
    a.x2 = cs.x_f8 ? at8(u) : at(u, cs.dtype);
    a.x2_bytes = (int32_t)ub;
    a.c_split = u.c;
    a.H2 = u.h;
    a.W2 = u.w;
    a.x2_pitch = u.pitch;
  }
  a.N = x.n; a.H = x.h; a.W = x.w; a.Cin = x.c; a.x_pitch = x.pitch;
  a.Ho = ho; a.Wo = wo; a.Cout = cout;
  a.kh = a.kw = cs.k; a.stride = cs.stride; a.pad = cs.k / 2;
  a.K = cs.k * cs.k * x.c;
  const int64_t M = (int64_t)x.n * ho * wo;
  if (M >= (1ll << 24))  // the kernels divide pixel indices through a float reciprocal
    return fail(VRS_EBADSHAPE, "conv: %lld output pixels per launch exceed 2^24 (split the batch)", (long long)M);
  a.M = (int32_t)M;
  a.act = cs.act;
  char name[64];
  int bm, bn, threads;
  if ((cs.tile & 0xff) == VRS_TILE_H3) {
    // halo-tiled 3x3 stride-1 kernel (conv3.hip)
    const int tw = h3_strip_width(x.w);
    if (cs.dtype != VRS_BF16 || cs.k != 3 || cs.stride != 1 || x.c % 32 != 0 || tw == 0 || cs.up)
      return fail(VRS_EUNSUPPORTED, "conv: the halo 3x3 tile needs bf16, k=3, stride 1, Cin %% 32 == 0, width >= 8 "
                  "and no fused upsample (k=%d s=%d Cin=%d W=%d)", cs.k, cs.stride, x.c, x.w);
    if (!a.stage || a.y_f32)
      return fail(VRS_EUNSUPPORTED, "conv: the halo 3x3 tile stores whole 16-byte channel chunks of a bf16 NHWC view");
    if (a.res && a.res_bytes < 0) return fail(VRS_EBADSHAPE, "conv: halo tile residual exceeds 2 GiB");
    bm = cout <= 32 ? 32 : 64;
    a.h3_tw = tw;
    a.h3_strips = (x.w + tw - 1) / tw;
    a.h3_chunks = (int)(((int64_t)x.h * tw + 255) / 256);
    a.tiles_m = (cout + bm - 1) / bm;
    a.tiles_n = 0;
    const int64_t blocks = (int64_t)a.tiles_m * x.n * a.h3_strips * a.h3_chunks;
    if (blocks >= (1ll << 31)) return fail(VRS_EBADSHAPE, "conv: grid too large");
    if ((int64_t)x.n * x.h * x.w * (int64_t)x.pitch * 2 >= (1ll << 31))
      return fail(VRS_EBADSHAPE, "conv: halo tile input exceeds 2 GiB");
    snprintf(name, sizeof name, "vrs_conv3h_bf16_%d", bm);
    hipFunction_t f;
    if ((rc = get_fn(ctx, name, &f))) return rc;
    out.push_back(make_launch(name, f, dim3((unsigned)blocks), dim3(256), 0, a));
    out.back().flops = 2.0 * (double)M * cout * 9.0 * (cs.cin_real > 0 ? cs.cin_real : x.c);
    out.back().bytes = (double)x.n * x.h * x.w * x.c * 2.0 + (double)cout * 9.0 * x.c * 2.0 + (double)M * cout * 2.0 +
                       (a.res ? (double)M * cout * 2.0 : 0.0) + 8.0 * cout;
    return VRS_OK;
  }
  if (f8 && ((cs.tile & 0xff) == VRS_TILE_W1_256 || (cs.tile & 0xff) == VRS_TILE_W1_128)) {
    // fp8 weight-stationary 1x1 kernel (conv1w8.hip): a 128-channel slice of
    // e4m3 weights in LDS, 128-pixel tiles
    if ((cs.tile & 0xff) != VRS_TILE_W1_128 || (cs.tile & ~0xff) || !w1_fp8_cin(x.c) || cs.k != 1 ||
        cs.stride != 1 || cs.up)
      return fail(VRS_EUNSUPPORTED, "conv fp8: the weight-stationary tile is the 128-channel one, for k=1, stride 1, "
                  "no fused upsample and Cin 128, 192, 256, 384, 512 or 768 (k=%d s=%d Cin=%d)", cs.k, cs.stride, x.c);
    if (a.res || a.stage != 1 || a.y_f32)
      return fail(VRS_EUNSUPPORTED, "conv fp8: the weight-stationary tile takes no residual and stores aligned "
                  "chunks of an NHWC view under 2 GiB");
    a.tiles_m = (cout + 127) / 128;
    a.tiles_n = (int32_t)((M + 127) / 128);
    snprintf(name, sizeof name, "vrs_conv1w_fp8_128_c%d%s%s", x.c, cs.x_f8 ? "_x8" : "", cs.y_f8 ? "_y8" : "");
    hipFunction_t f;
    if ((rc = get_fn(ctx, name, &f))) return rc;
    const int64_t resident = (int64_t)resident_wgs(f, 512) * (ctx->num_cu > 0 ? ctx->num_cu : 256);
    const int64_t streams = std::max<int64_t>(1, std::min<int64_t>(resident / a.tiles_m, a.tiles_n));
    out.push_back(make_launch(name, f, dim3((unsigned)(streams * a.tiles_m)), dim3(512), 0, a));
    out.back().flops = 2.0 * (double)M * cout * (cs.cin_real > 0 ? cs.cin_real : x.c);
    out.back().bytes = (double)M * x.c * (double)xs + (double)cout * x.c + (double)M * cout * (cs.y_f8 ? 1.0 : 2.0) +
                       8.0 * cout;
    return VRS_OK;
  }
  if ((cs.tile & 0xff) == VRS_TILE_W1_256 || (cs.tile & 0xff) == VRS_TILE_W1_128) {
    // weight-stationary 1x1 kernel (conv1w.hip)
    bm = (cs.tile & 0xff) == VRS_TILE_W1_256 ? 256 : 128;
    // Cin 384 on the 128-channel tile: each pixel tile streams in two halves
    const bool cin_ok = bm == 256 ? x.c <= 192 : (x.c <= 256 || x.c == 384);
    if (cs.dtype != VRS_BF16 || cs.k != 1 || cs.stride != 1 || cs.up || x.c % 64 != 0 || !cin_ok)
      return fail(VRS_EUNSUPPORTED, "conv: the weight-stationary %d-channel tile needs bf16, k=1, stride 1, no fused "
                  "upsample and Cin a multiple of 64 up to %s (k=%d s=%d Cin=%d)", bm,
                  bm == 256 ? "192" : "256, or 384", cs.k, cs.stride, x.c);
    const bool flat = a.y_f32 && a.stage == 2;   // channel-major float32 (the Detect head's outputs)
    if (a.res || (!flat && (!a.stage || a.y_f32)) || (flat && bm != 128))
      return fail(VRS_EUNSUPPORTED, "conv: the weight-stationary tile takes no residual and stores 8-channel-aligned "
                  "chunks of a bf16 NHWC view under 2 GiB (or, on the 128-channel tile, a channel-major float32 "
                  "output)");
    a.tiles_m = (cout + bm - 1) / bm;
    a.tiles_n = (int32_t)((M + 63) / 64);
    snprintf(name, sizeof name, "vrs_conv1w_bf16_%d_c%d%s", bm, x.c, flat ? "_f" : "");
    if (flat && x.c != 64 && x.c != 256)
      return fail(VRS_EUNSUPPORTED, "conv: the weight-stationary float32 output tile takes Cin 64 or 256 (Cin=%d)", x.c);
    hipFunction_t f;
    if ((rc = get_fn(ctx, name, &f))) return rc;
    // persistent grid: the resident workgroups, a whole number of streams
    // (one workgroup per channel slice each), no more streams than tiles
    const int64_t resident = (int64_t)resident_wgs(f, 512) * (ctx->num_cu > 0 ? ctx->num_cu : 256);
    const int64_t streams = std::max<int64_t>(1, std::min<int64_t>(resident / a.tiles_m, a.tiles_n));
    out.push_back(make_launch(name, f, dim3((unsigned)(streams * a.tiles_m)), dim3(512), 0, a));
    out.back().flops = 2.0 * (double)M * cout * (cs.cin_real > 0 ? cs.cin_real : x.c);
    out.back().bytes = (double)M * x.c * 2.0 + (double)cout * x.c * 2.0 + (double)M * cout * (flat ? 4.0 : 2.0) +
                       8.0 * cout;
    return VRS_OK;
  }
  const int tile = cs.tile ? cs.tile
                            : f8 ? (cout <= 64 && !cs.up ? VRS_TILE_64x256 : VRS_TILE_128x128)
                                 : cs.up ? VRS_TILE_128x128   // built in every fused-upsample dtype
                                         : auto_tile(cout, x.c, M, cs.dtype, ctx->num_cu);
  if ((rc = tile_kernel(tile, x.c, cs.dtype, cs.up != nullptr, name, sizeof name, &bm, &bn, &threads, cs.x_f8,
                        cs.y_f8)))
    return rc;
  a.tiles_m = (cout + bm - 1) / bm;
  a.tiles_n = (int32_t)((M + bn - 1) / bn);
  int64_t blocks = (int64_t)a.tiles_m * a.tiles_n;
  if (blocks >= (1ll << 31)) return fail(VRS_EBADSHAPE, "conv: grid too large");
  hipFunction_t f;
  if ((rc = get_fn(ctx, name, &f))) return rc;
  const int64_t tiles_total = blocks;
  if (tile & VRS_TILE_PERSIST) {
    const int bk = strstr(name, "_k64_") ? 64 : 32;
    if (a.res || !a.stage || a.y_f32 || a.K % (2 * bk) != 0)
      return fail(VRS_EUNSUPPORTED, "conv: persistent tile needs no residual, a staged bf16 output and an even "
                  "number of %d-deep K steps (K=%d)", bk, a.K);
    blocks = std::min<int64_t>(blocks, (int64_t)resident_wgs(f, threads) * (ctx->num_cu > 0 ? ctx->num_cu : 256));
  }
  const double es = (double)elt_size(cs.dtype);
  const double cin = cs.cin_real > 0 ? cs.cin_real : x.c;
  const double kk = (double)cs.k * cs.k;
  const double flops = 2.0 * (double)M * cout * kk * cin;
  const double cin_up = cs.up ? (double)cs.up->c : 0.0;   // read at a quarter of the pixels
  const double bytes = (double)x.n * x.h * x.w * (cin - 0.75 * cin_up) * (double)xs +
                       (double)cout * kk * cin * (f8 ? 1.0 : es) +
                       (double)M * cout * (a.y_f32 ? 4.0 : cs.y_f8 ? 1.0 : es) +
                       (a.res ? (double)M * cout * (cs.res_f8 ? 1.0 : es) : 0.0) + 8.0 * cout;
  // Partial last round of 256x256 tiles (one workgroup per CU): when the
  // tiles leave a last round at most half full, the full rounds run on the
  // 256x256 tile (persistent: one workgroup per CU looping over an equal
  // share of them) and the leftover pixel tiles on the 128x128 tile of the
  // same 64-deep K order (four times the workgroups for the same work, two
  // per CU: the round takes about a quarter of the time).  Same results: each
  // output is one workgroup's accumulation over K in the same step order.
  if ((tile & 0xff) == VRS_TILE_256x256 && !f8 && cs.dtype == VRS_BF16 && a.K % 64 == 0 && cout % 256 == 0) {
    const int64_t G = (int64_t)resident_wgs(f, threads) * (ctx->num_cu > 0 ? ctx->num_cu : 256);
    const int64_t R = tiles_total % G;
    if (tiles_total > G && R > 0 && 2 * R <= G && R % a.tiles_m == 0) {
      const char* rname = cs.up ? "vrs_conv_bf16_128x128_k64_u" : "vrs_conv_bf16_128x128_k64_a";
      hipFunction_t fr;
      if ((rc = get_fn(ctx, rname, &fr))) return rc;
      const double share = (double)R / (double)tiles_total;
      if (tile & VRS_TILE_PERSIST) {   // one workgroup per CU, each taking the same number of tiles
        vrs_conv_args p = a;
        p.tiles_n = (int32_t)((tiles_total - R) / a.tiles_m);
        out.push_back(make_launch(name, f, dim3((unsigned)G), dim3(threads), 0, p));
      } else {
        out.push_back(make_launch(name, f, dim3((unsigned)(tiles_total - R)), dim3(threads), 0, a));
      }
      out.back().flops = flops * (1.0 - share);
      out.back().bytes = bytes * (1.0 - share);
      vrs_conv_args b = a;
      b.tiles_m = cout / 128;
      b.n_tile0 = (int32_t)((tiles_total - R) / a.tiles_m * 2);   // in 128-pixel tiles
      b.tiles_n = (int32_t)((M + 127) / 128);
      const int64_t rb = (int64_t)b.tiles_m * (b.tiles_n - b.n_tile0);
      out.push_back(make_launch(rname, fr, dim3((unsigned)rb), dim3(256), 0, b));
      out.back().flops = flops * share;
      out.back().bytes = bytes * share;
      return VRS_OK;
    }
  }
  out.push_back(make_launch(name, f, dim3((unsigned)blocks), dim3(threads), 0, a));
  out.back().flops = flops;
  out.back().bytes = bytes;
  return VRS_OK;
}

// Grouped conv, 1 < groups < channels: conv_bn with any g (blocks/conv.rs:
// 51-69).  Weights [Cout][k][k][cin_g], so group g's output channels are the
// rows from g*cout_g on.  Groups that fit the implicit-GEMM kernels
// (cin_g % 8 == 0, cout_g % 4 == 0, aligned channel offsets and pitches) and
// bring a tile enough work per pixel (cin_g * cout_g >= 1024) run as one dense
// launch per group on channel slices of the views; the rest on the direct
// kernel (one thread per output element).  fp8 only on the dense route.
static int prep_grouped(vrs_ctx* ctx, const ConvSpec& cs, const vrs_nhwc& x, const void* w, const float* scale,
                        const float* shift, const vrs_nhwc* res, const vrs_nhwc& y, std::vector<Launch>& out) {
  int rc;
  const int G = cs.groups;
  if (x.c % G || y.c % G)
    return fail(VRS_EBADSHAPE, "grouped conv: channels %d -> %d not divisible by groups %d", x.c, y.c, G);
  if (cs.up) return fail(VRS_EUNSUPPORTED, "grouped conv: no fused upsample");
  if (!w || !scale || !shift) return fail(VRS_EINVAL, "grouped conv: null weight/scale/shift");
  if (cs.k < 1 || cs.k > 7 || cs.k % 2 == 0 || cs.stride < 1)
    return fail(VRS_EBADSHAPE, "grouped conv: k=%d s=%d", cs.k, cs.stride);
  if (y.n != x.n || y.h != out_size(x.h, cs.k, cs.stride) || y.w != out_size(x.w, cs.k, cs.stride))
    return fail(VRS_EBADSHAPE, "grouped conv: output shape");
  if (res && (res->n != y.n || res->h != y.h || res->w != y.w || res->c != y.c))
    return fail(VRS_EBADSHAPE, "grouped conv: residual shape differs from output");
  const int cin_g = x.c / G, cout_g = y.c / G;
  const bool aligned = x.c_off % 8 == 0 && x.pitch % 8 == 0 && y.c_off % 4 == 0 && y.pitch % 4 == 0 &&
                       (!res || (res->c_off % 4 == 0 && res->pitch % 4 == 0));
  const bool dense = aligned && cin_g % 8 == 0 && cout_g % 4 == 0 && (int64_t)cin_g * cout_g >= 1024 &&
                     (cs.dtype != VRS_FP8 || cin_g % 64 == 0);
  if (dense) {
    const int64_t wrow = (int64_t)cs.k * cs.k * cin_g * (cs.dtype == VRS_FP8 ? 1 : (int64_t)elt_size(cs.dtype));
    ConvSpec gs = cs;
    gs.groups = 1;
    gs.cin_real = 0;
    for (int g = 0; g < G; ++g) {
      vrs_nhwc xg = x, yg = y, rg{};
      xg.c_off += g * cin_g;
      xg.c = cin_g;
      yg.c_off += g * cout_g;
      yg.c = cout_g;
      if (res) {
        rg = *res;
        rg.c_off += g * cout_g;
        rg.c = cout_g;
      }
      if ((rc = prep_conv(ctx, gs, xg, static_cast<const char*>(w) + (int64_t)g * cout_g * wrow, scale + g * cout_g,
                          shift + g * cout_g, res ? &rg : nullptr, yg, out)))
        return rc;
    }
    return VRS_OK;
  }
  if (cs.dtype == VRS_FP8)
    return fail(VRS_EUNSUPPORTED, "grouped conv fp8: needs Cin/groups %% 64 == 0 (got %d) and aligned views", cin_g);
  if ((rc = check_dtype(cs.dtype))) return rc;
  if ((rc = check_view(x, "grouped conv input", 1)) || (rc = check_view(y, "grouped conv output", 1))) return rc;
  if (res && (rc = check_view(*res, "grouped conv residual", 1))) return rc;
  vrs_gconv_args a{};
  a.x = at(x, cs.dtype);
  a.w = w;
  a.scale = scale;
  a.shift = shift;
  a.res = res ? at(*res, cs.dtype) : nullptr;
  a.y = const_cast<void*>(at(y, cs.dtype));
  a.total = (int64_t)y.n * y.h * y.w * y.c;
  a.H = x.h; a.W = x.w; a.x_pitch = x.pitch;
  a.Ho = y.h; a.Wo = y.w; a.y_pitch = y.pitch; a.r_pitch = res ? res->pitch : 0;
  a.cin_g = cin_g; a.cout = y.c; a.cout_g = cout_g;
  a.k = cs.k; a.stride = cs.stride; a.pad = cs.k / 2; a.act = cs.act;
  const int64_t blocks = (a.total + 255) / 256;
  if (blocks >= (1ll << 31)) return fail(VRS_EBADSHAPE, "grouped conv: grid too large");
  char name[32];
  snprintf(name, sizeof name, "vrs_gconv_%s", dsuffix(cs.dtype));
  hipFunction_t f;
  if ((rc = get_fn(ctx, name, &f))) return rc;
  out.push_back(make_launch(name, f, dim3((unsigned)blocks), dim3(256), 0, a));
  const double es = (double)elt_size(cs.dtype);
  out.back().flops = 2.0 * (double)a.total * cs.k * cs.k * cin_g;
  out.back().bytes = ((double)x.n * x.h * x.w * x.c + (double)a.total * (res ? 2 : 1) +
                      (double)y.c * cs.k * cs.k * cin_g) * es + 8.0 * y.c;
  return VRS_OK;
}

int prep_conv(vrs_ctx* ctx, const ConvSpec& cs, const vrs_nhwc& x, const void* w, const float* scale,
              const float* shift, const vrs_nhwc* res, const vrs_nhwc& y, std::vector<Launch>& out) {
  int rc;
  if (cs.groups > 1 && !cs.depthwise) return prep_grouped(ctx, cs, x, w, scale, shift, res, y, out);
  if ((rc = check_view(y, "conv output", cs.depthwise ? 8 : 4))) return rc;
  if (y.n != x.n) return fail(VRS_EBADSHAPE, "conv: batch mismatch %d vs %d", x.n, y.n);
  if (cs.depthwise) {
    if ((rc = check_dtype(cs.dtype))) return rc;
    if ((rc = check_view(x, "dwconv input", 8))) return rc;
    if (res) return fail(VRS_EUNSUPPORTED, "dwconv: residual not supported");
    if (x.c != y.c) return fail(VRS_EBADSHAPE, "dwconv: channels %d -> %d", x.c, y.c);
    if (cs.k != 3 || (cs.stride != 1 && cs.stride != 2))
      return fail(VRS_EUNSUPPORTED, "dwconv: k=%d s=%d (3x3, stride 1 or 2)", cs.k, cs.stride);
    if (y.h != out_size(x.h, cs.k, cs.stride) || y.w != out_size(x.w, cs.k, cs.stride))
      return fail(VRS_EBADSHAPE, "dwconv: output size");
    if (!w || !scale || !shift) return fail(VRS_EINVAL, "dwconv: null weight/scale/shift");
    vrs_dw_args a{};
    a.x = at(x, cs.dtype); a.w = w; a.scale = scale; a.shift = shift;
    a.y = const_cast<void*>(at(y, cs.dtype));
    a.N = x.n; a.H = x.h; a.W = x.w; a.C = x.c; a.x_pitch = x.pitch;
    a.Ho = y.h; a.Wo = y.w; a.y_pitch = y.pitch;
    a.kh = a.kw = cs.k; a.stride = cs.stride; a.pad = cs.k / 2; a.act = cs.act;
    char name[48];
    hipFunction_t f;
    const int64_t xb = ((int64_t)x.n * x.h * x.w * x.pitch - x.c_off) * (int64_t)elt_size(cs.dtype);
    if (cs.stride == 1 && xb < (1ll << 31)) {
      // row-walking kernel: bands of 40 output rows on maps of 32 rows or
      // more (few band halos and per-wave start-ups: 80 and 40 rows divide
      // evenly), 10 on small ones (enough waves to fill the chip)
      const int rb = x.h >= 32 ? 40 : 10;
      a.x_bytes = (int32_t)xb;
      a.cblocks = (x.c + 63) / 64;
      a.patches = (x.w + 7) / 8;
      a.bands = (x.h + rb - 1) / rb;
      const int64_t wgs = (int64_t)x.n * a.bands * a.cblocks * ((a.patches + 3) / 4);
      if (wgs >= (1ll << 31)) return fail(VRS_EBADSHAPE, "dwconv: grid too large");
      snprintf(name, sizeof name, "vrs_dwconv3_s1w%d_%s", rb, dsuffix(cs.dtype));
      if ((rc = get_fn(ctx, name, &f))) return rc;
      out.push_back(make_launch(name, f, dim3((unsigned)wgs), dim3(256), 0, a));
    } else {
      const int64_t per_img = (int64_t)((y.h + 3) / 4) * y.w * (x.c / 8);
      if (per_img >= (1ll << 24)) return fail(VRS_EBADSHAPE, "dwconv: map too large for one grid row");
      snprintf(name, sizeof name, "vrs_dwconv3_s%d_%s", cs.stride, dsuffix(cs.dtype));
      if ((rc = get_fn(ctx, name, &f))) return rc;
      out.push_back(make_launch(name, f, dim3((unsigned)((per_img + 255) / 256), (unsigned)x.n), dim3(256), 0, a));
    }
    const double es = (double)elt_size(cs.dtype);
    out.back().flops = 2.0 * x.n * y.h * y.w * (double)x.c * cs.k * cs.k;
    out.back().bytes = (double)x.n * x.h * x.w * x.c * es + (double)y.n * y.h * y.w * y.c * es +
                       (double)x.c * (cs.k * cs.k * es + 8.0);
    return VRS_OK;
  }
  vrs_conv_args a{};
  if (res) {
    if ((rc = check_view(*res, "conv residual", 4))) return rc;
    if (res->n != y.n || res->h != y.h || res->w != y.w || res->c != y.c)
      return fail(VRS_EBADSHAPE, "conv: residual shape differs from output");
    if (cs.res_f8 && !pow2_step(cs.res_step))
      return fail(VRS_EINVAL, "conv fp8: res_step %g must be a positive power of two", (double)cs.res_step);
    a.res = cs.res_f8 ? at8(*res) : at(*res, cs.dtype);
    a.r_sb = (int64_t)res->h * res->w * res->pitch; a.r_sp = res->pitch; a.r_sc = 1;
    const int64_t rb = ((int64_t)res->n * res->h * res->w * res->pitch - res->c_off) *
                       (cs.res_f8 ? 1 : (int64_t)elt_size(cs.dtype));
    a.res_bytes = rb < (1ll << 31) ? (int32_t)rb : -1;   // -1: too large for 32-bit buffer offsets
    a.res_f8 = cs.res_f8 ? 1 : 0;
    a.res_step = cs.res_f8 ? cs.res_step : 0.f;
  } else if (cs.res_f8) {
    return fail(VRS_EINVAL, "conv: e4m3 residual flag without a residual");
  }
  a.y = const_cast<void*>(cs.y_f8 ? at8(y) : at(y, cs.dtype));
  a.y_sb = (int64_t)y.h * y.w * y.pitch; a.y_sp = y.pitch; a.y_sc = 1;
  a.y_f32 = 0;
  // 16-byte chunks of 8 (bf16), 4 (f32) or 16 (e4m3) channels must be whole
  // and aligned; the staged stores (and residual loads) address the views
  // with 32-bit raw-buffer byte offsets: pixel m at m * pitch from the view's
  // base
  const int chunk = cs.y_f8 ? 16 : cs.dtype == VRS_F32 ? 4 : 8;
  const int64_t yb = ((int64_t)y.n * y.h * y.w * y.pitch - y.c_off) * (cs.y_f8 ? 1 : (int64_t)elt_size(cs.dtype));
  a.y_bytes = yb < (1ll << 31) ? (int32_t)yb : 0;
  a.stage = (y.c % chunk == 0 && y.c % 8 == 0 && y.c_off % chunk == 0 && y.pitch % chunk == 0 && a.y_bytes > 0 &&
             (!res || a.res_bytes >= 0)) ? 1 : 0;
  return prep_dense(ctx, cs, x, w, scale, shift, y.c, y.h, y.w, a, out);
}

int prep_conv_flat(vrs_ctx* ctx, const ConvSpec& cs, const vrs_nhwc& x, const void* w, const float* scale,
                   const float* shift, int cout, float* y, int64_t sb, int64_t sp, int64_t sc,
                   std::vector<Launch>& out) {
  if (!y) return fail(VRS_EINVAL, "conv: null output");
  vrs_conv_args a{};
  a.y = y; a.y_sb = sb; a.y_sp = sp; a.y_sc = sc; a.y_f32 = 1;
  const int ho = out_size(x.h, cs.k, cs.stride), wo = out_size(x.w, cs.k, cs.stride);
  // bf16 tiles stage a channel-major output (sp == 1) through LDS for 16-byte
  // stores of 4 pixels of one channel: whole pixel quads per image, 16-byte
  // aligned rows, and every touched byte within 32-bit raw-buffer offsets
  const int64_t hw = (int64_t)ho * wo;
  const int64_t last = (int64_t)(x.n - 1) * sb + (hw - 1) * sp + (int64_t)(cout - 1) * sc + 1;
  if (cs.dtype == VRS_BF16 && sp == 1 && hw % 4 == 0 && sb % 4 == 0 && sc % 4 == 0 && sb >= 0 && sc >= 0 &&
      reinterpret_cast<uintptr_t>(y) % 16 == 0 && last * 4 < (1ll << 31)) {
    a.stage = 2;
    a.y_bytes = (int32_t)(last * 4);
  }
  return prep_dense(ctx, cs, x, w, scale, shift, cout, ho, wo, a, out);
}

int prep_pack_input(vrs_ctx* ctx, const float* x, int n, int c, int h, int w, const vrs_nhwc& y, int dtype,
                    std::vector<Launch>& out) {
  int rc;
  if ((rc = check_dtype(dtype))) return rc;
  if (!x) return fail(VRS_EINVAL, "pack_input: null input");
  if (y.c_off != 0 || y.pitch != y.c) return fail(VRS_EBADSHAPE, "pack_input: output must be a whole buffer");
  if (y.n != n || y.h != h || y.w != w || y.c < c || y.c >= c + 8)
    return fail(VRS_EBADSHAPE, "pack_input: output view %dx%dx%dx%d for input %dx%dx%dx%d (c padded by < 8)", y.n,
                y.h, y.w, y.c, n, c, h, w);
  vrs_pack_args a{x, y.data, n, c, h, w, y.c};
  char name[48];
  snprintf(name, sizeof name, "vrs_pack_nchw_%s", dsuffix(dtype));
  hipFunction_t f;
  if ((rc = get_fn(ctx, name, &f))) return rc;
  const int64_t threads = (int64_t)n * h * w;
  out.push_back(make_launch(name, f, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, a));
  out.back().bytes = (double)n * h * w * (4.0 * c + (double)y.c * elt_size(dtype));
  return VRS_OK;
}

int prep_unpack(vrs_ctx* ctx, const vrs_nhwc& x, int dtype, float* y, std::vector<Launch>& out) {
  int rc;
  if ((rc = check_dtype(dtype))) return rc;
  if ((rc = check_view(x, "unpack input", 1))) return rc;
  if (!y) return fail(VRS_EINVAL, "unpack: null output");
  vrs_pack_args a{};
  a.x = static_cast<const float*>(at(x, dtype));
  a.y = y;
  a.N = x.n; a.C = x.c; a.H = x.h; a.W = x.w; a.c_pad = x.pitch;
  char name[48];
  snprintf(name, sizeof name, "vrs_unpack_nchw_%s", dsuffix(dtype));
  hipFunction_t f;
  if ((rc = get_fn(ctx, name, &f))) return rc;
  const int64_t threads = (int64_t)x.n * x.c * x.h * x.w;
  out.push_back(make_launch(name, f, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, a));
  out.back().bytes = (double)threads * (4.0 + elt_size(dtype));
  return VRS_OK;
}

int prep_pool(vrs_ctx* ctx, const vrs_nhwc& buf, int dtype, std::vector<Launch>& out) {
  int rc;
  if ((rc = check_dtype(dtype))) return rc;
  if ((rc = check_view(buf, "sppf buffer", 8))) return rc;
  if (buf.c % 32) return fail(VRS_EBADSHAPE, "sppf: view must hold 4*c channels with c %% 8 == 0");
  const int c = buf.c / 4;
  const int hw = buf.h * buf.w;
  if (dtype == VRS_BF16 && (int64_t)3 * hw * 16 <= 64 * 1024) {
    // wave-per-channel-group kernel: three LDS planes of 16-byte pixels per
    // wave, four waves per workgroup when two such workgroups fit a CU's
    // 160 KB, else two when they fit 64 KB
    const int64_t plane3 = 3ll * hw * 16;
    const int G = (c / 8) % 4 == 0 && 4 * plane3 <= 80 * 1024 ? 4 : 2 * plane3 <= 64 * 1024 ? 2 : 1;
    vrs_pool_args a{};
    a.buf = const_cast<void*>(at(buf, dtype));
    a.N = buf.n; a.H = buf.h; a.W = buf.w; a.c = c; a.pitch = buf.pitch; a.cgroups_per_block = 1;
    const int64_t waves = (int64_t)buf.n * (c / 8);
    if ((waves + G - 1) / G >= (1ll << 31)) return fail(VRS_EBADSHAPE, "sppf: grid too large");
    char name[48];
    snprintf(name, sizeof name, "vrs_sppf_pool_w%d_bf16", G);
    hipFunction_t f;
    if ((rc = get_fn(ctx, name, &f))) return rc;
    out.push_back(make_launch(name, f, dim3((unsigned)((waves + G - 1) / G)), dim3(64 * G), (uint32_t)(G * 3 * hw * 16),
                              a));
    out.back().bytes = 4.0 * buf.n * hw * (double)c * elt_size(dtype);
    return VRS_OK;
  }
  const int64_t per_group = 2ll * hw * 8 * (int64_t)elt_size(dtype);
  // 64 KB of planes per workgroup, or up to the CU's 160 KB for one group of
  // a large map (one workgroup per CU then)
  const int64_t budget = per_group <= 64 * 1024 ? 64 * 1024 : 160 * 1024;
  int cg = (int)std::min<int64_t>(c / 8, budget / per_group);
  if (cg < 1) return fail(VRS_EUNSUPPORTED, "sppf: %dx%d map does not fit the LDS plane", buf.h, buf.w);
  // a power of two of channel groups per workgroup: each pixel's writes then
  // cover whole 64-byte spans where the budget allows (at 3 groups, 48-byte
  // spans cost 1.8x the algorithmic HBM bytes in partial-line traffic)
  while (cg & (cg - 1)) cg &= cg - 1;
  vrs_pool_args a{};
  a.buf = const_cast<void*>(at(buf, dtype));
  a.N = buf.n; a.H = buf.h; a.W = buf.w; a.c = c; a.pitch = buf.pitch; a.cgroups_per_block = cg;
  const int blocks_per_img = (c / 8 + cg - 1) / cg;
  char name[48];
  snprintf(name, sizeof name, "vrs_sppf_pool_%s", dsuffix(dtype));
  hipFunction_t f;
  if ((rc = get_fn(ctx, name, &f))) return rc;
  out.push_back(make_launch(name, f, dim3(buf.n * blocks_per_img), dim3(256), (uint32_t)(cg * per_group), a));
  out.back().bytes = 4.0 * buf.n * hw * (double)c * elt_size(dtype);
  return VRS_OK;
}

int prep_up(vrs_ctx* ctx, const vrs_nhwc& x, const vrs_nhwc& y, int dtype, std::vector<Launch>& out) {
  int rc;
  if ((rc = check_dtype(dtype))) return rc;
  if ((rc = check_view(x, "upsample input", 8)) || (rc = check_view(y, "upsample output", 8))) return rc;
  if (y.n != x.n || y.h != 2 * x.h || y.w != 2 * x.w || y.c != x.c)
    return fail(VRS_EBADSHAPE, "upsample2x: output must be [n, 2h, 2w, c]");
  vrs_up_args a{at(x, dtype), const_cast<void*>(at(y, dtype)), x.n, x.h, x.w, x.c, x.pitch, y.pitch};
  char name[48];
  snprintf(name, sizeof name, "vrs_upsample2x_%s", dsuffix(dtype));
  hipFunction_t f;
  if ((rc = get_fn(ctx, name, &f))) return rc;
  const int64_t threads = (int64_t)y.n * y.h * y.w * (y.c / 8);
  out.push_back(make_launch(name, f, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, a));
  out.back().bytes = 5.0 * x.n * x.h * x.w * (double)x.c * elt_size(dtype);
  return VRS_OK;
}

int prep_attn(vrs_ctx* ctx, int heads, int dtype, const vrs_nhwc& qkv, const void* pe_w, const float* pe_scale,
              const float* pe_shift, const vrs_nhwc& o, std::vector<Launch>& out) {
  int rc;
  if ((rc = check_dtype(dtype))) return rc;
  if ((rc = check_view(qkv, "psa qkv", 8)) || (rc = check_view(o, "psa out", 4))) return rc;
  if (heads < 1 || qkv.c != heads * 128 || o.c != heads * 64)
    return fail(VRS_EBADSHAPE, "psa: heads=%d needs qkv %d and out %d channels", heads, heads * 128, heads * 64);
  if (o.n != qkv.n || o.h != qkv.h || o.w != qkv.w) return fail(VRS_EBADSHAPE, "psa: out/qkv spatial mismatch");
  if (!pe_w || !pe_scale || !pe_shift) return fail(VRS_EINVAL, "psa: null pe parameters");
  vrs_attn_args a{};
  a.qkv = at(qkv, dtype); a.pe_w = pe_w; a.pe_scale = pe_scale; a.pe_shift = pe_shift;
  a.out = const_cast<void*>(at(o, dtype));
  a.B = qkv.n; a.H = qkv.h; a.W = qkv.w; a.heads = heads; a.qkv_pitch = qkv.pitch; a.out_pitch = o.pitch;
  a.scale_log2e = (float)(1.0 / std::sqrt(32.0) * 1.4426950408889634);
  const int N = qkv.h * qkv.w;
  {
    const int64_t qb = ((int64_t)qkv.n * qkv.h * qkv.w * qkv.pitch - qkv.c_off) * (int64_t)elt_size(dtype);
    a.qkv_bytes = qb < (1ll << 31) ? (int32_t)qb : 0;   // 0: the resident kernel is not used
  }
  char name[48];
  int threads;
  if (dtype == VRS_BF16 && N <= 512 && a.qkv_bytes > 0) {
    // the head's K and V^T resident in LDS, one wave per 32 queries: tiles
    // of 7 query tiles (two workgroups per 20x20 head) while those fit in
    // one round over the CUs, else one workgroup per head (at 20x20 and
    // 4 heads: 17.3 vs 24.1 us at batch 32, 30.1 vs 24.6 us at batch 48)
    const int tiles = (N + 31) / 32;
    const int ncu = ctx->num_cu > 0 ? ctx->num_cu : 256;
    int qt = 7;
    if ((int64_t)a.B * heads * ((tiles + 6) / 7) > ncu) qt = tiles <= 7 ? 7 : tiles <= 13 ? 13 : 16;
    a.q_blocks = (tiles + qt - 1) / qt;
    threads = qt * 64;
    snprintf(name, sizeof name, "vrs_psa_attn_res%d_bf16", qt);
  } else {
    a.q_blocks = (N + 79) / 80;  // streamed K/V: 5 waves x 16 queries per workgroup
    threads = 320;
    snprintf(name, sizeof name, "vrs_psa_attn_%s", dsuffix(dtype));
  }
  if ((int64_t)a.B * heads * a.q_blocks >= (1ll << 31)) return fail(VRS_EBADSHAPE, "psa: grid too large");
  hipFunction_t f;
  if ((rc = get_fn(ctx, name, &f))) return rc;
  out.push_back(make_launch(name, f, dim3(a.B * heads * a.q_blocks), dim3(threads), 0, a));
  const double Nd = (double)N;
  out.back().flops = 2.0 * a.B * heads * Nd * Nd * (32 + 64) + 2.0 * a.B * Nd * o.c * 9;
  out.back().bytes = (double)a.B * Nd * (qkv.c + o.c) * elt_size(dtype) + (double)o.c * (9 * elt_size(dtype) + 8);
  return VRS_OK;
}

int prep_absmax(vrs_ctx* ctx, const vrs_nhwc& x, unsigned* out, std::vector<Launch>& ls) {
  int rc;
  if ((rc = check_view(x, "absmax input", 8))) return rc;
  vrs_absmax_args a{};
  a.x = at(x, VRS_BF16);
  a.out = out;
  a.npix = (int64_t)x.n * x.h * x.w;
  a.c = x.c;
  a.pitch = x.pitch;
  hipFunction_t f;
  if ((rc = get_fn(ctx, "vrs_absmax_bf16", &f))) return rc;
  const int64_t items = a.npix * (x.c / 8);
  const int64_t cap = 8ll * (ctx->num_cu > 0 ? ctx->num_cu : 256);
  const int64_t blocks = std::min<int64_t>(cap, (items + 255) / 256);
  ls.push_back(make_launch("vrs_absmax_bf16", f, dim3((unsigned)std::max<int64_t>(1, blocks)), dim3(256), 0, a));
  ls.back().bytes = (double)items * 16.0;
  return VRS_OK;
}


int prep_stem(vrs_ctx* ctx, int act, int dtype, const float* x, int n, int h, int w, const void* wp,
              const float* scale, const float* shift, int cout, const vrs_nhwc& y, std::vector<Launch>& ls) {
  int rc;
  if ((rc = check_dtype(dtype))) return rc;
  if (!x || !wp || !scale || !shift) return fail(VRS_EINVAL, "stem: null argument");
  if (reinterpret_cast<uintptr_t>(x) % 16) return fail(VRS_EBADSHAPE, "stem: image not 16-byte aligned");
  if ((rc = check_view(y, "stem output", 4))) return rc;
  const int ho = out_size(h, 3, 2), wo = out_size(w, 3, 2);
  if (y.n != n || y.h != ho || y.w != wo || y.c != cout)
    return fail(VRS_EBADSHAPE, "stem: output view %dx%dx%dx%d for input %dx3x%dx%d, cout %d", y.n, y.h, y.w, y.c, n,
                h, w, cout);
  if (cout < 8 || cout > 128 || cout % 8) return fail(VRS_EUNSUPPORTED, "stem: cout %d (8..128, multiple of 8)", cout);
  if (y.pitch % 8 || y.c_off % 8) return fail(VRS_EBADSHAPE, "stem: output pitch/offset must be multiples of 8");
  vrs_stem_args a{};
  a.x = x; a.w = wp; a.scale = scale; a.shift = shift; a.y = const_cast<void*>(at(y, dtype));
  a.N = n; a.H = h; a.W = w; a.Ho = ho; a.Wo = wo; a.cout = cout; a.cout_pad = (cout + 31) / 32 * 32;
  a.y_pitch = y.pitch; a.act = act;
  a.segs = (wo + 63) / 64;
  const int64_t items = (int64_t)n * ((ho + 1) / 2) * a.segs;   // 2 output rows x 64 pixels each
  if (items >= (1ll << 31)) return fail(VRS_EBADSHAPE, "stem: grid too large");
  // persistent grid: the resident workgroups loop over the items
  if ((int64_t)3 * h * w * 4 >= (1ll << 31) || (int64_t)ho * wo * y.pitch * (int64_t)elt_size(dtype) >= (1ll << 31))
    return fail(VRS_EBADSHAPE, "stem: one image (in or out) must be under 2 GiB");
  char name[32];
  snprintf(name, sizeof name, "vrs_stem_%s_c%d%s", dsuffix(dtype), a.cout_pad / 32, w % 4 ? "_u" : "");
  hipFunction_t f;
  if ((rc = get_fn(ctx, name, &f))) return rc;
  // persistent grid: the resident workgroups loop over the items
  const int64_t wgs = std::min<int64_t>(items, (int64_t)resident_wgs(f) * (ctx->num_cu > 0 ? ctx->num_cu : 256));
  ls.push_back(make_launch(name, f, dim3((unsigned)wgs), dim3(256), 0, a));
  const double es = (double)elt_size(dtype);
  ls.back().flops = 2.0 * n * ho * wo * (double)cout * 27;
  ls.back().bytes = (double)n * 3 * h * w * 4 + (double)n * ho * wo * cout * es + (double)cout * 27 * es + 8.0 * cout;
  return VRS_OK;
}

int stem_pair_check(int dtype, int act0, int act1, int h, int w) {
  if (dtype != VRS_BF16) return fail(VRS_EUNSUPPORTED, "stem pair: bf16 only");
  if (act0 != VRS_ACT_SILU || act1 != VRS_ACT_SILU) return fail(VRS_EUNSUPPORTED, "stem pair: SiLU on both layers only");
  if (w % 4) return fail(VRS_EUNSUPPORTED, "stem pair: image width %d not a multiple of 4", w);
  if ((int64_t)3 * h * w * 4 >= (1ll << 31)) return fail(VRS_EBADSHAPE, "stem pair: one image must be under 2 GiB");
  return VRS_OK;
}

int prep_stem_pair(vrs_ctx* ctx, const float* x, int n, int h, int w, const void* w0, const float* scale0,
                   const float* shift0, const void* w1, const float* scale1, const float* shift1, const vrs_nhwc& y,
                   std::vector<Launch>& ls) {
  int rc;
  if ((rc = stem_pair_check(VRS_BF16, VRS_ACT_SILU, VRS_ACT_SILU, h, w))) return rc;
  if (!x || !w0 || !scale0 || !shift0 || !w1 || !scale1 || !shift1) return fail(VRS_EINVAL, "stem pair: null argument");
  if (reinterpret_cast<uintptr_t>(x) % 16) return fail(VRS_EBADSHAPE, "stem pair: image not 16-byte aligned");
  if ((rc = check_view(y, "stem pair output", 8))) return rc;
  const int h0 = out_size(h, 3, 2), w0o = out_size(w, 3, 2);
  const int h1 = out_size(h0, 3, 2), w1o = out_size(w0o, 3, 2);
  if (y.n != n || y.h != h1 || y.w != w1o || y.c != 128)
    return fail(VRS_EBADSHAPE, "stem pair: output view %dx%dx%dx%d for input %dx3x%dx%d (expects %dx%dx%dx128)", y.n,
                y.h, y.w, y.c, n, h, w, n, h1, w1o);
  if ((int64_t)h1 * w1o * y.pitch * 2 >= (1ll << 31))
    return fail(VRS_EBADSHAPE, "stem pair: one output image must be under 2 GiB");
  vrs_stem_pair_args a{};
  a.x = x; a.w0 = w0; a.scale0 = scale0; a.shift0 = shift0;
  a.w1 = w1; a.scale1 = scale1; a.shift1 = shift1;
  a.y = const_cast<void*>(at(y, VRS_BF16));
  a.N = n; a.H = h; a.W = w; a.H0 = h0; a.W0 = w0o; a.H1 = h1; a.W1 = w1o; a.y_pitch = y.pitch;
  a.strips = (w1o + 31) / 32;
  a.sps = (h1 + 1) / 2;
  const int64_t total = (int64_t)n * a.strips * a.sps;
  if (total >= (1ll << 31)) return fail(VRS_EBADSHAPE, "stem pair: grid too large");
  a.total = (int32_t)total;
  const char* name = "vrs_stem_pair_bf16";
  hipFunction_t f;
  if ((rc = get_fn(ctx, name, &f))) return rc;
  // persistent: one workgroup per CU, each walking total / grid consecutive steps
  const int64_t wgs = std::min<int64_t>(total, (int64_t)resident_wgs(f, 512) * (ctx->num_cu > 0 ? ctx->num_cu : 256));
  ls.push_back(make_launch(name, f, dim3((unsigned)wgs), dim3(512), 0, a));
  ls.back().flops = 2.0 * n * h0 * w0o * 64.0 * 27 + 2.0 * n * h1 * w1o * 128.0 * 576;
  ls.back().bytes = (double)n * 3 * h * w * 4 + (double)n * h1 * w1o * 128 * 2 + 64.0 * 32 * 2 + 128.0 * 576 * 2 +
                    8.0 * (64 + 128);
  return VRS_OK;
}

// Bottleneck pair (bpair.hip): the channel counts it is built for.
int bpair_check(int dtype, int act1, int act2, int cin, int ch, int cout) {
  if (dtype != VRS_BF16) return fail(VRS_EUNSUPPORTED, "bottleneck pair: bf16 only");
  if (act1 != VRS_ACT_SILU || act2 != VRS_ACT_SILU)
    return fail(VRS_EUNSUPPORTED, "bottleneck pair: BN + SiLU on both convs only");
  if (cin != 64 || ch != 32 || cout != 64)
    return fail(VRS_EUNSUPPORTED, "bottleneck pair: built for 64 -> 32 -> 64 channels (got %d -> %d -> %d)", cin, ch,
                cout);
  return VRS_OK;
}

int prep_bpair(vrs_ctx* ctx, const vrs_nhwc& x, const void* w1, const float* s1, const float* b1, int ch,
               const void* w2, const float* s2, const float* b2, const vrs_nhwc* res, const vrs_nhwc& y,
               std::vector<Launch>& ls) {
  int rc;
  if ((rc = bpair_check(VRS_BF16, VRS_ACT_SILU, VRS_ACT_SILU, x.c, ch, y.c))) return rc;
  if (!w1 || !s1 || !b1 || !w2 || !s2 || !b2) return fail(VRS_EINVAL, "bottleneck pair: null weight/scale/shift");
  if ((rc = check_view(x, "bottleneck pair input", 8)) || (rc = check_view(y, "bottleneck pair output", 8)) ||
      (res && (rc = check_view(*res, "bottleneck pair residual", 8))))
    return rc;
  if (y.n != x.n || y.h != x.h || y.w != x.w)
    return fail(VRS_EBADSHAPE, "bottleneck pair: output %dx%dx%d for input %dx%dx%d (3x3 stride 1 keeps the size)",
                y.n, y.h, y.w, x.n, x.h, x.w);
  if (res && (res->n != y.n || res->h != y.h || res->w != y.w || res->c != y.c))
    return fail(VRS_EBADSHAPE, "bottleneck pair: residual shape differs from the output");
  auto extent = [](const vrs_nhwc& v) { return ((int64_t)v.n * v.h * v.w * v.pitch - v.c_off) * 2; };
  const int64_t xb = extent(x), yb = extent(y), rb = res ? extent(*res) : 0;
  if (xb >= (1ll << 31) || yb >= (1ll << 31) || rb >= (1ll << 31))
    return fail(VRS_EBADSHAPE, "bottleneck pair: views must be under 2 GiB (32-bit buffer offsets)");
  vrs_bpair_args a{};
  a.x = at(x, VRS_BF16);
  a.w1 = w1; a.s1 = s1; a.b1 = b1;
  a.w2 = w2; a.s2 = s2; a.b2 = b2;
  a.res = res ? at(*res, VRS_BF16) : nullptr;
  a.y = const_cast<void*>(at(y, VRS_BF16));
  a.N = x.n; a.H = x.h; a.W = x.w;
  a.x_pitch = x.pitch; a.y_pitch = y.pitch; a.r_pitch = res ? res->pitch : 0;
  a.strips = (x.w + 31) / 32;   // 32-pixel strips, runs of 8 rows (256 output pixels)
  a.runs = (x.h + 7) / 8;
  a.x_bytes = (int32_t)xb; a.y_bytes = (int32_t)yb; a.res_bytes = (int32_t)rb;
  a.w1_bytes = ch * 9 * x.c * 2;
  a.w2_bytes = y.c * 9 * ch * 2;
  const int64_t blocks = (int64_t)x.n * a.strips * a.runs;
  if (blocks >= (1ll << 31)) return fail(VRS_EBADSHAPE, "bottleneck pair: grid too large");
  const char* name = "vrs_bpair_bf16_c64_h32_w32";
  hipFunction_t f;
  if ((rc = get_fn(ctx, name, &f))) return rc;
  ls.push_back(make_launch(name, f, dim3((unsigned)blocks), dim3(256), 0, a));
  const double M = (double)x.n * x.h * x.w;
  ls.back().flops = 2.0 * M * 9.0 * ((double)x.c * ch + (double)ch * y.c);
  ls.back().bytes = M * x.c * 2.0 + M * y.c * 2.0 + (res ? M * y.c * 2.0 : 0.0) + 2.0 * 9.0 * x.c * ch * 2.0 +
                    8.0 * (ch + y.c);
  return VRS_OK;
}

// Pointwise pair (pwpair.hip): the shapes it is built for.
int pwpair_check(int dtype, int act1, int act2, int cin, int cm, int nc) {
  if (dtype != VRS_BF16) return fail(VRS_EUNSUPPORTED, "pointwise pair: bf16 only");
  if (act1 != VRS_ACT_SILU || act2 != VRS_ACT_NONE)
    return fail(VRS_EUNSUPPORTED, "pointwise pair: BN + SiLU on the first conv, none on the second");
  if (cin != 256 || cm != 256 || nc < 1 || nc > 96)
    return fail(VRS_EUNSUPPORTED, "pointwise pair: built for 256 -> 256 -> (1..96) channels (got %d -> %d -> %d)",
                cin, cm, nc);
  return VRS_OK;
}

int prep_pwpair(vrs_ctx* ctx, const vrs_nhwc& x, const void* w1, const float* s1, const float* b1, int cm,
                const void* w2, const float* s2, const float* b2, int nc, float* y, int64_t sb, int64_t sp,
                int64_t sc, std::vector<Launch>& ls) {
  int rc;
  if ((rc = pwpair_check(VRS_BF16, VRS_ACT_SILU, VRS_ACT_NONE, x.c, cm, nc))) return rc;
  if (!w1 || !s1 || !b1 || !w2 || !s2 || !b2 || !y) return fail(VRS_EINVAL, "pointwise pair: null pointer");
  if ((rc = check_view(x, "pointwise pair input", 8))) return rc;
  const int64_t M = (int64_t)x.n * x.h * x.w, hw = (int64_t)x.h * x.w;
  const int64_t xb = (M * x.pitch - x.c_off) * 2;
  if (sb < 0 || sp < 1 || sc < 1) return fail(VRS_EBADSHAPE, "pointwise pair: output strides must be positive");
  const int64_t last = (x.n - 1) * sb + (hw - 1) * sp + (int64_t)(nc - 1) * sc + 1;
  if (M >= (1ll << 31) || xb >= (1ll << 31) || last * 4 >= (1ll << 31))
    return fail(VRS_EBADSHAPE, "pointwise pair: input and output must be under 2 GiB (32-bit buffer offsets)");
  vrs_pwpair_args a{};
  a.x = at(x, VRS_BF16);
  a.w1 = w1; a.s1 = s1; a.b1 = b1;
  a.w2 = w2; a.s2 = s2; a.b2 = b2;
  a.y = y;
  a.y_sb = sb; a.y_sp = sp; a.y_sc = sc;
  a.M = (int32_t)M; a.HW = (int32_t)hw; a.NC = nc;
  a.x_pitch = x.pitch; a.x_bytes = (int32_t)xb; a.y_bytes = (int32_t)(last * 4);
  // maps of at least two tiles per CU: the weight-stationary persistent
  // kernel (one 8-wave group per CU, W1 and W2 in registers); smaller ones:
  // one 4-wave group per 64-pixel tile, two per CU (measured at YOLO26m
  // bs64: 80x80 104 vs 224 us, 40x40 34 vs 57 us)
  const int64_t tiles = (M + 63) / 64;
  const bool ws = tiles >= 2ll * ctx->num_cu;
  const char* name = ws ? "vrs_pwpair_w_bf16_c256_m256" : "vrs_pwpair_bf16_c256_m256";
  hipFunction_t f;
  if ((rc = get_fn(ctx, name, &f))) return rc;
  ls.push_back(make_launch(name, f, dim3((unsigned)(ws ? ctx->num_cu : tiles)), dim3(ws ? 512 : 256), 0, a));
  ls.back().flops = 2.0 * M * ((double)x.c * cm + (double)cm * nc);
  ls.back().bytes = M * x.c * 2.0 + M * nc * 4.0 + ((double)cm * x.c + (double)nc * cm) * 2.0 + 8.0 * (cm + nc);
  return VRS_OK;
}

}  // namespace vrs

using namespace vrs;

extern "C" {

const char* vrs_last_error(void) { return g_err.c_str(); }
const char* vrs_version(void) { return "vrs 0.1 gfx950"; }

int vrs_ctx_create(int device, const char* hsaco_dir, vrs_ctx** out) {
  if (!out || !hsaco_dir) return fail(VRS_EINVAL, "vrs_ctx_create: null argument");
  *out = nullptr;
  DIR* d = opendir(hsaco_dir);
  if (!d) return fail(VRS_ENOMODULE, "code-object directory %s not found", hsaco_dir);
  std::vector<std::string> files;
  while (dirent* e = readdir(d)) {
    std::string n = e->d_name;
    if (n.size() > 6 && n.compare(n.size() - 6, 6, ".hsaco") == 0) files.push_back(std::string(hsaco_dir) + "/" + n);
  }
  closedir(d);
  if (files.empty()) return fail(VRS_ENOMODULE, "no .hsaco code objects under %s", hsaco_dir);
  int ndev = 0;
  VRS_HIP(hipGetDeviceCount(&ndev));
  if (device < 0 || device >= ndev) return fail(VRS_EINVAL, "device %d out of range (%d devices)", device, ndev);
  VRS_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  VRS_HIP(hipGetDeviceProperties(&prop, device));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(VRS_EUNSUPPORTED, "device %d is %s; this build targets gfx950 only", device, prop.gcnArchName);
  auto* ctx = new vrs_ctx;
  ctx->device = device;
  ctx->dir = hsaco_dir;
  ctx->num_cu = prop.multiProcessorCount;
  for (const auto& f : files) {
    hipModule_t m = nullptr;
    hipError_t e = hipModuleLoad(&m, f.c_str());
    if (e != hipSuccess) {
      for (auto mm : ctx->modules) (void)hipModuleUnload(mm);
      delete ctx;
      return fail(VRS_ENOMODULE, "hipModuleLoad(%s): %s", f.c_str(), hipGetErrorString(e));
    }
    ctx->modules.push_back(m);
  }
  scratch_attach(ctx);   // device address of the fixed detect workspace on this device
  *out = ctx;
  return VRS_OK;
}

int vrs_ctx_destroy(vrs_ctx* ctx) {
  if (!ctx) return VRS_OK;
  for (auto m : ctx->modules) (void)hipModuleUnload(m);
  delete ctx;
  return VRS_OK;
}

}  // extern "C"

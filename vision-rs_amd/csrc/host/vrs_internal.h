// Internal declarations of the host runtime behind include/vrs.h.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "../kargs.h"
#include "vrs.h"

struct vrs_ctx {
  int device = 0;
  std::string dir;
  std::vector<hipModule_t> modules;
  std::unordered_map<std::string, hipFunction_t> fns;
  int num_cu = 0;
  // device address of the library's fixed detect workspace on this device
  // (scratch.hip; null with the reason in scratch_err if the lookup failed)
  void* scratch = nullptr;
  std::string scratch_err;
};

namespace vrs {

// Thread-local error text; returns `code` so callers can `return fail(...)`.
int fail(int code, const char* fmt, ...);
int hip_check(hipError_t e, const char* what);
#define VRS_HIP(call)                                       \
  do {                                                      \
    hipError_t e_ = (call);                                 \
    if (e_ != hipSuccess) return ::vrs::hip_check(e_, #call); \
  } while (0)

// safetensors file in memory (safetensors.cpp): tensor table and raw bytes.
struct StTensor {
  std::string dtype;
  std::vector<int64_t> shape;
  size_t begin = 0, end = 0;   // byte range relative to the data section
  int64_t numel = 0;
};
struct StFile {
  std::vector<char> bytes;
  size_t data_begin = 0;
  std::unordered_map<std::string, StTensor> tensors;
};
int st_open(const char* path, StFile& f);
const StTensor* st_find(const StFile& f, const std::string& name);
int st_to_f32(const StFile& f, const std::string& name, const StTensor& t, std::vector<float>& out);

// Fixed device workspace of vrs_detect_postprocess_noalloc: look up this
// device's copy (ctx->device current) at context creation (scratch.hip).
void scratch_attach(vrs_ctx* ctx);
// Detect descriptor checks and anchor count shared by both post-process
// entry points (ops.cpp).
int det_check(const vrs_detect_desc* d);
int64_t det_anchors(const vrs_detect_desc* d);

// Resolve a kernel by name from the loaded code objects.
int get_fn(vrs_ctx* ctx, const char* name, hipFunction_t* out);

// One prepared kernel launch: everything hipModuleLaunchKernel needs, with the
// argument block stored by value so it can be replayed or captured.
struct Launch {
  std::string name;
  hipFunction_t fn = nullptr;
  dim3 grid, block;
  uint32_t shmem = 0;
  std::vector<uint8_t> args;
  double flops = 0.0;  // algorithmic work of this launch
  double bytes = 0.0;  // compulsory HBM bytes (inputs + weights + outputs)
};

int run(const Launch& l, hipStream_t s);

template <typename A>
Launch make_launch(const char* name, hipFunction_t fn, dim3 grid, dim3 block, uint32_t shmem, const A& a) {
  Launch l;
  l.name = name;
  l.fn = fn;
  l.grid = grid;
  l.block = block;
  l.shmem = shmem;
  l.args.resize(sizeof(A));
  memcpy(l.args.data(), &a, sizeof(A));
  return l;
}

inline size_t elt_size(int dtype) { return dtype == VRS_F32 ? 4 : 2; }
inline const char* dsuffix(int dtype) { return dtype == VRS_F32 ? "f32" : "bf16"; }

// Prepare (validate + fill) launches.  Each returns VRS_OK or an error and
// appends to `out`.  Pointers in views are device addresses.
struct ConvSpec {
  int k = 1, stride = 1, act = VRS_ACT_NONE, dtype = VRS_BF16;
  bool depthwise = false;
  // 1 < groups < channels (not depthwise): per-group channel slices
  int groups = 1;
  int cin_real = 0;  // unpadded input channels for work accounting (0: the view's)
  int tile = VRS_TILE_AUTO;  // dense conv tile (VRS_TILE_*)
  float in_scale = 1.f;      // VRS_FP8: activation quantisation step (power of two)
  // VRS_FP8 with e4m3 activations in memory: x (and the fused-upsample
  // source) hold e4m3 bytes on in_scale; y is written as e4m3 on out_step;
  // res holds e4m3 bytes on res_step
  bool x_f8 = false, y_f8 = false, res_f8 = false;
  float out_step = 0.f, res_step = 0.f;
  // fused nearest-2x upsample (1x1 stride-1 dense convs): input channels
  // [0, up->c) are read from this half-resolution view instead of x
  const vrs_nhwc* up = nullptr;
};
// stem conv (3x3 s2, Cin 3) straight from the NCHW float32 image; weights
// packed by vrs_pack_stem_weight
int prep_stem(vrs_ctx* ctx, int act, int dtype, const float* x, int n, int h, int w, const void* wp,
              const float* scale, const float* shift, int cout, const vrs_nhwc& y, std::vector<Launch>& ls);
// stem pair (model.0 + model.1, 64 -> 128 channels, bf16, SiLU) in one
// kernel from the NCHW float32 image; w0 from vrs_pack_stem_weight, w1 the
// dense [128][3][3][64] packing.  stem_pair_check: the shape/type conditions.
int stem_pair_check(int dtype, int act0, int act1, int h, int w);
int prep_stem_pair(vrs_ctx* ctx, const float* x, int n, int h, int w, const void* w0, const float* scale0,
                   const float* shift0, const void* w1, const float* scale1, const float* shift1, const vrs_nhwc& y,
                   std::vector<Launch>& ls);
// bottleneck pair (3x3 -> 3x3 + residual, bf16, SiLU on both) in one kernel:
// x the block input (C channels), w1 [ch][3][3][C], w2 [C][3][3][ch], res
// optional, y (C channels); bpair_check: the channel counts built
int bpair_check(int dtype, int act1, int act2, int cin, int ch, int cout);
// Pointwise pair (pwpair.hip): 1x1 BN+SiLU conv cin -> cm, then a plain 1x1
// cm -> nc into a float32 flat output y[b*sb + p*sp + c*sc].
int pwpair_check(int dtype, int act1, int act2, int cin, int cm, int nc);
int prep_pwpair(vrs_ctx* ctx, const vrs_nhwc& x, const void* w1, const float* s1, const float* b1, int cm,
                const void* w2, const float* s2, const float* b2, int nc, float* y, int64_t sb, int64_t sp,
                int64_t sc, std::vector<Launch>& ls);
int prep_bpair(vrs_ctx* ctx, const vrs_nhwc& x, const void* w1, const float* s1, const float* b1, int ch,
               const void* w2, const float* s2, const float* b2, const vrs_nhwc* res, const vrs_nhwc& y,
               std::vector<Launch>& ls);
// max |x| of a bfloat16 NHWC view into *out (float bits; caller zeroes it)
int prep_absmax(vrs_ctx* ctx, const vrs_nhwc& x, unsigned* out, std::vector<Launch>& ls);
// float -> e4m3 (OCP, max 448) with round-to-nearest-even; |v| > 448 saturates
uint8_t f32_to_e4m3(float v);
// Dense conv tiles worth trying for a layer (autotuning candidates).
// m: output pixels (0: unknown), num_cu: the device's CUs
std::vector<int> conv_tile_candidates(int cout, int cin, int dtype, int k, int stride, int w, int64_t m, int num_cu);
int prep_conv(vrs_ctx* ctx, const ConvSpec& cs, const vrs_nhwc& x, const void* w, const float* scale,
              const float* shift, const vrs_nhwc* res, const vrs_nhwc& y, std::vector<Launch>& out);
// Dense conv storing float32 into a strided (flat) output: element (b, p, co)
// at y + b*sb + p*sp + co*sc (the Detect head's channel_cat_flat layout).
int prep_conv_flat(vrs_ctx* ctx, const ConvSpec& cs, const vrs_nhwc& x, const void* w, const float* scale,
                   const float* shift, int cout, float* y, int64_t sb, int64_t sp, int64_t sc,
                   std::vector<Launch>& out);
int prep_pack_input(vrs_ctx* ctx, const float* x, int n, int c, int h, int w, const vrs_nhwc& y, int dtype,
                    std::vector<Launch>& out);
int prep_unpack(vrs_ctx* ctx, const vrs_nhwc& x, int dtype, float* y, std::vector<Launch>& out);
int prep_pool(vrs_ctx* ctx, const vrs_nhwc& buf, int dtype, std::vector<Launch>& out);
int prep_up(vrs_ctx* ctx, const vrs_nhwc& x, const vrs_nhwc& y, int dtype, std::vector<Launch>& out);
int prep_attn(vrs_ctx* ctx, int heads, int dtype, const vrs_nhwc& qkv, const void* pe_w, const float* pe_scale,
              const float* pe_shift, const vrs_nhwc& o, std::vector<Launch>& out);

}  // namespace vrs

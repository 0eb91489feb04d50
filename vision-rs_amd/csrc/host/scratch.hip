// Allocation-free detect post-process: vrs_detect_postprocess with its
// workspace in a fixed device array of this library instead of a caller or
// hipMalloc buffer.  For callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  No counterpart in the reference, whose decode/score/sort runs
// on the host (examples/yolo26.rs:1488-1529).
//
// The array lives in this library's own gfx950 code object (this file is
// compiled as HIP into libvrs.so); each GPU holds its own copy until the
// process ends.  Host code never uses the array's name as an address: at
// context creation the device copy's address is looked up once per device
// with hipGetSymbolAddress and kept; the stage-1/stage-2 kernels (loaded
// from detect.hsaco) receive that address as their workspace argument.
//
// Every call on one GPU uses the same array, which keeps the previous call's
// contents: calls that overlap in time on one GPU (other streams, threads or
// contexts) race.  Nothing needs clearing: stage 1 writes every key, class and
// box slot that stage 2 reads.
#include <mutex>

#include "vrs_internal.h"

namespace {

static __device__ __align__(256) uint8_t scratch[VRS_DETECT_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};   // device address of `scratch` per device (null: not looked up)

}  // namespace

namespace vrs {

// Called by vrs_ctx_create with ctx->device current.  A failed lookup leaves
// ctx->scratch null with the reason in ctx->scratch_err: the other entry
// points keep working and the allocation-free one reports it.
void scratch_attach(vrs_ctx* ctx) {
  ctx->scratch = nullptr;
  ctx->scratch_err.clear();
  if (ctx->device < 0 || ctx->device >= kMaxDevices) {
    ctx->scratch_err = "device index beyond the scratch table";
    return;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ptr[ctx->device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      ctx->scratch_err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
      return;
    }
    g_ptr[ctx->device] = p;
  }
  ctx->scratch = g_ptr[ctx->device];
}

}  // namespace vrs

using namespace vrs;

extern "C" int vrs_detect_postprocess_noalloc(vrs_ctx* ctx, const vrs_detect_desc* d, const float* boxes,
                                              const float* scores, int32_t* count, float* score, int32_t* cls,
                                              int32_t* anchor, float* xywh, void* stream) {
  if (!ctx) return fail(VRS_EINVAL, "vrs_detect_postprocess_noalloc: null ctx");
  int rc = det_check(d);   // the checks and error codes of vrs_detect_postprocess
  if (rc) return rc;
  const size_t need = (size_t)d->n * (size_t)det_anchors(d) * 28;
  if (need > (size_t)VRS_DETECT_SCRATCH_BYTES)
    return fail(VRS_EUNSUPPORTED,
                "vrs_detect_postprocess_noalloc: %d images x %lld anchors need %zu workspace bytes; the fixed "
                "array holds %d (use vrs_detect_postprocess with a caller workspace)",
                d->n, (long long)(need / 28 / (size_t)d->n), need, VRS_DETECT_SCRATCH_BYTES);
  if (!ctx->scratch)
    return fail(VRS_EHIP, "vrs_detect_postprocess_noalloc: no scratch address on device %d (%s)", ctx->device,
                ctx->scratch_err.c_str());
  return vrs_detect_postprocess(ctx, d, boxes, scores, ctx->scratch, (size_t)VRS_DETECT_SCRATCH_BYTES, count,
                                score, cls, anchor, xywh, stream);
}

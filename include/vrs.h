/*
 * vrs.h -- C ABI of the MI355X-native (gfx950) YOLO26 inference hot path.
 *
 * Drop-in boundary for spinorml/vision-rs.  The reference builds YOLO26 as a
 * symbolic graph from layer closures (src/models/yolo/yolo26/mod.rs:207-219
 * and the files of src/models/yolo/yolo26/blocks), compiles it with teeny-cuda/TritonLowering and replays a CUDA
 * graph (examples/yolo26.rs:3015-3141); its custom kernels plug in through
 * teeny-core's CustomOp/RuntimeOp traits (kernels/attention/psa.rs:744-1066,
 * kernels/detect_decode.rs:96-217).  This library replaces that L2/L1 stack:
 * each entry point below names the reference interface it stands in for.
 *
 * Conventions
 *  - Plain C: pointers, sizes and small POD descriptors; no torch/HIP types.
 *    `stream` is a hipStream_t passed as void* (NULL = default stream).
 *  - Device buffers are caller-owned, except inside a vrs_model, which owns
 *    its activations and packed parameters (as the reference's LoadedModel
 *    owns device buffers).
 *  - Every call returns VRS_OK (0) or a negative VRS_E* code and never aborts;
 *    vrs_last_error() returns a thread-local message for the last failure.
 *    All argument checks happen before any HIP call.
 *  - A vrs_ctx is not re-entrant: use one per host thread (the reference runs
 *    one stream per captured graph and serialises GPU tests).
 *  - Activations are NHWC; a vrs_nhwc is a channel slice of an NHWC buffer, so
 *    channel concat/chunk (blocks/concat.rs, blocks/c3k2.rs:26-41) cost nothing.
 */
#ifndef VRS_H
#define VRS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------- */
#define VRS_OK 0
#define VRS_EINVAL (-1)       /* null pointer or invalid argument */
#define VRS_EBADSHAPE (-2)    /* shapes/strides/alignment do not fit the kernel */
#define VRS_EUNSUPPORTED (-3) /* valid request this build does not implement */
#define VRS_ENOMODULE (-4)    /* a code object or kernel symbol is missing */
#define VRS_EHIP (-5)         /* the HIP runtime reported an error */
#define VRS_ENOTFOUND (-6)    /* unknown parameter name */
#define VRS_ESTATE (-7)       /* call not valid in the object's current state */

/* ---- enums -------------------------------------------------------------- */
#define VRS_F32 0
#define VRS_BF16 1
/* Dense convs with e4m3 weights (per-output-channel scale absmax/448) and
 * e4m3-quantised activations (a per-tensor power-of-two scale) on the fp8
 * MFMA; activations in memory are bfloat16, or e4m3 where every reader of a
 * tensor is an fp8 conv (vrs_conv_desc x_e4m3 / y_e4m3 / res_e4m3; inside a
 * model, planned per buffer).  No reference function: BASELINE config 5's
 * second run. */
#define VRS_FP8 2

#define VRS_ACT_NONE 0
#define VRS_ACT_SILU 1

typedef struct vrs_ctx vrs_ctx;
typedef struct vrs_model vrs_model;

/* ---- context ------------------------------------------------------------ */
/* Last error message of the calling thread ("" if none). */
const char* vrs_last_error(void);
const char* vrs_version(void);

/* Select `device`, hipModuleLoad every code object under `hsaco_dir` and
 * resolve the kernels.  Replaces CudaGraphCompiler::compile_model + load
 * (examples/yolo26.rs:3025-3040): kernels are compiled ahead of time. */
int vrs_ctx_create(int device, const char* hsaco_dir, vrs_ctx** out);
int vrs_ctx_destroy(vrs_ctx* ctx);

/* ---- tensors ------------------------------------------------------------ */
typedef struct {
  void* data;       /* device address of the buffer (pixel 0, channel 0) */
  int32_t n, h, w;  /* logical batch, height, width */
  int32_t c;        /* channels of this view */
  int32_t pitch;    /* channels per pixel of the underlying buffer */
  int32_t c_off;    /* first channel of the view inside the buffer */
} vrs_nhwc;

/* ---- single ops ----------------------------------------------------------- */
/* Dense-conv workgroup tiles (output channels x output pixels).  VRS_TILE_AUTO
 * picks by shape; OR VRS_TILE_K32 to force the 32-deep reduction step (the
 * 64-deep one is used when Cin % 64 == 0 and the tile has it). */
#define VRS_TILE_AUTO 0
#define VRS_TILE_128x128 1
#define VRS_TILE_256x128 2
#define VRS_TILE_128x256 3
#define VRS_TILE_64x256 4
#define VRS_TILE_32x256 5
#define VRS_TILE_256x256 6   /* 512 threads; bf16, Cin % 64 == 0 */
/* Halo-tiled 3x3 stride-1 kernel (bf16, Cin % 32 == 0, width >= 8): 64 (or,
 * for Cout <= 32, 32) output channels x 256 output pixels of one image strip
 * per workgroup, the strip rows plus a one-pixel halo staged in LDS once per
 * 16 input channels and read for all nine taps. */
#define VRS_TILE_H3 7
/* Weight-stationary 1x1 kernels (bf16, k = 1, stride 1, Cin a multiple of 64
 * up to 192 (_256) or 256 (_128), or Cin 384 (_128), no residual, output
 * channel offset/pitch/count multiples of 8, no fused upsample): a persistent
 * workgroup keeps a 256- or 128-channel slice of the weights in LDS and
 * streams 64-pixel tiles of whole input pixel rows through it (Cin 384: as
 * two 192-channel halves).  In model plans, _128 also serves the
 * Detect head's channel-major float32 output convs with Cin 64 or 256.
 * VRS_FP8: _128 only, e4m3 weights in LDS and 128-pixel tiles, Cin 128, 192,
 * 256, 384, 512 or 768, e4m3 or bf16 input and output, no residual; results
 * bit-identical to the tiled fp8 kernels. */
#define VRS_TILE_W1_256 8
#define VRS_TILE_W1_128 9
/* 64x64 tile (bf16, Cin % 32 == 0; 4 waves of 32x32): four times the
 * workgroups of 128x128 for the small maps whose larger tiles leave CUs idle */
#define VRS_TILE_64x64 10
/* Model plans only: the conv right after a 64-channel stem (3x3/s2, 64 -> 128,
 * BN + SiLU, bf16; it must be the stem output's only reader) runs fused with
 * the stem as one vrs_conv_stem_pair launch. */
#define VRS_TILE_STEM_PAIR 11
/* Model plans only: the second conv of a bottleneck (3x3 -> 3x3, bf16 model,
 * the shapes vrs_conv_bottleneck_pair is built for; the first conv's output
 * read by it alone) runs fused with the conv before it as one
 * vrs_conv_bottleneck_pair launch; the first conv then has no launch and no
 * output of its own. */
#define VRS_TILE_BPAIR 12
/* Model plans only: a flat float32 output conv (conv_plain, 1x1, the Detect
 * class logits) whose input is the output of the 1x1 BN + SiLU conv before
 * it (bf16 model, the shapes vrs_conv_pointwise_pair is built for, that
 * output read by it alone) runs fused with that conv as one
 * vrs_conv_pointwise_pair launch; the first conv then has no launch and no
 * output of its own. */
#define VRS_TILE_PWPAIR 13
#define VRS_TILE_K32 0x100
/* OR VRS_TILE_PERSIST: persistent grid (resident workgroups loop over the
 * tiles with one continuous load stream, so a tile's epilogue overlaps the
 * next tile's first loads); bf16, 128x128, 64x256 or 256x256 (64-deep steps),
 * Cin % step == 0, an even number of K steps, no residual, output channel
 * offset/pitch/count multiples of 8. */
#define VRS_TILE_PERSIST 0x200
/* OR VRS_TILE_K128 (VRS_FP8 only): 128-deep K steps, two fp8 MFMA k slices per
 * LDS stage and barrier; tile 256x256 with an e4m3 input (x_e4m3), Cin % 128
 * == 0, no fused upsample. */
#define VRS_TILE_K128 0x400

typedef struct {
  int32_t k;        /* square kernel size; padding = k/2 (blocks/conv.rs:36) */
  int32_t stride;
  int32_t groups;   /* 1 = dense (implicit GEMM on MFMA); == channels = depthwise;
                       else grouped (Cin and Cout divisible by groups) */
  int32_t act;      /* VRS_ACT_NONE or VRS_ACT_SILU */
  int32_t dtype;    /* VRS_BF16 or VRS_F32: element type of x, y, res;
                       VRS_FP8 (dense, Cin % 64 == 0): bf16 x/y/res, e4m3 weights */
  int32_t tile;     /* dense only: VRS_TILE_* (0 = automatic) */
  float in_scale;   /* VRS_FP8: activation quantisation step, a power of two:
                       x8 = rne(clamp(x, +-448*in_scale) / in_scale) */
  /* VRS_FP8 with activations stored as e4m3 (1 byte per channel, views
   * 16-channel aligned; tiles 128x128, 256x128, 128x256, 64x256, 256x256):
   * x_e4m3 -- x (and a fused-upsample source) already holds e4m3 on step
   * in_scale; y_e4m3 -- y is written as rne(clamp(y, +-448*out_step) /
   * out_step) of its bfloat16 value; res_e4m3 -- res holds e4m3 on step
   * res_step.  Steps are powers of two; 0 / 0.f when unused. */
  int32_t x_e4m3, y_e4m3, res_e4m3;
  float out_step, res_step;
} vrs_conv_desc;

/* Conv2d + folded BN (+SiLU) (+residual).  Replaces teeny-kernels
 * Conv2dForward / conv2d_bn_silu* + BatchNormForwardInference + SiluForward +
 * ElemwiseAddForward as the layers blocks/conv.rs:31-99 and
 * blocks/bottleneck.rs:24-63 record them.
 *   y = act(scale[co] * conv(x, w)[co] + shift[co]) + res
 * w: packed by vrs_pack_conv_weight in `dtype` elements (dense
 *    [Cout][k][k][Cin]; depthwise tap-major [k*k][C]; grouped
 *    [Cout][k][k][Cin/groups]).
 * Dense requires x->c % 8 == 0; depthwise is 3x3 with stride 1 or 2;
 * res may be NULL (not taken by depthwise).  Grouped (1 < groups, not
 * depthwise; conv_bn's Conv2d::new_grouped, blocks/conv.rs:51-69): groups
 * with Cin/groups % 8 == 0, Cout/groups % 4 == 0 and Cin*Cout/groups^2 >=
 * 1024 run as one implicit-GEMM launch per group on channel slices (VRS_FP8
 * also needs Cin/groups % 64 == 0), others on a direct kernel (bf16/f32, any
 * channel offsets). */
int vrs_conv2d(vrs_ctx* ctx, const vrs_conv_desc* d, const vrs_nhwc* x, const void* w,
               const float* scale, const float* shift, const vrs_nhwc* res, const vrs_nhwc* y,
               void* stream);

/* Host-side weight repack from the reference's OIHW float32 layout
 * (nn::Conv2d weight) into the device layout vrs_conv2d reads:
 *   dense:  [Cout][k][k][cin_pad] in `dtype` (cin_pad >= Cin, zero filled)
 *   depthwise (groups == Cout, cin_per_group == 1): tap-major [k*k][Cout]
 *   grouped (other groups > 1): [Cout][k][k][cin_per_group], cin_pad ==
 *     cin_per_group, Cout % groups == 0.
 * Returns the byte count needed when out == NULL. */
int64_t vrs_pack_conv_weight(const float* w_oihw, int32_t cout, int32_t cin_per_group, int32_t k,
                             int32_t groups, int32_t cin_pad, int32_t dtype, void* out);

/* fp8 weight pack (no reference function): per output channel c,
 * s[c] = max|w[c]| / 448 (1 when all zero) and q = rne_e4m3(w / s[c]) into
 * the dense layout [Cout][k][k][cin_pad] of bytes.  vrs_conv2d with VRS_FP8
 * expects scale[c] to include s[c] * in_scale (times the BN scale).
 * Returns the byte count needed when out == NULL. */
int64_t vrs_pack_conv_weight_fp8(const float* w_oihw, int32_t cout, int32_t cin, int32_t k, int32_t cin_pad,
                                 uint8_t* out, float* out_scale);

/* BN fold, examples/yolo26.rs:3437-3495: scale = gamma/sqrt(var+eps),
 * shift = beta - scale*mean (host arithmetic, done once at load time).
 * conv_plain layers have no BN: pass scale = 1, shift = bias to vrs_conv2d. */
int vrs_bn_fold(const float* gamma, const float* beta, const float* mean, const float* var,
                float eps, int32_t c, float* scale, float* shift);

/* The stem layer model.0 = conv(3, c, 3, 2) (yolo26/mod.rs:126-195, blocks/
 * conv.rs:31-46) straight from the NCHW float32 image, replacing
 * vrs_pack_input + vrs_conv2d for the first layer: y (NHWC view of Cout <= 128
 * channels, dtype) = act(scale * conv3x3s2(x) + shift).  Weights from
 * vrs_pack_stem_weight: [ceil32(Cout)][32] with k = c*9 + ky*3 + kx (27 used). */
int64_t vrs_pack_stem_weight(const float* w_oihw, int32_t cout, int32_t dtype, void* out);
int vrs_conv_stem(vrs_ctx* ctx, const vrs_conv_desc* d, const float* x_nchw, int32_t n, int32_t c, int32_t h,
                  int32_t w, const void* w_packed, const float* scale, const float* shift, const vrs_nhwc* y,
                  void* stream);

/* The stem pair model.0 + model.1 (yolo26/mod.rs:126-195: conv(3, 64, 3, 2)
 * then conv(64, 128, 3, 2), each blocks/conv.rs:31-46) in one kernel, for
 * the m and l widths in bf16 with SiLU on both: replaces vrs_conv_stem +
 * vrs_conv2d for these two layers, and the 64-channel stem map (the
 * network's largest activation) is never written to memory.
 *   y = silu(scale1 * conv3x3s2(s, w1) + shift1),
 *   s = bf16(silu(scale0 * conv3x3s2(x, w0) + shift0))
 * with the same results as the two calls.  w0 from vrs_pack_stem_weight
 * (Cout 64), w1 from vrs_pack_conv_weight ([128][3][3][64]); y: 128 channels,
 * image width a multiple of 4. */
int vrs_conv_stem_pair(vrs_ctx* ctx, const vrs_conv_desc* d0, const vrs_conv_desc* d1, const float* x_nchw,
                       int32_t n, int32_t c, int32_t h, int32_t w, const void* w0_packed, const float* scale0,
                       const float* shift0, const void* w1_packed, const float* scale1, const float* shift1,
                       const vrs_nhwc* y, void* stream);

/* A bottleneck's two convs in one kernel: bottleneck(c, c, shortcut, e)
 * (blocks/bottleneck.rs:37-63) records conv(c, c_h, 3, 1) then conv(c_h, c,
 * 3, 1) (blocks/conv.rs:31-46) and, with the shortcut, adds the block input:
 *   y = bf16(silu(scale2 * conv3x3(m, w2) + shift2) + res),
 *   m = bf16(silu(scale1 * conv3x3(x, w1) + shift1))
 * with the same results as two vrs_conv2d calls on the halo 3x3 tile
 * (VRS_TILE_H3); the middle map m never goes to memory.  bf16, SiLU on both,
 * 3x3 stride 1, built for c = 64, c_hidden = 32 (YOLO26m's P2 C3k2 block);
 * w1 [c_hidden][3][3][c] and w2 [c][3][3][c_hidden] from
 * vrs_pack_conv_weight; res optional (NULL: no shortcut), shaped as y; x, y,
 * res: 8-channel aligned views under 2 GiB.  Other shapes:
 * VRS_EUNSUPPORTED. */
int vrs_conv_bottleneck_pair(vrs_ctx* ctx, const vrs_conv_desc* d1, const vrs_conv_desc* d2, const vrs_nhwc* x,
                             const void* w1_packed, const float* scale1, const float* shift1, int32_t c_hidden,
                             const void* w2_packed, const float* scale2, const float* shift2, const vrs_nhwc* res,
                             const vrs_nhwc* y, void* stream);

/* The last two convs of a Detect class branch in one kernel: the branch
 * (blocks/detect.rs:117-155) records conv(c, c3, 1, 1) (blocks/conv.rs:31-46)
 * then conv_plain(c3, nc, 1) (blocks/conv.rs:90-99) writing the class logits:
 *   y[b*sb + p*sp + co*sc] = scale2[co] * (w2 . m)[co] + shift2[co],
 *   m = bf16(silu(scale1 * (w1 . x) + shift1))
 * with the same results as the two convs launched separately (the second
 * on a flat float32 output, as vrs_model_forward runs the Detect head); the
 * map m never goes to memory.  bf16, 1x1 stride 1, SiLU on the first conv
 * and none on the second, built for x->c = c_mid = 256 and 1 <= nc <= 96;
 * w1 [c_mid][256], w2 [nc][c_mid] from vrs_pack_conv_weight; x an 8-channel
 * aligned view and the output under 2 GiB.  Other shapes: VRS_EUNSUPPORTED.
 * No counterpart in the reference's API (it records the two convs). */
int vrs_conv_pointwise_pair(vrs_ctx* ctx, const vrs_conv_desc* d1, const vrs_conv_desc* d2, const vrs_nhwc* x,
                            const void* w1_packed, const float* scale1, const float* shift1, int32_t c_mid,
                            const void* w2_packed, const float* scale2, const float* shift2, int32_t nc, float* y,
                            int64_t sb, int64_t sp, int64_t sc, void* stream);

/* NCHW float32 -> NHWC dtype, zero-padding channels C..y->c-1 (C <= y->c < C+8). */
int vrs_pack_input(vrs_ctx* ctx, const float* x_nchw, int32_t n, int32_t c, int32_t h, int32_t w,
                   const vrs_nhwc* y, int32_t dtype, void* stream);
/* NHWC dtype view -> NCHW float32 [n][x->c][h][w]. */
int vrs_unpack_output(vrs_ctx* ctx, const vrs_nhwc* x, int32_t dtype, float* y_nchw, void* stream);

/* SPPF pooling cascade (blocks/sppf.rs:43-61 + teeny-core MaxPool2d(5,1,2)):
 * `buf` is a view of 4*c channels whose first c hold y; writes
 * p1 = max5(y), p2 = max5(p1), p3 = max5(p2) into the next 3*c channels. */
int vrs_sppf_pool(vrs_ctx* ctx, const vrs_nhwc* buf, int32_t dtype, void* stream);

/* Nearest 2x upsample into a (concat) view (blocks/upsample.rs:23-35). */
int vrs_upsample2x(vrs_ctx* ctx, const vrs_nhwc* x, const vrs_nhwc* y, int32_t dtype, void* stream);

/* PSA attention core + fused PE (blocks/c2psa.rs:61-116).  Replaces the
 * PsaPackQkvOp, FlashAttn2PsaOp (lo and hi), PsaMergeAttnOp, PsaExtractVOp
 * custom ops (kernels/attention/psa.rs:744-1066), the PE conv_bn and the add:
 *   out = softmax(q k^T * key_dim^-0.5) v + pe_scale * dw3x3(v) + pe_shift
 * qkv: view of heads*128 channels (per head q 32 | k 32 | v 64);
 * out: view of heads*64 channels; pe_w: the PE conv weight packed as a
 * depthwise weight (tap-major [9][heads*64], dtype elements). */
typedef struct {
  int32_t heads;
  int32_t key_dim;   /* must be 32 (blocks/c2psa.rs:159) */
  int32_t head_dim;  /* must be 64 (c / num_heads with num_heads = c/64) */
  int32_t dtype;
} vrs_psa_desc;
int vrs_psa_attention(vrs_ctx* ctx, const vrs_psa_desc* d, const vrs_nhwc* qkv, const void* pe_w,
                      const float* pe_scale, const float* pe_shift, const vrs_nhwc* out, void* stream);

/* Detect post-process on the raw head outputs (DetectOutput,
 * blocks/detect.rs:157-172), doing on the GPU what the reference does on the
 * host (examples/yolo26.rs:1488-1529): decode, sigmoid, argmax (last max
 * wins), threshold, stable descending sort, keep max_det (<= 1024).
 * boxes [n][4*A] and scores [n][nc*A] float32 in per-scale blocks.
 * Outputs per image: count[n]; score/cls/anchor [n][max_det]; xywh [n][max_det][4];
 * rows past count are score 0, cls -1, anchor -1. */
typedef struct {
  int32_t n, nc, img_h, img_w;
  int32_t nscales;        /* <= 4 */
  int32_t strides[4];     /* e.g. 8, 16, 32 (loss/anchor.rs:33-35) */
  float thr;              /* 0.25 viewer, 0.001 eval (examples/yolo26.rs:1507) */
  int32_t max_det;
} vrs_detect_desc;
size_t vrs_detect_workspace_size(const vrs_detect_desc* d);
int vrs_detect_postprocess(vrs_ctx* ctx, const vrs_detect_desc* d, const float* boxes,
                           const float* scores, void* workspace, size_t workspace_bytes,
                           int32_t* count, float* score, int32_t* cls, int32_t* anchor, float* xywh,
                           void* stream);

/* Allocation-free vrs_detect_postprocess.  No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, checks and results as vrs_detect_postprocess, with the workspace
 * in a fixed device array of the library (VRS_DETECT_SCRATCH_BYTES per GPU,
 * held until the process ends) instead of a caller buffer; requires
 * n * anchors * 28 <= VRS_DETECT_SCRATCH_BYTES (64 images at 640x640 fit),
 * else VRS_EUNSUPPORTED.  It allocates nothing.  Every call on one GPU shares
 * that array: calls that overlap in time on one GPU (other streams, threads
 * or contexts) race; serialise them. */
#define VRS_DETECT_SCRATCH_BYTES (16 << 20)
int vrs_detect_postprocess_noalloc(vrs_ctx* ctx, const vrs_detect_desc* d, const float* boxes,
                                   const float* scores, int32_t* count, float* score, int32_t* cls,
                                   int32_t* anchor, float* xywh, void* stream);

/* Un-letterbox (examples/yolo26.rs:1531-1547): the post-processed xywh in
 * letterbox pixels ([n][max_det][4], vrs_detect_postprocess) -> [cx, cy, w, h]
 * normalised to each original image, i.e. Detection::bbox
 * (src/detect/mod.rs:52-60).  orig_wh [n][2] int32 (device): width and
 * height before the letterbox to img_size.  Slots past count[b] get zeros. */
int vrs_detect_unletterbox(vrs_ctx* ctx, int32_t n, int32_t max_det, int32_t img_size,
                           const int32_t* orig_wh, const int32_t* count, const float* xywh,
                           float* out, void* stream);

/* Letterbox preprocessing, preprocess_image_raw (examples/yolo26.rs:1229-1253):
 * n RGB8 images in device memory (image i: wh[2i] x wh[2i+1] pixels, rows of
 * 3*w bytes with no padding, starting at byte offsets[i] of rgb; offsets and
 * wh are HOST arrays, every image must lie inside rgb_bytes) -> the model input
 * [n][3][img_size][img_size] float32 (device).  scale = img_size / max(w, h)
 * in f64, new = round(dim * scale); the image crate's Triangle resize (image
 * 0.25.10 imageops::resize: vertical then horizontal pass, float32, rounded
 * half away from zero to u8); centred with integer padding (img_size - new)/2
 * on a 114/255 canvas; values u8 / 255.  Images shrunk by more than 62x per
 * axis are rejected (VRS_EUNSUPPORTED). */
int vrs_letterbox(vrs_ctx* ctx, int32_t n, int32_t img_size, const uint8_t* rgb, int64_t rgb_bytes,
                  const int64_t* offsets, const int32_t* wh, float* out, void* stream);

/* DetectDecodeOp / detect_decode_forward (kernels/detect_decode.rs:36-217):
 * grid-unit anchors, [n][4][A] in and out. */
int vrs_detect_decode_grid(vrs_ctx* ctx, const float* boxes, const float* anchor_x,
                           const float* anchor_y, const float* strides, int32_t n, int32_t a,
                           float* out, void* stream);

/* Multi-scale deformable attention (RF-DETR decoder; no reference function).
 * value [n][S][heads][32] f32, ref [n][q][2], off [n][q][heads][L][P][2],
 * attw [n][q][heads][L][P] (softmaxed), out [n][q][heads*32]. */
typedef struct {
  int32_t n, q, heads, head_dim; /* head_dim must be 32 */
  int32_t levels, points;        /* levels <= 8 */
  int32_t level_h[8], level_w[8];
} vrs_msda_desc;
int vrs_msda(vrs_ctx* ctx, const vrs_msda_desc* d, const float* value, const float* ref,
             const float* off, const float* attw, float* out, void* stream);

/* ---- models (layer closures + graph runtime) ------------------------------ */
#define VRS_BLOCK_CONV 1        /* conv / conv_bn / dwconv / conv_plain (blocks/conv.rs) */
#define VRS_BLOCK_C3K2 2        /* c3k2 (blocks/c3k2.rs:94-127) */
#define VRS_BLOCK_C3K2_PSA 3    /* c3k2_psa (blocks/c3k2.rs:134-164) */
#define VRS_BLOCK_C2PSA 4       /* c2psa (blocks/c2psa.rs:150-179) */
#define VRS_BLOCK_SPPF 5        /* sppf (blocks/sppf.rs:43-61) */
#define VRS_BLOCK_PSA_ATTN 6    /* psa_attention (blocks/c2psa.rs:61-116) */
#define VRS_BLOCK_DETECT_BOX 7  /* one Detect box branch cv2[i] (blocks/detect.rs:117-131) */
#define VRS_BLOCK_YOLO26 8      /* yolo26() (yolo26/mod.rs:207-219) */
/* detect::<D>(nc, &ch, head) (blocks/detect.rs:108-172): the whole Detect head
 * on three feature maps with ch[0], ch[1], ch[2] channels at h x w, h/2 x w/2
 * and h/4 x w/4 (the strides 8/16/32 maps of a YOLO26 neck; h, w multiples of
 * 4; c_in == ch[0]).  The model input holds the three NCHW float32 tensors back
 * to back ([batch][ch[0]][h][w], then [batch][ch[1]][h/2][w/2], then
 * [batch][ch[2]][h/4][w/4]); the outputs are DetectOutput's boxes
 * [batch][4A] and scores [batch][nc*A] (channel_cat_flat, blocks/detect.rs:
 * 62-80), A = h*w + h*w/4 + h*w/16.  one2one selects the head's weight names
 * (DetectHead::OneToOne "one2one_cv2/3", else OneToMany "cv2/3"). */
#define VRS_BLOCK_DETECT 9

#define VRS_CONV_BN_SILU 0      /* conv() */
#define VRS_CONV_BN 1           /* conv_bn() */
#define VRS_CONV_PLAIN 2        /* conv_plain(): bias, no BN, no act */

typedef struct {
  int32_t kind;
  int32_t c_in, c_out;
  int32_t k, s, g;          /* VRS_BLOCK_CONV; g: groups (1 dense, c_in == c_out
                               depthwise, else grouped; conv_plain is dense) */
  int32_t conv_kind;        /* VRS_CONV_* for VRS_BLOCK_CONV */
  int32_t n;                /* repeats (c3k2, c2psa, c3k2_psa) */
  int32_t c3k, shortcut;    /* c3k2 flags; sppf shortcut */
  float e;                  /* expansion (c3k2, c2psa, c3k2_psa) */
  int32_t heads;            /* psa_attention */
  int32_t nc;               /* yolo26: classes */
  int32_t variant;          /* yolo26: 'n','s','m','l','x' */
  int32_t one2one;          /* yolo26, detect: 1 = one2one_cv2/cv3 head (DetectHead::OneToOne),
                               0 = cv2/cv3 (DetectHead::OneToMany) */
  int32_t ch[3];            /* detect: channels of the three feature maps */
} vrs_block_desc;

/* Record the block's layers for a fixed batch and input size, mirroring the
 * reference closures; parameter names are the reference's name_scope paths
 * (e.g. "model.6.m.0.m.1.cv2.conv.weight").  bn_eps is 1e-3 for the model
 * (blocks/conv.rs:39); the reference's PyTorch fixtures use 1e-5.
 * ctx may be NULL for a record-only model (parameter/output introspection
 * without a GPU); finalize/forward then fail with VRS_ESTATE. */
int vrs_model_create(vrs_ctx* ctx, const vrs_block_desc* d, int32_t batch, int32_t h, int32_t w,
                     int32_t dtype, float bn_eps, vrs_model** out);
/* Per-layer tile autotuning at finalize (replaces TritonLowering's
 * shape-adaptive tile choice, examples/yolo26.rs:3027).  mode 1 (default):
 * every dense conv is timed with each applicable VRS_TILE_* on the model's own
 * buffers and the fastest is kept; in a VRS_FP8 model each eligible conv also
 * keeps bf16 when its best bf16 tile is faster.  mode 2 (VRS_FP8 models):
 * only fp8 tiles are timed and every eligible conv runs on fp8, except the
 * conv after a 64-channel stem when the stem pair (VRS_TILE_STEM_PAIR, a bf16
 * kernel that never writes the stem's map) beats the stem plus that conv's
 * best fp8 tile.  mode 0: the shape heuristic of VRS_TILE_AUTO. */
int vrs_model_set_autotune(vrs_model* m, int32_t mode);
/* Tile plan: one entry per conv (build order, vrs_model_num_convs): a
 * VRS_TILE_* code, OR VRS_PLAN_FP8 for a conv that runs on e4m3 (VRS_FP8
 * models); 0 for convs that take no tile (depthwise, stem, flat outputs) or
 * the heuristic.  vrs_model_get_plan (after finalize) returns the plan in use
 * (with plan == NULL: the entry count); vrs_model_set_plan (before finalize;
 * n = 0 clears it) makes finalize apply that plan instead of autotuning, each
 * entry checked against the kernels built for its conv.  A saved plan makes
 * every later run (benchmarks, profiler passes) use the same kernels.
 * No counterpart in the reference. */
#define VRS_PLAN_FP8 0x10000
int vrs_model_set_plan(vrs_model* m, const int32_t* plan, int32_t n);
int vrs_model_get_plan(const vrs_model* m, int32_t* plan, int32_t n);
int vrs_model_num_params(const vrs_model* m);
/* name is owned by the model; dims[0..*ndim) (ndim <= 4). */
int vrs_model_param_info(const vrs_model* m, int32_t i, const char** name, int32_t* dims, int32_t* ndim);
/* LoadedModel::load_param_f32 analogue: float32 host data, reference layout. */
int vrs_model_load_param(vrs_model* m, const char* name, const float* data, int64_t numel);
/* load_weights_from_safetensors (examples/yolo26.rs:3403-3550): every model
 * parameter is looked up by name in a local .safetensors file (raw BN
 * tensors; the fold happens at finalize, as vrs_model_load_param); "X.weight"
 * and "X.conv.weight" stand in for each other as in the reference's
 * fallback.  F32, F16, BF16 and F64 tensors are accepted (converted to f32);
 * an element-count mismatch is an error.  Parameters absent from the file
 * are counted in *n_missing, not an error (the reference warns and goes on);
 * they must still be loaded before vrs_model_finalize. */
int vrs_model_load_safetensors(vrs_model* m, const char* path, int32_t* n_loaded, int32_t* n_missing);
/* Fold BN, repack/upload weights and allocate activations.  All params must be loaded. */
int vrs_model_finalize(vrs_model* m);
int vrs_model_num_outputs(const vrs_model* m);
/* Output i: float32 element count and (up to 4) dims. */
int vrs_model_output_info(const vrs_model* m, int32_t i, int64_t* numel, int32_t* dims, int32_t* ndim);
/* Input: float32 NCHW [batch][c_in][h][w] device buffer (VRS_BLOCK_DETECT:
 * its three feature maps back to back).  Outputs: caller buffers of
 * output_info sizes (yolo26 and detect: boxes [batch][4A], scores
 * [batch][nc*A], the reference's DetectOutput; other blocks: NCHW float32).
 * 16-byte aligned outputs let the Detect output convs use the
 * weight-stationary kernel a tile plan may name; on other addresses they run
 * on the tiled kernels (same results). */
int vrs_model_forward(vrs_model* m, const float* x, float* const* outputs, void* stream);
/* capture_graph analogue (examples/yolo26.rs:3110): capture one forward with
 * these buffers into a hipGraph; vrs_model_replay launches it (run_inplace). */
int vrs_model_capture(vrs_model* m, const float* x, float* const* outputs, void* stream);
int vrs_model_replay(vrs_model* m, void* stream);
/* Capture concurrency (no counterpart in the reference, whose graphs run on
 * one stream): with streams > 1 (1..8, default 3) vrs_model_capture puts the
 * Detect head's six independent chains (box and class branch of each scale)
 * beside the trunk: a chain launch continues the stream whose latest launch
 * it depends on, else takes the least recently used of the caller's stream
 * and the model's streams - 1 side streams (default priority); every other
 * launch stays on the caller's stream.  Each launch waits only for earlier
 * launches that touch overlapping buffer channels.  All streams are captured
 * into the one graph (cross-stream waits as graph edges), whose parallel
 * branches the runtime replays on parallel hardware queues; the caller's
 * stream continues after all of them.  1 = one serial chain.  Models without
 * a Detect head capture one chain whatever the setting. */
int vrs_model_set_streams(vrs_model* m, int32_t streams);
/* Streams the last vrs_model_capture used (1 = a serial graph; 0 before a
 * capture). */
int vrs_model_num_capture_streams(const vrs_model* m);
/* Number of kernel launches in one forward and their "layer:kernel" names
 * (valid after the first vrs_model_forward / vrs_model_capture). */
int vrs_model_num_launches(const vrs_model* m);
const char* vrs_model_launch_name(const vrs_model* m, int32_t i);
/* Algorithmic work of launch i: flops (2*M*N*K for convs; QK^T + PV + PE for
 * attention) and compulsory bytes (inputs + weights + outputs, once each). */
int vrs_model_launch_work(const vrs_model* m, int32_t i, double* flops, double* bytes);
/* Run launches [first, first+count) of the prepared forward on `stream`
 * (per-kernel timing with events between launches). */
int vrs_model_run_launches(vrs_model* m, int32_t first, int32_t count, void* stream);
/* VRS_FP8 models: set the activation steps from one bfloat16 forward of `x`
 * (same layout as vrs_model_forward).  Buffers one conv reads together (its
 * input and a fused-upsample source) form a step group; a group's step is the
 * smallest power of two >= max|value| / 448 over every write into its
 * buffers.  An fp8 conv's in_scale is its input's step; buffers stored as
 * e4m3 (every writer and reader an fp8 conv) hold values on that step.
 * Required once before the first fp8 forward/capture; synchronises
 * `stream`. */
int vrs_model_calibrate(vrs_model* m, const float* x, void* stream);
/* Convs in build order: parameter prefix (e.g. "model.3"), whether it runs on
 * fp8 and its activation scale (0 before calibration). */
int vrs_model_num_convs(const vrs_model* m);
int vrs_model_conv_info(const vrs_model* m, int32_t i, const char** prefix, int32_t* fp8, float* in_scale);
/* Where conv i of the prepared forward reads and writes (device views of
 * the model's own buffers), for per-layer inspection such as checking each
 * layer against a CPU restatement on the layer's actual input (the analogue
 * of reading a node's tensor from the reference's LoadedModel).  Valid after
 * vrs_model_finalize; `launch` after the first forward/capture.  Views whose
 * data is NULL are absent: x for the stem (which reads the model input), y
 * for convs that write a model output (out_idx >= 0, float32 element
 * (b, p, co) at output[out_idx] + out_off + b*out_sb + p*out_sp + co*out_sc).
 * A stem pair (VRS_TILE_STEM_PAIR): the stem has no launch (-1) and no y; the
 * conv after it has stem = 2 and no x (its input is the stem of the model
 * input, computed on chip).  A bottleneck pair (VRS_TILE_BPAIR): the first
 * conv has no launch and no y; the second has fused_in = 1 and no x (its
 * input is the first conv's output, computed on chip from the first conv's
 * x). */
typedef struct {
  int32_t launch;          /* index among vrs_model_launch_name's launches of the conv's
                              last launch (its output is complete after it; a
                              256x256 conv whose last round of tiles is at most
                              half full runs two: the full rounds, then the
                              leftover tiles on the 128x128 tile), -1: none */
  int32_t k, stride, groups, act;
  int32_t plain;           /* conv_plain: bias, no BN */
  int32_t stem;            /* 1: reads the NCHW float32 model input; 2: reads it
                              through the stem before it (a stem pair) */
  int32_t fp8;             /* runs on the fp8 MFMA (input quantised with in_scale) */
  float in_scale;
  int32_t dtype;           /* element type of x, y, res, up */
  int32_t cin, cout;       /* unpadded input channels, output channels */
  vrs_nhwc x, y, res, up;  /* up: source of a fused nearest-2x upsample (first up.c input channels) */
  int32_t out_idx;
  int64_t out_off, out_sb, out_sp, out_sc;
  /* VRS_FP8 models: views whose buffer is stored as e4m3 (1 byte per
   * channel, value = e4m3 * step; the others hold dtype elements) */
  int32_t x_e4m3, y_e4m3, res_e4m3, up_e4m3;
  float x_step, y_step, res_step, up_step;
  int32_t fused_in;        /* 1: the input is the conv before it, computed inside this launch */
} vrs_conv_io;
int vrs_model_conv_io(const vrs_model* m, int32_t i, vrs_conv_io* io);
int vrs_model_destroy(vrs_model* m);

#ifdef __cplusplus
}
#endif
#endif /* VRS_H */

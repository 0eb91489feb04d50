/* Kernel argument blocks shared by the host runtime and the gfx950 kernels.
 * Plain C layout: each kernel takes exactly one of these by value, and the host
 * passes it through hipModuleLaunchKernel's kernelParams.
 * Element offsets are in elements of the tensor's dtype. */
#ifndef VRS_KARGS_H
#define VRS_KARGS_H
#include <stdint.h>

#define VRS_ACT_NONE 0
#define VRS_ACT_SILU 1

/* Implicit-GEMM convolution (dense, groups == 1).
 * x: NHWC view; element (b, iy, ix, ci) at x[((b*H + iy)*W + ix)*x_pitch + ci]
 *    (the pointer already includes the view's channel offset).
 * w: packed [Cout][kh][kw][Cin] (K = kh*kw*Cin contiguous per output channel).
 * y: element (b, p, co) at y[b*y_sb + p*y_sp + co*y_sc], p = oy*Wo + ox.
 * res (optional): same addressing with r_* strides, added after the activation.
 * out = act(acc*scale[co] + shift[co]) + res. */
typedef struct {
  const void* x;
  const void* w;
  const float* scale;
  const float* shift;
  const void* res;
  void* y;
  int64_t y_sb, y_sp, y_sc;
  int64_t r_sb, r_sp, r_sc;
  int32_t N, H, W, Cin, x_pitch;
  int32_t Ho, Wo, Cout;
  int32_t kh, kw, stride, pad;
  int32_t K;      /* kh*kw*Cin */
  int32_t M;      /* N*Ho*Wo */
  int32_t act;
  int32_t y_f32;  /* 1: store float32, 0: store the kernel's element type */
  int32_t tiles_m, tiles_n; /* grid decomposition: Cout tiles x pixel tiles */
  int32_t stage;  /* 1: NHWC output staged through LDS for 16-byte stores
                     (element-type output, y_sc == 1, Cout % 8 == 0, 16-byte
                     aligned channel offset and pitch); 2 (bf16 tiles): a
                     channel-major float32 output (y_sp == 1) staged for
                     16-byte stores of 4 pixels of one channel, y_bytes the
                     extent written */
  int32_t x_bytes;  /* readable bytes from x to the end of its buffer (< 2^31) */
  int32_t w_bytes;  /* bytes of the packed weights (< 2^31) */
  /* fp8 kernels: activations are quantised to e4m3 as x / in_scale (a power
   * of two) after clamping |x| to 448 * in_scale, whose bfloat16 bits are
   * clamp_bits (in both halves) */
  float in_scale;
  uint32_t clamp_bits;
  /* persistent kernels: bytes from y to the end of the output view's last
   * pixel (< 2^31) */
  int32_t y_bytes;
  /* fused nearest-2x upsample (1x1 stride-1 convs, 32-deep-step aligned
   * kernels): input channels [0, c_split) are read from x2, an NHWC buffer of
   * H2 x W2 = (H/2) x (W/2) pixels with pitch x2_pitch (pointer at its first
   * channel, x2_bytes readable), at pixel (y/2, x/2); channels [c_split, Cin)
   * from x as usual.  c_split = 0: no fusion. */
  const void* x2;
  int32_t x2_bytes, c_split, H2, W2, x2_pitch;
  /* halo-tiled 3x3 stride-1 kernels: each image is cut into h3_strips
   * vertical strips h3_tw pixels wide (the last one may be partial), and each
   * strip into h3_chunks runs of 256 consecutive output pixels (row-major
   * within the strip); y_bytes and res_bytes bound the raw-buffer stores and
   * residual loads */
  int32_t h3_tw, h3_strips, h3_chunks;
  int32_t res_bytes;
  /* first pixel tile of this launch (tiled kernels: tile_n = n_tile0 +
   * logical / tiles_m); non-zero for the launch that takes the pixel tiles
   * left over by a larger tile's full rounds */
  int32_t n_tile0;
  /* fp8 kernels with e4m3 activations in memory: the output's quantisation
   * step (e4m3-output kernels: y = e4m3(clamp(out, +-448*out_step) /
   * out_step)); a residual stored as e4m3 (res_f8 = 1) is read as
   * e4m3 * res_step */
  float out_step;
  float res_step;
  int32_t res_f8;
} vrs_conv_args;

/* Fused bottleneck pair (bf16): y = act2(s2 * conv3x3(w2, act1(s1 * conv3x3(w1,
 * x) + b1)) + b2) + res, both convs 3x3 stride 1 pad 1 with SiLU, the middle
 * map never leaving the workgroup.  x, y, res: NHWC views of N x H x W pixels
 * (pointers at their first channel, pitches in elements, bytes readable from
 * the pointer < 2^31); w1 [CH][3][3][C], w2 [C][3][3][CH] in bf16.  The grid
 * is N x strips x runs: strips of TW columns, runs of 256 / TW rows. */
typedef struct {
  const void* x;
  const void* w1;
  const float* s1;
  const float* b1;
  const void* w2;
  const float* s2;
  const float* b2;
  const void* res;   /* null: no residual */
  void* y;
  int32_t N, H, W;
  int32_t x_pitch, y_pitch, r_pitch;
  int32_t strips, runs;
  int32_t x_bytes, y_bytes, res_bytes, w1_bytes, w2_bytes;
} vrs_bpair_args;

/* Fused pointwise pair (pwpair.hip): 1x1 C -> CM (+BN, SiLU, bf16) then 1x1
 * CM -> NC (+scale, shift) into a float32 flat output y[b*sb + p*sp + c*sc]. */
typedef struct {
  const void* x;     /* bf16 NHWC view, first channel of pixel 0 */
  const void* w1;    /* [CM][C] bf16 */
  const float* s1;
  const float* b1;
  const void* w2;    /* [NC][CM] bf16 */
  const float* s2;
  const float* b2;
  float* y;
  int64_t y_sb, y_sp, y_sc;
  int32_t M, HW, NC;  /* pixels (N*H*W), pixels per image, output channels */
  int32_t x_pitch, x_bytes, y_bytes;
} vrs_pwpair_args;

/* Depthwise 3x3 conv (groups == C), NHWC, weights tap-major [9][C] in the
 * element type. */
typedef struct {
  const void* x;
  const void* w;
  const float* scale;
  const float* shift;
  void* y;
  int32_t N, H, W, C, x_pitch;
  int32_t Ho, Wo, y_pitch;
  int32_t kh, kw, stride, pad;
  int32_t act;
  /* row-walking stride-1 kernel: raw-buffer extent of x, 64-channel blocks,
   * 8-column patches and row bands per image */
  int32_t x_bytes, cblocks, patches, bands;
} vrs_dw_args;

/* Grouped conv (1 < groups < channels), NHWC, direct form.  x, y, res point
 * at the views' first channels; weights [Cout][kh][kw][cin_g] in the element
 * type; output channel co reads input channels [g*cin_g, (g+1)*cin_g) of
 * group g = co / cout_g.  out = act(acc*scale[co] + shift[co]) + res. */
typedef struct {
  const void* x;
  const void* w;
  const float* scale;
  const float* shift;
  const void* res;
  void* y;
  int64_t total;        /* N*Ho*Wo*Cout output elements */
  int32_t H, W, x_pitch;
  int32_t Ho, Wo, y_pitch, r_pitch;
  int32_t cin_g, cout, cout_g;
  int32_t k, stride, pad, act;
} vrs_gconv_args;

/* SPPF pooling: reads channels [0,c) of a NHWC buffer (pitch) and writes the
 * cascade p1 = max5(y), p2 = max5(p1), p3 = max5(p2) (stride 1, pad 2, -inf
 * padding) into channels [c,2c), [2c,3c), [3c,4c) of the same buffer. */
typedef struct {
  void* buf;
  int32_t N, H, W, c, pitch;
  int32_t cgroups_per_block;
} vrs_pool_args;

/* Nearest 2x upsample from a NHWC view into a NHWC view. */
typedef struct {
  const void* x;
  void* y;
  int32_t N, H, W, C, x_pitch, y_pitch;
} vrs_up_args;

/* NCHW float32 image batch -> NHWC element-type buffer with c_pad channels
 * (channels >= C are zero). */
typedef struct {
  const float* x;
  void* y;
  int32_t N, C, H, W, c_pad;
} vrs_pack_args;

/* PSA attention, key_dim 32, head_dim 64 (blocks/c2psa.rs:61-116).
 * qkv: NHWC [B, N, heads*128] (per head: q 32 | k 32 | v 64).
 * out[b, n, h*64 + d] = softmax(q.k * scale) v + pe_scale*dw3x3(v) + pe_shift. */
typedef struct {
  const void* qkv;
  const void* pe_w;     /* tap-major [9][heads*64], element type */
  const float* pe_scale;
  const float* pe_shift;
  void* out;
  int32_t B, H, W, heads, qkv_pitch, out_pitch;
  float scale_log2e;    /* kd^-0.5 * log2(e) */
  int32_t q_blocks;
  int32_t qkv_bytes;    /* readable bytes from qkv to the end of its buffer (< 2^31) */
} vrs_attn_args;

/* Detect post-process stage 1: per anchor decode + sigmoid/argmax + threshold. */
typedef struct {
  const float* boxes;   /* [B, 4*A] per-scale [4][A_s] blocks */
  const float* scores;  /* [B, nc*A] per-scale [nc][A_s] blocks */
  uint64_t* keys;       /* [B, A] (score_bits << 32 | ~anchor) or 0 */
  int32_t* cls;         /* [B, A] */
  float* xywh;          /* [B, A, 4] */
  int32_t B, nc, A, nscales;
  int32_t a_base[4];    /* anchor offset of each scale */
  int32_t fw[4];        /* grid width of each scale */
  float stride[4];
  float thr;
} vrs_det1_args;

/* Detect post-process stage 2: per image exact top-k (radix select over the
 * unique 64-bit keys) + sort, one workgroup per image. */
typedef struct {
  const uint64_t* keys;
  const int32_t* cls;
  const float* xywh;
  int32_t* count;
  float* out_score;
  int32_t* out_cls;
  int32_t* out_anchor;
  float* out_xywh;
  int32_t B, A, max_det;
} vrs_det2_args;

/* Un-letterbox of post-processed detections (examples/yolo26.rs:1531-1547). */
typedef struct {
  const int32_t* orig_wh;  /* [B][2] original width, height */
  const int32_t* count;    /* [B] */
  const float* xywh;       /* [B][max_det][4] letterbox pixels */
  float* out;              /* [B][max_det][4] normalised to the original image */
  int32_t B, max_det, img_size;
} vrs_unlb_args;

/* Letterbox preprocessing, up to VRS_LB_MAX_IMAGES images per launch (grid.y
 * = image).  Per image: RGB8 rows of w*3 bytes at rgb + off, the resized size
 * (nw, nh), the canvas offset (px, py) and the output slot, all computed on
 * the host. */
#define VRS_LB_MAX_IMAGES 16
#define VRS_LB_MAX_TAPS 128   /* direct kernel: taps per output row/column (ratio <= 62) */
#define VRS_LB_STAGED_RATIO 8 /* staged kernels: images shrunk at most 8x per axis */
typedef struct {
  int64_t off;
  int32_t w, h, nw, nh, px, py, slot, pad_;
} vrs_lb_image;
typedef struct {
  const uint8_t* rgb;
  float* out;           /* [slots][3][S][S] */
  float pad;            /* 114 / 255 in float32 */
  int32_t S, count;
  vrs_lb_image img[VRS_LB_MAX_IMAGES];
} vrs_lb_args;

/* Grid-unit decode on [B,4,A] (kernels/detect_decode.rs:36-86). */
typedef struct {
  const float* boxes;
  const float* ax;
  const float* ay;
  const float* st;
  float* out;
  int32_t B, A;
} vrs_dec_args;

/* Multi-scale deformable attention, Dh = 32.
 * value [B, S, heads, 32]; ref [B, Q, 2]; off [B, Q, heads, L, P, 2];
 * attw [B, Q, heads, L, P]; out [B, Q, heads*32]. */
typedef struct {
  const float* value;
  const float* ref;
  const float* off;
  const float* attw;
  float* out;
  int32_t B, S, Q, heads, L, P;
  int32_t lh[8], lw[8], lstart[8];
} vrs_msda_args;


/* max |x| over an NHWC view (npix pixels x c channels, channel pitch) into
 * *out as float bits (atomic max on the non-negative float's bit pattern) */
typedef struct {
  const void* x;
  unsigned* out;
  int64_t npix;
  int32_t c, pitch;
} vrs_absmax_args;


/* Stem conv straight from the NCHW float32 image: 3x3, stride 2, pad 1,
 * Cin = 3 (K = 27 padded to 32, k = c*9 + ky*3 + kx), Cout <= 128, folded BN
 * + SiLU, NHWC output of the element type. */
typedef struct {
  const float* x;
  const void* w;       /* [cout_pad][32] element type */
  const float* scale;
  const float* shift;
  void* y;             /* view base (pixel 0, first channel of the view) */
  int32_t N, H, W, Ho, Wo, cout, cout_pad, y_pitch, act;
  int32_t segs;        /* 64-pixel segments per output row */
} vrs_stem_args;

/* Stem pair: the stem conv (64 output channels) and the 3x3 stride-2 conv
 * 64 -> 128 that reads it, in one kernel (bf16, SiLU on both).  A step is 2
 * output rows x 32 output columns of one image strip; step q of the batch is
 * (image, strip, row pair) = (q / (strips*sps), q / sps % strips, q % sps). */
typedef struct {
  const float* x;       /* NCHW float32 images */
  const void* w0;       /* stem weights [64][32] bf16 (vrs_pack_stem_weight) */
  const float* scale0;
  const float* shift0;
  const void* w1;       /* [128][3][3][64] bf16 */
  const float* scale1;
  const float* shift1;
  void* y;              /* view base (pixel 0, first channel of the view) */
  int32_t N, H, W;      /* images */
  int32_t H0, W0;       /* stem output */
  int32_t H1, W1;       /* output */
  int32_t y_pitch;
  int32_t strips, sps;  /* 32-column strips per image, row pairs per strip */
  int32_t total;        /* N * strips * sps */
} vrs_stem_pair_args;

#endif

// Bandwidth-bound NHWC kernels for gfx950: depthwise conv, the SPPF pooling
// cascade and nearest 2x upsample.  No MFMA: these move bytes, so each lane
// moves 8 consecutive channels (one 16-byte bf16 group) and consecutive lanes
// walk the channel dimension first for coalesced HBM access.  Also the direct
// grouped conv for group shapes the implicit-GEMM tiles do not take.
#include "common.h"

// ---------------------------------------------------------------------------
// Depthwise 3x3 conv + folded BN (+ SiLU): blocks/conv.rs:75-85 (dwconv) and
// the PE conv_bn with g = c (blocks/c2psa.rs:66).  Weights are tap-major
// [9][C] in the element type, so the 9 taps of 8 channels are 9 vector loads.
// One thread computes 8 channels of DW_ROWS vertically adjacent output pixels;
// every loop is unrolled at compile time (stride is a template parameter) so
// weights and accumulators stay in registers, and the (DW_ROWS-1)*S+3 input
// rows x 3 columns are independent loads in flight together.
namespace {
constexpr int DW_ROWS = 4;

template <typename T, int S>
__device__ __forceinline__ void dw_body(const vrs_dw_args& a) {
  using E = Elt<T>;
  using G = typename E::group;
  constexpr int NR = (DW_ROWS - 1) * S + 3;
  const int cg = a.C >> 3;                       // channel groups of 8
  const int row_tiles = (a.Ho + DW_ROWS - 1) / DW_ROWS;
  const int per_img = row_tiles * a.Wo * cg;     // < 2^24, checked on the host
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= per_img) return;
  const int b = blockIdx.y;                      // one grid row per image
  int g, ox;
  const int t = fdivmod(i, cg, 1.0f / (float)cg, g);
  const int rt = fdivmod(t, a.Wo, 1.0f / (float)a.Wo, ox);
  const int c0 = g * 8;
  const int oy0 = rt * DW_ROWS;

  const T* wp = reinterpret_cast<const T*>(a.w);
  float wv[9][8];
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    G gw = E::load(wp + (int64_t)k * a.C + c0);
    const T* ew = reinterpret_cast<const T*>(&gw);
#pragma unroll
    for (int c = 0; c < 8; ++c) wv[k][c] = E::to_f(ew[c]);
  }
  float acc[DW_ROWS][8];
#pragma unroll
  for (int r = 0; r < DW_ROWS; ++r)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[r][c] = 0.f;

  const T* x = reinterpret_cast<const T*>(a.x) + (int64_t)b * a.H * a.W * a.x_pitch + c0;
  const int iy0 = oy0 * S - 1, ix0 = ox * S - 1;
#pragma unroll
  for (int rr = 0; rr < NR; ++rr) {
    const int iy = iy0 + rr;
    const bool rok = iy >= 0 && iy < a.H;
    G gv[3];
#pragma unroll
    for (int kx = 0; kx < 3; ++kx) {
      const int ix = ix0 + kx;
      gv[kx] = (rok && ix >= 0 && ix < a.W) ? E::load(x + ((int64_t)iy * a.W + ix) * a.x_pitch) : E::zero();
    }
#pragma unroll
    for (int kx = 0; kx < 3; ++kx) {
      const T* ev = reinterpret_cast<const T*>(&gv[kx]);
      float xv[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) xv[c] = E::to_f(ev[c]);
#pragma unroll
      for (int r = 0; r < DW_ROWS; ++r) {
        const int ky = rr - r * S;   // tap row for output row oy0 + r (compile-time)
        if (ky < 0 || ky > 2) continue;
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[r][c] += wv[ky * 3 + kx][c] * xv[c];
      }
    }
  }
  T* y = reinterpret_cast<T*>(a.y);
  float sc[8], sh[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) { sc[c] = a.scale[c0 + c]; sh[c] = a.shift[c0 + c]; }
#pragma unroll
  for (int r = 0; r < DW_ROWS; ++r) {
    const int oy = oy0 + r;
    if (oy >= a.Ho) break;
    G out;
    T* ov = reinterpret_cast<T*>(&out);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float v = acc[r][c] * sc[c] + sh[c];
      if (a.act == VRS_ACT_SILU) v = silu_t<T>(v);
      ov[c] = E::from_f(v);
    }
    E::store(y + (((int64_t)b * a.Ho + oy) * a.Wo + ox) * a.y_pitch + c0, out);
  }
}
}  // namespace

// ---------------------------------------------------------------------------
// Stride-1 depthwise 3x3, row walking.  A wave owns 8 output columns x 64
// channels (lane = channel group g + 8 * column cx) of one band of RB output
// rows and walks down the band's RB + 2 input rows once: each lane loads its
// own column (16 bytes per bf16 group), takes the left/right neighbours from
// the lanes 8 below/above (ds_bpermute), and only the patch's edge lanes load
// the halo column.  Every input row feeds the three output rows it touches
// through a 3-slot accumulator ring, so an input pixel is read once per band
// (plus the 2-row band halo) instead of once per tap.  Loads run five rows
// ahead in a 6-slot ring (bf16; the kernel is bound by the bytes it keeps in
// flight: two waves per SIMD at ~230 registers), and rows past the band are
// not fetched.  The four waves of a workgroup take adjacent column patches so
// their edge columns meet in L1.
template <typename T, int RB>
__device__ __forceinline__ void dww_body(const vrs_dw_args& a) {
  using E = Elt<T>;
  using G = typename E::group;
  constexpr int NW = (int)sizeof(G) / 4;          // dwords per group
  // prefetch ring slots (rows in flight + 1); float32 rows take twice the
  // registers, so the parity path keeps three
  constexpr int NP = sizeof(T) == 2 ? 6 : 3;
  static_assert((RB + 2) % NP == 0, "rows per band: RB + 2 must be a multiple of the ring");
  // the accumulator slot of band row u (u % 3) is taken from its prefetch
  // slot u % NP at compile time, which needs NP to be a multiple of 3
  static_assert(NP % 3 == 0, "prefetch ring: a multiple of the 3-slot accumulator ring");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int gl = lane & 7, cx = lane >> 3;
  // workgroup -> (image, band, channel block, 4 adjacent patches)
  const int pq = (a.patches + 3) >> 2;
  int wgi = blockIdx.x;
  const int pquad = wgi % pq; wgi /= pq;
  const int cb = wgi % a.cblocks; wgi /= a.cblocks;
  const int band = wgi % a.bands;
  const int b = wgi / a.bands;
  const int patch = pquad * 4 + wave;
  if (patch >= a.patches) return;                 // a workgroup's spare waves (no barriers here)
  const int ox = patch * 8 + cx;
  const int c0 = cb * 64 + gl * 8;
  const bool cok = c0 < a.C && patch < a.patches;
  const bool colok = cok && ox < a.W;             // stride 1: Wo == W, Ho == H
  const int oy0 = band * RB;

  float wv[9][8];
  {
    const T* wp = reinterpret_cast<const T*>(a.w);
    const int cw = cok ? c0 : 0;
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      G gw = E::load(wp + (int64_t)k * a.C + cw);
      const T* ew = reinterpret_cast<const T*>(&gw);
#pragma unroll
      for (int c = 0; c < 8; ++c) wv[k][c] = E::to_f(ew[c]);
    }
  }
  float sc[8], sh[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    sc[c] = a.scale[(cok ? c0 : 0) + c];
    sh[c] = a.shift[(cok ? c0 : 0) + c];
  }

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes);
  const int img = b * a.H;
  // halo column of the patch-edge lanes: left for cx == 0, right for cx == 7
  const int hx = cx == 0 ? ox - 1 : (cx == 7 ? ox + 1 : -1);
  const bool hok = cok && (cx == 0 || cx == 7) && (unsigned)hx < (unsigned)a.W;
  auto row_off = [&](int iy, int xx, bool ok) -> uint32_t {
    return (ok && (unsigned)iy < (unsigned)a.H)
               ? (uint32_t)((((img + iy) * a.W + xx) * a.x_pitch + c0) * (int)sizeof(T))
               : kOOB;
  };
  G own[NP], halo[NP];   // prefetch ring of input rows (own column, halo column)
  // band row u (0..RB+1) into slot u % NP; rows past the band read nothing
  auto fetch = [&](int slot, int u) {
    const bool in = u < RB + 2;
    own[slot] = E::bload(rx, row_off(oy0 - 1 + u, ox, colok && in), 0);
    halo[slot] = E::bload(rx, row_off(oy0 - 1 + u, hx, hok && in), 0);
  };

  float acc[3][8];
#pragma unroll
  for (int s = 0; s < 3; ++s)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[s][c] = 0.f;

  T* y = reinterpret_cast<T*>(a.y);
  // Input row u of the band (0..RB+1) sits in prefetch slot u % NP and feeds
  // output rows v = u - ky (ky = 0..2) through accumulator slot v % 3; after
  // row u, output row u - 2 is complete (slot (u + 1) % 3).  q = u % NP.
  auto process = [&](int q, int u) {
    const int p = q % 3;
    const uint32_t* ov = reinterpret_cast<const uint32_t*>(&own[q]);
    const uint32_t* hv = reinterpret_cast<const uint32_t*>(&halo[q]);
    uint32_t lw[NW], rw[NW];
#pragma unroll
    for (int d = 0; d < NW; ++d) {
      const uint32_t fromleft = (uint32_t)__shfl((int)ov[d], cx == 0 ? lane : lane - 8);
      const uint32_t fromright = (uint32_t)__shfl((int)ov[d], cx == 7 ? lane : lane + 8);
      lw[d] = cx == 0 ? hv[d] : fromleft;
      rw[d] = cx == 7 ? hv[d] : fromright;
    }
    const T* el = reinterpret_cast<const T*>(lw);
    const T* eo = reinterpret_cast<const T*>(ov);
    const T* er = reinterpret_cast<const T*>(rw);
    float xv[3][8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      xv[0][c] = E::to_f(el[c]);
      xv[1][c] = E::to_f(eo[c]);
      xv[2][c] = E::to_f(er[c]);
    }
#pragma unroll
    for (int ky = 0; ky < 3; ++ky) {
      const int s = ((p - ky) % 3 + 3) % 3;   // accumulator slot of v = u - ky (static)
#pragma unroll
      for (int kx = 0; kx < 3; ++kx)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[s][c] += wv[ky * 3 + kx][c] * xv[kx][c];
    }
    const int sv = (p + 1) % 3;
    const int oy = oy0 + u - 2;
    if (u >= 2 && oy < a.H && colok) {
      G out;
      T* o = reinterpret_cast<T*>(&out);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float t = acc[sv][c] * sc[c] + sh[c];
        if (a.act == VRS_ACT_SILU) t = silu_t<T>(t);
        o[c] = E::from_f(t);
      }
      E::store(y + ((int64_t)(img + oy) * a.W + ox) * a.y_pitch + c0, out);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[sv][c] = 0.f;
  };

#pragma unroll
  for (int q = 0; q < NP - 1; ++q) fetch(q, q);
  for (int u = 0; u < RB + 2; u += NP) {
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      fetch((q + NP - 1) % NP, u + q + NP - 1);
      process(q, u + q);
    }
  }
}

extern "C" __global__ __launch_bounds__(256) void vrs_dwconv3_s1w40_bf16(vrs_dw_args a) { dww_body<bf16_t, 40>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_dwconv3_s1w10_bf16(vrs_dw_args a) { dww_body<bf16_t, 10>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_dwconv3_s1w40_f32(vrs_dw_args a) { dww_body<float, 40>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_dwconv3_s1w10_f32(vrs_dw_args a) { dww_body<float, 10>(a); }

extern "C" __global__ __launch_bounds__(256) void vrs_dwconv3_s1_bf16(vrs_dw_args a) { dw_body<bf16_t, 1>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_dwconv3_s2_bf16(vrs_dw_args a) { dw_body<bf16_t, 2>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_dwconv3_s1_f32(vrs_dw_args a) { dw_body<float, 1>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_dwconv3_s2_f32(vrs_dw_args a) { dw_body<float, 2>(a); }

// ---------------------------------------------------------------------------
// Grouped conv with 1 < groups < channels + folded BN (+ SiLU) (+ residual):
// conv_bn with any g (blocks/conv.rs:51-69, Conv2d::new_grouped) for groups
// whose per-group channel counts do not fit the implicit-GEMM tiles.  Direct
// form: one thread per output element, channel fastest across lanes, so the
// lanes of one group read the same input pixels (one cache line) and each
// lane streams its own weight row [k][k][cin_g].  float32 accumulation in
// (ky, kx, ci) order.
namespace {
template <typename T>
__device__ __forceinline__ void gconv_body(const vrs_gconv_args& a) {
  using E = Elt<T>;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.total) return;
  const int co = (int)(i % a.cout);
  const int64_t pix = i / a.cout;                // (b*Ho + oy)*Wo + ox
  const int ox = (int)(pix % a.Wo);
  const int64_t bo = pix / a.Wo;
  const int oy = (int)(bo % a.Ho);
  const int64_t b = bo / a.Ho;
  const T* x = static_cast<const T*>(a.x) + (int64_t)(co / a.cout_g) * a.cin_g;
  const T* w = static_cast<const T*>(a.w) + (int64_t)co * a.k * a.k * a.cin_g;
  float acc = 0.f;
  for (int ky = 0; ky < a.k; ++ky) {
    const int iy = oy * a.stride - a.pad + ky;
    if (iy < 0 || iy >= a.H) continue;
    for (int kx = 0; kx < a.k; ++kx) {
      const int ix = ox * a.stride - a.pad + kx;
      if (ix < 0 || ix >= a.W) continue;
      const T* xp = x + ((b * a.H + iy) * a.W + ix) * a.x_pitch;
      const T* wp = w + (ky * a.k + kx) * a.cin_g;
      for (int c = 0; c < a.cin_g; ++c) acc = fmaf(E::to_f(xp[c]), E::to_f(wp[c]), acc);
    }
  }
  float v = acc * a.scale[co] + a.shift[co];
  if (a.act == VRS_ACT_SILU) v = silu_t<T>(v);
  if (a.res) v += E::to_f(static_cast<const T*>(a.res)[pix * a.r_pitch + co]);
  static_cast<T*>(a.y)[pix * a.y_pitch + co] = E::from_f(v);
}
}  // namespace

extern "C" __global__ __launch_bounds__(256) void vrs_gconv_bf16(vrs_gconv_args a) { gconv_body<bf16_t>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_gconv_f32(vrs_gconv_args a) { gconv_body<float>(a); }

// ---------------------------------------------------------------------------
// SPPF pooling cascade (blocks/sppf.rs:43-61): p1 = max5(y), p2 = max5(p1),
// p3 = max5(p2), stride 1, pad 2 with -inf semantics (windows clipped to the
// map, teeny-core MaxPool2d::with_padding at blocks/sppf.rs:48-50).
// One workgroup owns one image and 8*cgroups_per_block channels; the plane is
// staged in LDS and every 5x5 max is done separably (row pass, column pass).
// Max of stored values is exact, so LDS keeps the element type.
namespace {
constexpr int POOL_LDS_BYTES = 48 * 1024;

template <typename T>
__device__ __forceinline__ void pool_body(const vrs_pool_args& a) {
  using E = Elt<T>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int HW = a.H * a.W;
  const int CG = a.cgroups_per_block;             // channel groups of 8 per block
  const int groups_total = a.c >> 3;
  const int blocks_per_img = (groups_total + CG - 1) / CG;
  const int b = blockIdx.x / blocks_per_img;
  const int g0 = (blockIdx.x % blocks_per_img) * CG;
  const int ng = min(CG, groups_total - g0);
  // two planes of [HW][ng*8] elements: cur and tmp
  T* cur = reinterpret_cast<T*>(smem);
  T* tmp = cur + (size_t)HW * CG * 8;
  T* base = reinterpret_cast<T*>(a.buf) + (int64_t)b * HW * a.pitch;
  const int nvec = HW * ng;  // (pixel, group) items

  for (int it = threadIdx.x; it < nvec; it += blockDim.x) {
    const int p = it / ng, g = it - p * ng;
    E::store(cur + ((size_t)p * CG + g) * 8, E::load(base + (int64_t)p * a.pitch + (g0 + g) * 8));
  }
  __syncthreads();
  for (int stage = 1; stage <= 3; ++stage) {
    // row pass: tmp = max over x-window of cur
    for (int it = threadIdx.x; it < nvec; it += blockDim.x) {
      const int p = it / ng, g = it - p * ng;
      const int y = p / a.W, xx = p - y * a.W;
      float m[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) m[c] = -INFINITY;
      for (int dx = -2; dx <= 2; ++dx) {
        const int xs = xx + dx;
        if (xs < 0 || xs >= a.W) continue;
        const T* s = cur + ((size_t)(y * a.W + xs) * CG + g) * 8;
#pragma unroll
        for (int c = 0; c < 8; ++c) m[c] = fmaxf(m[c], E::to_f(s[c]));
      }
      T* d = tmp + ((size_t)p * CG + g) * 8;
#pragma unroll
      for (int c = 0; c < 8; ++c) d[c] = E::from_f(m[c]);
    }
    __syncthreads();
    // column pass: cur = max over y-window of tmp; also write to the buffer
    for (int it = threadIdx.x; it < nvec; it += blockDim.x) {
      const int p = it / ng, g = it - p * ng;
      const int y = p / a.W, xx = p - y * a.W;
      float m[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) m[c] = -INFINITY;
      for (int dy = -2; dy <= 2; ++dy) {
        const int ys = y + dy;
        if (ys < 0 || ys >= a.H) continue;
        const T* s = tmp + ((size_t)(ys * a.W + xx) * CG + g) * 8;
#pragma unroll
        for (int c = 0; c < 8; ++c) m[c] = fmaxf(m[c], E::to_f(s[c]));
      }
      typename E::group out;
      T* ov = reinterpret_cast<T*>(&out);
#pragma unroll
      for (int c = 0; c < 8; ++c) ov[c] = E::from_f(m[c]);
      E::store(cur + ((size_t)p * CG + g) * 8, out);
      E::store(base + (int64_t)p * a.pitch + stage * a.c + (g0 + g) * 8, out);
    }
    __syncthreads();
  }
}
}  // namespace

extern "C" __global__ __launch_bounds__(256) void vrs_sppf_pool_bf16(vrs_pool_args a) { pool_body<bf16_t>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_sppf_pool_f32(vrs_pool_args a) { pool_body<float>(a); }

// Wave-per-channel-group SPPF pool (bfloat16, maps of up to 682 pixels: the
// 20x20 of YOLO26 at 640).  A wave owns one (image, 8-channel group) and keeps
// three planes of the map in LDS; the G waves of a workgroup take adjacent
// groups, so each pixel's reads and writes span 16*G contiguous bytes.  The cascade p1 = max5(y), p2 = max5(p1),
// p3 = max5(p2) with -inf padding equals windows of 5, 9 and 13 clipped to
// the map, computed separably: row windows R5 (five reads), R9 = max(R5 at
// x-2, x+2), R13 = max(R9 at x-2, x+2) (neighbours clamped to the row: the
// clamped position always lies inside the clipped window), then column
// windows of 5, 9 and 13 rows of R5, R9, R13.  Each pass spreads the map's
// pixels over the 64 lanes.  bfloat16 values are compared as ordered 16-bit
// integers (the sign-magnitude bits with the magnitude flipped for negative
// values), two per packed v_pk_max_i16.
namespace {
typedef short i16x8v_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ uint32_t ord_bf16x2(uint32_t u) { return u ^ (((u >> 15) & 0x00010001u) * 0x7fffu); }
__device__ __forceinline__ u32x4_t ord16(u32x4_t v) {
  return (u32x4_t){ord_bf16x2(v[0]), ord_bf16x2(v[1]), ord_bf16x2(v[2]), ord_bf16x2(v[3])};
}
__device__ __forceinline__ u32x4_t max16(u32x4_t a, u32x4_t b) {
  return __builtin_bit_cast(u32x4_t, __builtin_elementwise_max(__builtin_bit_cast(i16x8v_t, a),
                                                               __builtin_bit_cast(i16x8v_t, b)));
}

// Vertical window of 2R+1 rows (clipped to the map) over column x of plane
// Pl for output rows y0..y0+3, stored at channel offset coff of each pixel.
// Rows y0-R .. y0+3+R are read once (clamped to the map: a clamped row lies
// inside every clipped window that asks for it); rows y0-R+3 .. y0+R lie in
// all four windows.
template <int R>
__device__ __forceinline__ void pool_col4(const u32x4_t* Pl, int x, int y0, int W, int H, bf16_t* base, int pitch,
                                          int coff) {
  u32x4_t v[2 * R + 4];
#pragma unroll
  for (int k = 0; k < 2 * R + 4; ++k) v[k] = Pl[min(max(y0 - R + k, 0), H - 1) * W + x];
  u32x4_t common = v[3];
#pragma unroll
  for (int k = 4; k <= 2 * R; ++k) common = max16(common, v[k]);
  const u32x4_t o[4] = {max16(max16(max16(common, v[0]), v[1]), v[2]),
                        max16(max16(max16(common, v[1]), v[2]), v[2 * R + 1]),
                        max16(max16(max16(common, v[2]), v[2 * R + 1]), v[2 * R + 2]),
                        max16(max16(max16(common, v[2 * R + 1]), v[2 * R + 2]), v[2 * R + 3])};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (y0 + i < H) *reinterpret_cast<u32x4_t*>(base + (int64_t)((y0 + i) * W + x) * pitch + coff) = ord16(o[i]);
}

template <int G>
__device__ __forceinline__ void pool_wave_body(const vrs_pool_args& a) {
  extern __shared__ __attribute__((aligned(16))) u32x4_t pw_sm[];
  const int W = a.W, H = a.H, HW = H * W;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int groups = a.c >> 3;
  // consecutive channel groups of an image stay on one XCD, so the partial
  // 16-byte pixel reads and writes of its waves meet in the same L2
  const int gid = xcd_remap(blockIdx.x, gridDim.x) * G + wave;
  const bool live = gid < a.N * groups;       // idle waves still take part in the barriers
  const int b = live ? gid / groups : 0, g = live ? gid % groups : 0;
  u32x4_t* P0 = pw_sm + wave * 3 * HW;
  u32x4_t* P1 = P0 + HW;
  u32x4_t* P2 = P1 + HW;
  bf16_t* base = reinterpret_cast<bf16_t*>(a.buf) + (int64_t)b * HW * a.pitch + g * 8;
  if (live)
    for (int p0 = lane; p0 < HW; p0 += 8 * 64) {   // eight loads in flight per lane
      u32x4_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (p0 + j * 64 < HW) v[j] = *reinterpret_cast<const u32x4_t*>(base + (int64_t)(p0 + j * 64) * a.pitch);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (p0 + j * 64 < HW) P0[p0 + j * 64] = ord16(v[j]);
    }
  __syncthreads();
  if (live)
    for (int p = lane; p < HW; p += 64) {   // R5 -> P1
      const int x = p % W, row = p - x;
      u32x4_t m = P0[p];
#pragma unroll
      for (int d = 1; d <= 2; ++d) m = max16(max16(m, P0[row + max(x - d, 0)]), P0[row + min(x + d, W - 1)]);
      P1[p] = m;
    }
  __syncthreads();
  if (live)
    for (int p = lane; p < HW; p += 64) {   // R9 -> P2
      const int x = p % W, row = p - x;
      P2[p] = max16(P1[row + max(x - 2, 0)], P1[row + min(x + 2, W - 1)]);
    }
  __syncthreads();
  if (live)
    for (int p = lane; p < HW; p += 64) {   // R13 -> P0 (y is no longer needed)
      const int x = p % W, row = p - x;
      P0[p] = max16(P2[row + max(x - 2, 0)], P2[row + min(x + 2, W - 1)]);
    }
  __syncthreads();
  if (!live) return;
  // column windows -> p1, p2, p3: a lane takes four rows y0..y0+3 of one
  // column (lanes on consecutive columns), reading each needed row once
  const int QH = (H + 3) >> 2;
  for (int it = lane; it < W * QH; it += 64) {
    const int x = it % W, y0 = (it / W) * 4;
    pool_col4<2>(P1, x, y0, W, H, base, a.pitch, a.c);
    pool_col4<4>(P2, x, y0, W, H, base, a.pitch, 2 * a.c);
    pool_col4<6>(P0, x, y0, W, H, base, a.pitch, 3 * a.c);
  }
}
}  // namespace

extern "C" __global__ __launch_bounds__(256) void vrs_sppf_pool_w4_bf16(vrs_pool_args a) { pool_wave_body<4>(a); }
extern "C" __global__ __launch_bounds__(128) void vrs_sppf_pool_w2_bf16(vrs_pool_args a) { pool_wave_body<2>(a); }
extern "C" __global__ __launch_bounds__(64) void vrs_sppf_pool_w1_bf16(vrs_pool_args a) { pool_wave_body<1>(a); }

// ---------------------------------------------------------------------------
// Nearest 2x upsample (blocks/upsample.rs:23-35) into a channel slice of a
// concat buffer (blocks/concat.rs:24-38): y[b, oy, ox, c] = x[b, oy/2, ox/2, c].
template <typename T>
__device__ __forceinline__ void up_body(const vrs_up_args& a) {
  using E = Elt<T>;
  const int cg = a.C >> 3;
  const int Ho = a.H * 2, Wo = a.W * 2;
  const int64_t total = (int64_t)a.N * Ho * Wo * cg;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int g = (int)(i % cg);
  int64_t t = i / cg;
  const int ox = (int)(t % Wo); t /= Wo;
  const int oy = (int)(t % Ho);
  const int b = (int)(t / Ho);
  const T* x = reinterpret_cast<const T*>(a.x);
  T* y = reinterpret_cast<T*>(a.y);
  E::store(y + (((int64_t)b * Ho + oy) * Wo + ox) * a.y_pitch + g * 8,
           E::load(x + (((int64_t)b * a.H + (oy >> 1)) * a.W + (ox >> 1)) * a.x_pitch + g * 8));
}

extern "C" __global__ __launch_bounds__(256) void vrs_upsample2x_bf16(vrs_up_args a) { up_body<bf16_t>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_upsample2x_f32(vrs_up_args a) { up_body<float>(a); }

// ---------------------------------------------------------------------------
// Calibration reduction for the fp8 path: max |x| of a bfloat16 NHWC view.
// Lanes take 8-channel groups (16 bytes) in a grid-stride loop; the wave
// maximum goes out with one atomic max on the float bits (non-negative
// floats order like their bit patterns).
extern "C" __global__ __launch_bounds__(256) void vrs_absmax_bf16(vrs_absmax_args a) {
  const int cg = a.c >> 3;
  const int64_t n = a.npix * cg;
  float m = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t p = i / cg;
    const int g = (int)(i - p * cg);
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const bf16_t*>(a.x) + p * a.pitch + g * 8);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      m = fmaxf(m, fabsf(__uint_as_float(v[d] << 16)));
      m = fmaxf(m, fabsf(__uint_as_float(v[d] & 0xffff0000u)));
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if ((threadIdx.x & 63) == 0) atomicMax(a.out, __float_as_uint(m));
}

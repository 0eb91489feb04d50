// Weight-stationary 1x1 convolution + folded BatchNorm + SiLU for gfx950
// (bfloat16, stride 1, no residual).
//
// Semantics as the dense conv (blocks/conv.rs:31-46 with k = 1):
// y[p, co] = act(scale[co] * sum_ci W[co, ci] x[p, ci] + shift[co]).
//
// The memory-bound 1x1 layers (Cin <= 256) spend most of a tiled GEMM's
// in-flight capacity re-reading the weight tile from L2 for every pixel
// tile.  Here a persistent workgroup keeps one BM-channel slice of the
// weights in LDS for its whole run and streams 64-pixel tiles through it:
//
// * 512 threads (8 wave64), one slice of BM output channels (the grid is a
//   multiple of the slice count; the slices of one pixel stream are
//   neighbouring logical blocks, so they share an XCD and its L2 serves the
//   later slices' pixel reads);
// * a tile is 64 pixels x all Cin channels, loaded as whole pixel rows
//   (Cin*2 contiguous bytes) into registers two tiles ahead and written into
//   one of two LDS buffers one tile ahead: one barrier per tile;
// * wave tile 32 channels x (64 / waves-per-column) pixels on
//   v_mfma_f32_32x32x16_bf16, the whole K = Cin per tile from LDS;
// * epilogue straight from the accumulators: each lane owns 4 consecutive
//   channels of one pixel per register quad, stored as one 8-byte raw-buffer
//   store (out-of-range pixels and channels get an offset the resource
//   rejects).  The folded-BN constants of the wave's channels are read once;
//   tile k-1's epilogue is interleaved with tile k's MFMAs (two accumulator
//   sets).
//
// LDS rows are Cin + 8 elements: the 32 rows a fragment read touches start
// on distinct 4-bank groups for every Cin that is a multiple of 64.
//
// NC > 1 (Cin 384: a 128-channel weight slice is 98 KB, and two whole
// 64-pixel tiles would not fit beside it): a tile streams through the LDS
// double buffer as NC chunks of Cin/NC channels (the pixel rows' matching
// byte ranges), one barrier per chunk; the tile's accumulators carry over
// its chunks and the previous tile's epilogue is spread over all of them.
#include "common.h"

namespace {

constexpr int W1_BN = 64;    // pixels per tile
constexpr int W1_NT = 512;   // threads per workgroup

// FLAT: float32 output with the channel stride a.y_sc (the Detect head's
// channel-major outputs, y_sp == 1): each value of a store unit goes out as
// its own dword store, the 32 lanes of a half-wave covering 32 consecutive
// pixels of one channel.
template <int BM, int CIN, bool FLAT = false, int NC = 1>
__device__ __forceinline__ void conv1w_body(const vrs_conv_args& a) {
  using E = Elt<bf16_t>;
  using G = E::group;
  constexpr int KCH = CIN / NC;                // input channels per pixel chunk
  constexpr int LDK = CIN + 8;                 // LDS row stride of the weights (elements)
  constexpr int LDB = KCH + 8;                 // LDS row stride of a pixel chunk
  constexpr int CPR = CIN / 8;                 // 16-byte pieces per weight row
  constexpr int CPB = KCH / 8;                 // 16-byte pieces per pixel chunk row
  constexpr int NCH = W1_BN * CPB / W1_NT;     // pixel pieces per thread per chunk
  constexpr int NWI = BM * CPR / W1_NT;        // weight pieces per thread
  static_assert(CIN % (64 * NC) == 0 && W1_BN * CPB % W1_NT == 0 && BM * CPR % W1_NT == 0, "whole pieces");
  constexpr int WGM = BM / 32 < 8 ? BM / 32 : 8, WGN = 8 / WGM;
  constexpr int WTM = BM / WGM, WTN = W1_BN / WGN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
  __shared__ __attribute__((aligned(16))) bf16_t sW[BM * LDK];
  __shared__ __attribute__((aligned(16))) bf16_t sB0[W1_BN * LDB];
  __shared__ __attribute__((aligned(16))) bf16_t sB1[W1_BN * LDB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int frag_row = lane & 31, hq = lane >> 5;
  // workgroup -> (channel slice, pixel stream); the host sizes the grid as a
  // multiple of tiles_m
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int slice = L % a.tiles_m, stream = L / a.tiles_m;
  const int streams = gridDim.x / a.tiles_m;
  const int T = a.tiles_n;
  const int nt = stream < T ? (T - 1 - stream) / streams + 1 : 0;   // tiles of this workgroup
  if (nt == 0) return;   // uniform over the workgroup, before any barrier
  const int m0 = slice * BM;

  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w, a.w_bytes);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y, a.y_bytes);

  // weight slice -> LDS, once (rows past Cout read zeros)
  {
    G wv[NWI];
#pragma unroll
    for (int i = 0; i < NWI; ++i) {
      const int q = tid + i * W1_NT, r = q / CPR, c = q % CPR;
      wv[i] = E::bload(rw, m0 + r < a.Cout ? (uint32_t)(((m0 + r) * CIN + c * 8) * 2) : kOOB, 0);
    }
#pragma unroll
    for (int i = 0; i < NWI; ++i) {
      const int q = tid + i * W1_NT;
      E::store(&sW[(q / CPR) * LDK + (q % CPR) * 8], wv[i]);
    }
  }

  // this thread's pixel pieces: row (pixel within the tile) and element
  // column within the chunk, the same for every chunk
  int b_row[NCH], b_col[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int q = tid + i * W1_NT;
    b_row[i] = q / CPB;
    b_col[i] = (q % CPB) * 8;
  }
  const uint32_t pitch_b = (uint32_t)a.x_pitch * 2u;
  // chunk c = tile c / NC, channels (c % NC) * KCH onwards
  auto load_chunk = [&](int c, G (&R)[NCH]) {
    const int k = c / NC;
    const int n0 = (stream + k * streams) * W1_BN;
    const bool live = k < nt;
    const int c0 = (c % NC) * KCH;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int m = n0 + b_row[i];
      R[i] = E::bload(rx, live && m < a.M ? (uint32_t)m * pitch_b + (uint32_t)(c0 + b_col[i]) * 2u : kOOB, 0);
    }
  };
  auto store_chunk = [&](bf16_t* sB, const G (&R)[NCH]) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) E::store(&sB[b_row[i] * LDB + b_col[i]], R[i]);
  };

  // folded-BN constants of this lane's channels: register quad g of MFMA
  // row block i holds channels m0 + wm*WTM + i*32 + g*8 + hq*4 + 0..3
  const ChanConst c_scale(a.scale, a.Cout), c_shift(a.shift, a.Cout);
  const uint32_t hmask = upper_half_mask();
  float sc[TM][4][4], sh[TM][4][4];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      c_scale.quad(m0 + wm * WTM + i * 32 + g * 8, hmask, sc[i][g]);
      c_shift.quad(m0 + wm * WTM + i * 32 + g * 8, hmask, sh[i][g]);
    }
  const int HWo = a.Ho * a.Wo;
  const float inv_hwo = 1.0f / (float)HWo;

  // Tile k's MFMAs run into one accumulator set while the epilogue of tile
  // k-1 drains the other, a few store units (4 channels of one pixel) after
  // each 16-deep k slice: its VALU work (two transcendentals per value)
  // issues between MFMAs instead of after them.
  constexpr int KK = KCH / 16;       // 16-deep k slices per chunk
  constexpr int NU = TN * TM * 4;   // store units per tile and lane
  constexpr int NUC = NU / NC;      // of them drained per chunk
  static_assert(NU % NC == 0, "store units per chunk");
  struct Out { uint32_t pix[TN]; bool ok[TN]; };
  auto out_addr = [&](int k) {   // tile k's per-lane pixel offsets (none for k < 0)
    Out o;
    const int n0 = (stream + k * streams) * W1_BN;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int m = n0 + wn * WTN + j * 32 + frag_row;
      o.ok[j] = k >= 0 && m < a.M;
      int pp;
      const int bb = fdivmod(o.ok[j] ? m : 0, HWo, inv_hwo, pp);
      o.pix[j] = (uint32_t)(((int64_t)bb * a.y_sb + (int64_t)pp * a.y_sp) * (FLAT ? 4 : 2));
    }
    return o;
  };
  auto epi_unit = [&](int u, const f32x16_t (&ap)[TM][TN], const Out& o) {
    const int j = u / (TM * 4), i = (u / 4) % TM, g = u % 4;
    const int co = m0 + wm * WTM + i * 32 + g * 8 + hq * 4;
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float t = ap[i][j][g * 4 + r] * sc[i][g][r] + sh[i][g][r];
      if (a.act == VRS_ACT_SILU) t = silu_fast(t);
      v[r] = t;
    }
    if constexpr (FLAT) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t off = o.ok[j] && co + r < a.Cout ? o.pix[j] + (uint32_t)((co + r) * a.y_sc * 4) : kOOB;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[r]), ry, off, 0, 0);
      }
    } else {
      const uint32_t off = o.ok[j] && co < a.Cout ? o.pix[j] + (uint32_t)co * 2u : kOOB;
      __builtin_amdgcn_raw_buffer_store_b64((u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])}, ry, off, 0,
                                            0);
    }
  };
  // chunk h of a tile: its first zeroes the accumulators
  auto compute = [&](const bf16_t* sB, int h, f32x16_t (&ac)[TM][TN], const f32x16_t (&ap)[TM][TN],
                     const Out& op) {
    if (h == 0) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) ac[i][j][r] = 0.f;
    }
    const bf16_t* pa = sW + (wm * WTM + frag_row) * LDK + h * KCH + hq * 8;
    const bf16_t* pb = sB + (wn * WTN + frag_row) * LDB + hq * 8;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      G fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = E::load(pa + i * 32 * LDK + kk * 16);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = E::load(pb + j * 32 * LDB + kk * 16);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) ac[i][j] = mfma32_k16(fa[i], fb[j], ac[i][j]);
#pragma unroll
      for (int u = h * NUC + kk * NUC / KK; u < h * NUC + (kk + 1) * NUC / KK; ++u) epi_unit(u, ap, op);
    }
  };

  // chunk c: LDS buffer c&1 holds it; register set (c+1)&1 holds chunk c+1
  // (written to the other buffer during chunk c); set c&1 receives chunk
  // c+2; accumulator set k&1 receives tile k = c / NC while set (k+1)&1
  // drains tile k-1
  G r0[NCH], r1[NCH];
  f32x16_t acc0[TM][TN], acc1[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc1[i][j][r] = 0.f;
  load_chunk(0, r0);
  load_chunk(1, r1);
  store_chunk(sB0, r0);
  __syncthreads();
  auto step = [&](const bf16_t* cur, bf16_t* nxt, G (&ld)[NCH], const G (&st)[NCH], f32x16_t (&ac)[TM][TN],
                  const f32x16_t (&ap)[TM][TN], int k, int h) {   // h: a constant at every call
    load_chunk(k * NC + h + 2, ld);
    store_chunk(nxt, st);
    compute(cur, h, ac, ap, out_addr(k - 1));
    __syncthreads();
  };
  if constexpr (NC == 1) {
    for (int k = 0; k < nt; k += 2) {
      step(sB0, sB1, r0, r1, acc0, acc1, k, 0);
      if (k + 1 < nt) step(sB1, sB0, r1, r0, acc1, acc0, k + 1, 0);
    }
  } else {
    static_assert(NC == 2, "chunks per tile: 1 or 2");
    for (int k = 0; k < nt; k += 2) {
      step(sB0, sB1, r0, r1, acc0, acc1, k, 0);
      step(sB1, sB0, r1, r0, acc0, acc1, k, 1);
      if (k + 1 < nt) {
        step(sB0, sB1, r0, r1, acc1, acc0, k + 1, 0);
        step(sB1, sB0, r1, r0, acc1, acc0, k + 1, 1);
      }
    }
  }
  // the last tile's epilogue
  const Out ol = out_addr(nt - 1);
  if ((nt - 1) & 1) {
#pragma unroll
    for (int u = 0; u < NU; ++u) epi_unit(u, acc1, ol);
  } else {
#pragma unroll
    for (int u = 0; u < NU; ++u) epi_unit(u, acc0, ol);
  }
}
}  // namespace

// vrs_conv1w_bf16_<BM>_c<Cin>: LDS = (BM + 128) * (Cin + 8) * 2 bytes
// (256 x 192: 150 KB, one workgroup per CU; 128 x 64: 24.8 KB); _c384 in
// two chunks: 128 * 392 * 2 + 128 * 200 * 2 = 148 KB.
#define VRS_CONV1W(BM, CIN)                                                                        \
  extern "C" __global__ __launch_bounds__(512) void vrs_conv1w_bf16_##BM##_c##CIN(vrs_conv_args a) { \
    conv1w_body<BM, CIN>(a);                                                                       \
  }
VRS_CONV1W(256, 64)
VRS_CONV1W(256, 128)
VRS_CONV1W(256, 192)
VRS_CONV1W(128, 64)
VRS_CONV1W(128, 128)
VRS_CONV1W(128, 192)
VRS_CONV1W(128, 256)
extern "C" __global__ __launch_bounds__(512) void vrs_conv1w_bf16_128_c384(vrs_conv_args a) {
  conv1w_body<128, 384, false, 2>(a);
}
// float32 channel-major outputs (the Detect head's box and class convs)
#define VRS_CONV1W_F(BM, CIN)                                                                        \
  extern "C" __global__ __launch_bounds__(512) void vrs_conv1w_bf16_##BM##_c##CIN##_f(vrs_conv_args a) { \
    conv1w_body<BM, CIN, true>(a);                                                                     \
  }
VRS_CONV1W_F(128, 64)
VRS_CONV1W_F(128, 256)

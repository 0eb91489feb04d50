// Weight-stationary 1x1 convolution + folded BatchNorm (+SiLU) on the fp8
// MFMA for gfx950 (BASELINE config 5's e4m3 run; the layers are
// blocks/conv.rs:31-46 with k = 1): e4m3 weights with a per-output-channel
// step, activations e4m3 (_x8) or bfloat16 quantised to e4m3 on the layer's
// step while staged, output bfloat16 or e4m3 on the output's step (_y8).
//
// As the bfloat16 kernel (conv1w.hip): a persistent workgroup keeps one
// 128-channel slice of the weights in LDS (1 byte per weight: up to 768
// input channels) and streams pixel tiles through it, so the memory-bound
// 1x1 layers spend their loads on pixels instead of re-reading weight tiles
// from L2 for every pixel tile:
//
// * 512 threads (8 wave64 as 4 x 2), a tile is 128 pixels x all Cin
//   channels, loaded as whole pixel rows in NC chunks of Cin/NC channels
//   (registers two chunks ahead, written to one of two LDS buffers after the
//   current chunk's MFMAs, one barrier per chunk);
// * wave tile 32 channels x 64 pixels on v_mfma_scale_f32_32x32x64_f8f6f4
//   (unit block scales): 1.5 fragment reads per MFMA;
// * tile k-1's epilogue (scale*acc + shift, SiLU, rounding, one store per 4
//   channels of a pixel) is spread over tile k's k slices (two accumulator
//   sets).
//
// Results equal the tiled fp8 kernels' (conv_body.h in F8 mode) bit for bit:
// the same e4m3 staging of bfloat16 inputs, the k slices of 64 channels in
// the same order, and an e4m3 output is the e4m3 rounding of the value
// rounded to bfloat16 first.
//
// LDS rows are (channels + 16) bytes: the 16 rows a quarter-wave's 16-byte
// fragment reads touch start on distinct 4-bank groups for every chunk and
// weight width used here (144, 208, 272, 400, 528, 784 bytes).
#include "common.h"

namespace {

constexpr int W8_BN = 128;   // pixels per tile
constexpr int W8_NT = 512;   // threads per workgroup

template <int I, int N, typename F>
__device__ __forceinline__ void w8_static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    w8_static_for<I + 1, N>(f);
  }
}

template <int CIN, int NC, bool XF8, bool YF8>
__device__ __forceinline__ void conv1w8_body(const vrs_conv_args& a) {
  constexpr int BM = 128;                       // output channels per slice
  constexpr int KCH = CIN / NC;                 // input channels per pixel chunk
  constexpr int LDW = CIN + 16;                 // LDS row stride of the weights (bytes)
  constexpr int LDB = KCH + 16;                 // LDS row stride of a pixel chunk (bytes)
  constexpr int CPR = CIN / 16;                 // 16-byte weight pieces per row
  constexpr int CEB = XF8 ? 16 : 8;             // activation elements per 16-byte piece
  constexpr int XS = XF8 ? 1 : 2;               // bytes per activation element in memory
  constexpr int CPB = KCH / CEB;                // pieces per pixel chunk row
  constexpr int NCH = W8_BN * CPB / W8_NT;      // pixel pieces per thread per chunk
  constexpr int NWI = BM * CPR / W8_NT;         // weight pieces per thread
  static_assert(KCH % 64 == 0 && W8_BN * CPB % W8_NT == 0 && BM * CPR % W8_NT == 0, "whole pieces");
  static_assert(NC == 1 || NC == 2 || NC == 4, "chunks per tile");
  constexpr int WGM = 4, WGN = 2;               // waves: 4 over channels x 2 over pixels
  constexpr int WTM = BM / WGM, WTN = W8_BN / WGN;
  constexpr int TM = WTM / 32, TN = WTN / 32;   // 1 x 2 MFMA tiles per wave
  constexpr int KK = KCH / 64;                  // 64-deep k slices per chunk
  __shared__ __attribute__((aligned(16))) unsigned char sW[BM * LDW];
  __shared__ __attribute__((aligned(16))) unsigned char sB0[W8_BN * LDB];
  __shared__ __attribute__((aligned(16))) unsigned char sB1[W8_BN * LDB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int frag_row = lane & 31, hq = lane >> 5;
  // workgroup -> (channel slice, pixel stream); the host sizes the grid as a
  // multiple of tiles_m, so the slices of one stream are neighbouring logical
  // blocks (one XCD: its L2 serves the later slices' pixel reads)
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

  // weight slice -> LDS, once (rows past Cout read zeros); row co holds the
  // co-th output channel's Cin e4m3 weights
  {
    u32x4_t wv[NWI];
#pragma unroll
    for (int i = 0; i < NWI; ++i) {
      const int q = tid + i * W8_NT, r = q / CPR, c = q % CPR;
      wv[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, m0 + r < a.Cout ? (uint32_t)((m0 + r) * CIN + c * 16) : kOOB,
                                                    0, 0);
    }
#pragma unroll
    for (int i = 0; i < NWI; ++i) {
      const int q = tid + i * W8_NT;
      *reinterpret_cast<u32x4_t*>(sW + (q / CPR) * LDW + (q % CPR) * 16) = wv[i];
    }
  }

  // this thread's pixel pieces: pixel row within the tile and piece index
  // within the chunk, the same for every chunk; the byte offset of a piece
  // is b_off (per lane) + tile row * pitch + chunk channel offset (uniform:
  // the scalar offset of the load), so no per-chunk address stays live
  int b_row[NCH], b_col[NCH];
  uint32_t b_off[NCH];
  const uint32_t pitch_b = (uint32_t)a.x_pitch * (uint32_t)XS;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int q = tid + i * W8_NT;
    b_row[i] = q / CPB;
    b_col[i] = q % CPB;
    b_off[i] = (uint32_t)b_row[i] * pitch_b + (uint32_t)(b_col[i] * CEB * XS);
  }
  // chunk c = tile c / NC, channels (c % NC) * KCH onwards; pixels past M
  // (and every pixel of a chunk past the stream's last tile) read zeros
  // through an offset the resource rejects (kOOB plus a scalar offset below
  // 2^31 stays out of range)
  auto load_chunk = [&](int c, u32x4_t (&R)[NCH]) {
    const int k = c / NC;
    const int n0 = (stream + k * streams) * W8_BN;
    const int left = k < nt ? a.M - n0 : 0;   // pixels of the tile inside the view
    const uint32_t soff = k < nt ? (uint32_t)n0 * pitch_b + (uint32_t)((c % NC) * KCH * XS) : 0u;
#pragma unroll
    for (int i = 0; i < NCH; ++i)
      R[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, b_row[i] < left ? b_off[i] : kOOB, soff, 0);
  };
  auto store_chunk = [&](unsigned char* sB, const u32x4_t (&R)[NCH]) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      if constexpr (XF8) {   // 16 e4m3 activations, stored as read
        *reinterpret_cast<u32x4_t*>(sB + b_row[i] * LDB + b_col[i] * 16) = R[i];
      } else {               // 8 bfloat16 -> 8 e4m3 on the input step (as the tiled kernels stage them)
        const u32x4_t v = R[i];
        const u32x2_t q = {bf16x2_to_fp8x2(v[0], a.clamp_bits, a.in_scale) |
                               (bf16x2_to_fp8x2(v[1], a.clamp_bits, a.in_scale) << 16),
                           bf16x2_to_fp8x2(v[2], a.clamp_bits, a.in_scale) |
                               (bf16x2_to_fp8x2(v[3], a.clamp_bits, a.in_scale) << 16)};
        *reinterpret_cast<u32x2_t*>(sB + b_row[i] * LDB + b_col[i] * 8) = q;
      }
    }
  };

  // folded-BN constants of the slice's channels in LDS (visible after the
  // first barrier): a store unit reads its 4 channels' pairs as two 16-byte
  // loads instead of holding 32 registers through the loop
  __shared__ __attribute__((aligned(16))) float s_scale[BM];
  __shared__ __attribute__((aligned(16))) float s_shift[BM];
  for (int c = tid; c < BM; c += W8_NT) {
    const bool ok = m0 + c < a.Cout;
    s_scale[c] = ok ? a.scale[m0 + c] : 0.f;
    s_shift[c] = ok ? a.shift[m0 + c] : 0.f;
  }
  // e4m3 output: bfloat16 bits of 448 * out_step in both halves (exact)
  uint32_t lim = 0;
  if constexpr (YF8) {
    lim = __float_as_uint(448.f * a.out_step) >> 16;
    lim |= lim << 16;
  }

  // Store units: 4 channels of one pixel per lane (an 8-byte bfloat16 or a
  // 4-byte e4m3 store); the host stages only NHWC views whose pixel m starts
  // at m * pitch and whose bytes fit 32-bit offsets.
  constexpr int NU = TN * TM * 4;   // store units per tile and lane
  constexpr int NUC = NU / NC;      // of them drained per chunk
  static_assert(NU % NC == 0, "store units per chunk");
  auto epi_unit = [&](int u, const f32x16_t (&ap)[TM][TN], int k) {
    const int j = u / (TM * 4), i = (u / 4) % TM, g = u % 4;
    const int cl = wm * WTM + i * 32 + g * 8 + hq * 4;   // channel within the slice
    const int co = m0 + cl;
    const int m = (stream + k * streams) * W8_BN + wn * WTN + j * 32 + frag_row;
    const bool ok = k >= 0 && m < a.M && co < a.Cout;
    const f32x4_t sc = *reinterpret_cast<const f32x4_t*>(&s_scale[cl]);
    const f32x4_t sh = *reinterpret_cast<const f32x4_t*>(&s_shift[cl]);
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float t = ap[i][j][g * 4 + r] * sc[r] + sh[r];
      if (a.act == VRS_ACT_SILU) t = silu_fast(t);
      v[r] = t;
    }
    const uint32_t p01 = pack_bf16x2(v[0], v[1]), p23 = pack_bf16x2(v[2], v[3]);
    if constexpr (YF8) {
      const uint32_t off = ok ? (uint32_t)m * (uint32_t)a.y_sp + (uint32_t)co : kOOB;
      __builtin_amdgcn_raw_buffer_store_b32(bf16x2_to_fp8x2(p01, lim, a.out_step) |
                                                (bf16x2_to_fp8x2(p23, lim, a.out_step) << 16),
                                            ry, off, 0, 0);
    } else {
      const uint32_t off = ok ? ((uint32_t)m * (uint32_t)a.y_sp + (uint32_t)co) * 2u : kOOB;
      __builtin_amdgcn_raw_buffer_store_b64((u32x2_t){p01, p23}, ry, off, 0, 0);
    }
  };
  auto ld32 = [&](const unsigned char* p) {
    const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(p);
    const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(p + 16);
    return (i32x8_t){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };
  // chunk h of a tile (its first zeroes the accumulators); tile k-1's units
  // h*NUC .. (h+1)*NUC-1 drain between the k slices.  h is a compile-time
  // constant, so every unit index is one and the accumulators stay in
  // registers.
  auto compute = [&](const unsigned char* sB, auto hc, f32x16_t (&ac)[TM][TN], const f32x16_t (&ap)[TM][TN],
                     int k) __attribute__((always_inline)) {
    constexpr int h = decltype(hc)::value;
    if constexpr (h == 0) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) ac[i][j][r] = 0.f;
    }
    const unsigned char* pa = sW + (wm * WTM + frag_row) * LDW + h * KCH + hq * 32;
    const unsigned char* pb = sB + (wn * WTN + frag_row) * LDB + hq * 32;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      i32x8_t fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = ld32(pa + i * 32 * LDW + kk * 64);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = ld32(pb + j * 32 * LDB + kk * 64);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) ac[i][j] = mfma32_fp8_k64(fa[i], fb[j], ac[i][j]);
#pragma unroll
      for (int u = h * NUC + kk * NUC / KK; u < h * NUC + (kk + 1) * NUC / KK; ++u) epi_unit(u, ap, k - 1);
    }
  };

  // chunk c: LDS buffer c&1 holds it; register set (c+1)&1 holds chunk c+1
  // (written to the other buffer during chunk c); set c&1 receives chunk
  // c+2; accumulator set k&1 receives tile k = c / NC while set (k+1)&1
  // drains tile k-1
  u32x4_t r0[NCH], r1[NCH];
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
  // The LDS write of chunk c+1 goes after chunk c's MFMAs (its buffer was
  // last read by chunk c-1, before the previous barrier): its loads, issued
  // one step earlier, then have two steps of MFMAs to land instead of one
  // (an fp8 step is short next to the load latency).
  auto step = [&](const unsigned char* cur, unsigned char* nxt, u32x4_t (&ld)[NCH], const u32x4_t (&st)[NCH],
                  f32x16_t (&ac)[TM][TN], const f32x16_t (&ap)[TM][TN], int k, auto hc) __attribute__((always_inline)) {
    load_chunk(k * NC + decltype(hc)::value + 2, ld);
    compute(cur, hc, ac, ap, k);
    store_chunk(nxt, st);
    __syncthreads();
  };
  // one tile: chunk parity (k*NC + h) & 1 is h & 1 for even NC, k & 1 for NC 1
  auto tile = [&](auto odd_tag, f32x16_t (&ac)[TM][TN], const f32x16_t (&ap)[TM][TN], int k) {
    constexpr bool ODD = decltype(odd_tag)::value;
    w8_static_for<0, NC>([&](auto hc) {
      constexpr int h = decltype(hc)::value;
      constexpr int par = (NC == 1 ? (ODD ? 1 : 0) : h) & 1;
      if constexpr (par == 0) step(sB0, sB1, r0, r1, ac, ap, k, hc);
      else step(sB1, sB0, r1, r0, ac, ap, k, hc);
    });
  };
  for (int k = 0; k < nt; k += 2) {
    tile(std::false_type{}, acc0, acc1, k);
    if (k + 1 < nt) tile(std::true_type{}, acc1, acc0, k + 1);
  }
  // the last tile's epilogue
  if ((nt - 1) & 1) {
#pragma unroll
    for (int u = 0; u < NU; ++u) epi_unit(u, acc1, nt - 1);
  } else {
#pragma unroll
    for (int u = 0; u < NU; ++u) epi_unit(u, acc0, nt - 1);
  }
}

}  // namespace

// vrs_conv1w_fp8_128_c<Cin>[_x8][_y8]: LDS = 128 * (Cin + 16) + 2 * 128 *
// (Cin/NC + 16) bytes (Cin 768 in four 192-channel chunks: 153.6 KB).
#define VRS_CONV1W8(CIN, NC, TAG, XF8, YF8)                                                            \
  extern "C" __global__ __launch_bounds__(512) void vrs_conv1w_fp8_128_c##CIN##TAG(vrs_conv_args a) { \
    conv1w8_body<CIN, NC, XF8, YF8>(a);                                                                \
  }
// NC8 / NC16: chunks per tile with e4m3 / bfloat16 inputs (a bfloat16 piece
// carries half the channels, so its chunks are kept to 6 pieces per thread)
#define VRS_CONV1W8_IO(CIN, NC8, NC16)           \
  VRS_CONV1W8(CIN, NC16, , false, false)         \
  VRS_CONV1W8(CIN, NC8, _x8, true, false)        \
  VRS_CONV1W8(CIN, NC16, _y8, false, true)       \
  VRS_CONV1W8(CIN, NC8, _x8_y8, true, true)
VRS_CONV1W8_IO(128, 1, 1)
VRS_CONV1W8_IO(192, 1, 1)
VRS_CONV1W8_IO(256, 1, 2)
VRS_CONV1W8_IO(384, 2, 2)
VRS_CONV1W8_IO(512, 2, 4)
VRS_CONV1W8_IO(768, 4, 4)

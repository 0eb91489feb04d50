// Fused bottleneck pair for gfx950 (bfloat16): the 3x3 -> 3x3 (+ residual)
// of blocks/bottleneck.rs:37-63 (each conv blocks/conv.rs:31-46 with BN and
// SiLU) in one kernel, so the middle map never goes to memory and the block
// input is read once:
//   m = bf16(silu(s1 * conv3x3(x, w1) + b1))          (C -> CH channels)
//   y = bf16(silu(s2 * conv3x3(m, w2) + b2) + res)    (CH -> C channels)
//
// A workgroup owns a run of 256 output pixels -- R = 256/TW whole rows of a
// vertical strip TW pixels wide -- and all C output channels:
//   * cv1 runs on the (R+2) x (TW+2) middle-map positions the run's 3x3
//     windows read (one pixel of halo, recomputed by the neighbouring runs),
//     from the (R+4) x (TW+4) input positions staged in LDS 16 channels at a
//     time with the chunk's weights for all nine taps (two stages, two
//     register sets, one barrier per chunk, as the halo kernel conv3.hip);
//     middle-map positions outside the image are zero (cv2's padding);
//   * the middle map stays in LDS as bfloat16 (rows of CH + 8 elements: the
//     16 positions a quarter-wave reads start on distinct 4-bank groups), the
//     cv2 weights (all taps, loaded during cv1's last two chunks) replace the
//     cv1 stages, and cv2's MFMAs read both from LDS with no further barrier;
//   * the cv2 epilogue (BN, SiLU, the residual prefetched before the cv1
//     loop) is staged through LDS for 16-byte NHWC stores.
// Both convs take their K steps in the halo kernel's order (16-channel chunk
// outer, tap inner) and round like it, so the outputs equal the two halo
// kernel launches bit for bit.  4 waves: cv1 position tiles of 32 dealt
// round-robin over the waves, cv2 wave tile C channels x 64 pixels, all on
// v_mfma_f32_32x32x16_bf16.
#include "common.h"

namespace {

constexpr int bp_max(int a, int b) { return a > b ? a : b; }

// element offset of 16-byte half `half` of staged input position `pos` (16
// channels per position; the halves of every other group of 8 positions
// swapped: 16 consecutive positions cover the 64 banks once)
__device__ __forceinline__ int bp_swz(int pos, int half) { return pos * 16 + ((half ^ ((pos >> 3) & 1)) << 3); }

template <int C, int CH, int TW>
__device__ __forceinline__ void bpair_body(const vrs_bpair_args& a) {
  using E = Elt<bf16_t>;
  using G = E::group;
  constexpr int NT = 256;
  constexpr int R = 256 / TW;                       // output rows per run
  static_assert(R * TW == 256, "a run is whole rows of the strip");
  constexpr int MW = TW + 2, MH = R + 2, NMP = MW * MH;   // middle-map positions
  constexpr int XW = TW + 4, XH = R + 4, NXP = XW * XH;   // input positions
  constexpr int NMT = (NMP + 31) / 32;              // cv1 position tiles
  constexpr int MTW = (NMT + 3) / 4;                // of them per wave
  constexpr int TM1 = CH / 32;                      // cv1 MFMA row blocks
  constexpr int TM2 = C / 32, TN2 = 2;              // cv2 wave tile C x 64 pixels
  constexpr int NCH1 = C / 16, NCH2 = CH / 16;      // 16-channel chunks of cv1 / cv2 inputs
  static_assert(C % 32 == 0 && CH % 32 == 0 && NCH1 >= 2, "channels");
  constexpr int W1ROW = 9 * 16 + 8;                 // cv1 weights of one chunk: 9 taps x 16 + 16-byte pad
  constexpr int SW1 = CH * W1ROW, SX = NXP * 16, STAGE1 = SW1 + SX;
  constexpr int W2ROW = 9 * CH + 8, SW2 = C * W2ROW;   // cv2 weights: [co][tap][CH] + pad
  constexpr int MROW = CH + 8, SM = NMP * MROW;
  constexpr int SROW = C + 8, SST = 4 * 64 * SROW;     // epilogue staging
  constexpr int AREA = bp_max(bp_max(2 * STAGE1, SW2), SST);
  __shared__ __attribute__((aligned(16))) bf16_t smem[AREA + SM];
  __shared__ __attribute__((aligned(16))) float cst[2 * CH + 2 * C];   // s1 | b1 | s2 | b2
  bf16_t* const sM = smem + AREA;
  constexpr int WI1 = (CH * 18 + NT - 1) / NT;      // cv1 weight pieces per thread (rows x 9 taps x 2 halves)
  constexpr int XI = (NXP * 2 + NT - 1) / NT;       // input pieces per thread
  constexpr int W2P = 9 * CH / 8;                   // 16-byte pieces per cv2 weight row
  constexpr int WI2 = C * W2P / NT;                 // cv2 weight pieces per thread
  static_assert(C * W2P % NT == 0, "whole cv2 weight pieces");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hq = lane >> 5;
  // runs of one strip are neighbouring logical blocks (one XCD: the rows
  // two runs share come from that XCD's L2)
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int run = logical % a.runs;
  const int rest = logical / a.runs;
  const int strip = rest % a.strips;
  const int b = rest / a.strips;
  const int y0 = run * R, x0 = strip * TW;

  for (int c = tid; c < 2 * CH + 2 * C; c += NT)
    cst[c] = c < CH ? a.s1[c] : c < 2 * CH ? a.b1[c - CH] : c < 2 * CH + C ? a.s2[c - 2 * CH] : a.b2[c - 2 * CH - C];

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t rw1 = make_rsrc(a.w1, a.w1_bytes);
  const __amdgpu_buffer_rsrc_t rw2 = make_rsrc(a.w2, a.w2_bytes);
  const uint32_t xrow = (uint32_t)a.x_pitch * 2u;

  // this thread's staging items (fixed over the chunks; the chunk moves the
  // channel offset): cv1 weight piece -> (row, tap, half), input piece ->
  // (position, half); positions outside the image read zeros
  uint32_t w_off[WI1], x_off[XI];
  int w_lds[WI1], x_lds[XI];
#pragma unroll
  for (int i = 0; i < WI1; ++i) {
    const int it = tid + i * NT;
    const int row = it / 18, r18 = it % 18, tap = r18 >> 1, g = r18 & 1;
    const bool ok = it < CH * 18;
    w_off[i] = ok ? (uint32_t)(((row * 9 + tap) * C + g * 8) * 2) : kOOB;
    w_lds[i] = ok ? row * W1ROW + tap * 16 + g * 8 : -1;
  }
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int it = tid + i * NT;
    const int pos = it >> 1, g = it & 1;
    const int hr = pos / XW, hc = pos - hr * XW;
    const int yy = y0 - 2 + hr, xx = x0 - 2 + hc;
    const bool ok = pos < NXP && (unsigned)yy < (unsigned)a.H && (unsigned)xx < (unsigned)a.W;
    x_off[i] = ok ? (uint32_t)((b * a.H + yy) * a.W + xx) * xrow + (uint32_t)(g * 16) : kOOB;
    x_lds[i] = pos < NXP ? bp_swz(pos, g) : -1;
  }
  auto load1 = [&](int c, u32x4_t (&wr)[WI1], u32x4_t (&xr)[XI]) {
    const uint32_t so = (uint32_t)(c * 32);   // 16 channels of bf16
#pragma unroll
    for (int i = 0; i < WI1; ++i) wr[i] = __builtin_amdgcn_raw_buffer_load_b128(rw1, w_off[i], so, 0);
#pragma unroll
    for (int i = 0; i < XI; ++i) xr[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, x_off[i], so, 0);
  };
  auto store1 = [&](int buf, const u32x4_t (&wr)[WI1], const u32x4_t (&xr)[XI]) {
    bf16_t* sW = smem + buf * STAGE1;
    bf16_t* sX = sW + SW1;
#pragma unroll
    for (int i = 0; i < WI1; ++i)
      if (w_lds[i] >= 0) *reinterpret_cast<u32x4_t*>(sW + w_lds[i]) = wr[i];
#pragma unroll
    for (int i = 0; i < XI; ++i)
      if (x_lds[i] >= 0) *reinterpret_cast<u32x4_t*>(sX + x_lds[i]) = xr[i];
  };
  // cv2 weights: piece q of the thread -> row q / W2P, 8 elements at (q % W2P) * 8
  u32x4_t w2r[WI2];
  auto load_w2 = [&]() {
#pragma unroll
    for (int i = 0; i < WI2; ++i) {
      const int q = tid + i * NT;
      w2r[i] = __builtin_amdgcn_raw_buffer_load_b128(rw2, (uint32_t)((q / W2P) * 9 * CH + (q % W2P) * 8) * 2u, 0, 0);
    }
  };

  // cv1: this lane's middle-map position in each of its tiles (tile wave +
  // 4t; positions past the map repeat the last one and are never stored)
  int pbase[MTW];   // input position of tap (0, 0): tap (ky, kx) adds ky*XW + kx
#pragma unroll
  for (int t = 0; t < MTW; ++t) {
    int p = (wave + 4 * t) * 32 + l32;
    p = p < NMP ? p : NMP - 1;
    const int pr = p / MW, pc = p - pr * MW;
    pbase[t] = pr * XW + pc;
  }
  f32x16_t acc1[TM1][MTW];
#pragma unroll
  for (int i = 0; i < TM1; ++i)
#pragma unroll
    for (int t = 0; t < MTW; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc1[i][t][r] = 0.f;
  auto compute1 = [&](int buf) {
    const bf16_t* sW = smem + buf * STAGE1;
    const bf16_t* sX = sW + SW1;
    G fa[2][TM1], fb[2][MTW];
    auto read_tap = [&](int tap, G (&ra)[TM1], G (&rb)[MTW]) {
      const int toff = (tap / 3) * XW + (tap % 3);
#pragma unroll
      for (int i = 0; i < TM1; ++i) ra[i] = E::load(sW + (i * 32 + l32) * W1ROW + tap * 16 + hq * 8);
#pragma unroll
      for (int t = 0; t < MTW; ++t) rb[t] = E::load(sX + bp_swz(pbase[t] + toff, hq));
    };
    read_tap(0, fa[0], fb[0]);
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      if (tap + 1 < 9) read_tap(tap + 1, fa[(tap + 1) & 1], fb[(tap + 1) & 1]);
#pragma unroll
      for (int i = 0; i < TM1; ++i)
#pragma unroll
        for (int t = 0; t < MTW; ++t) acc1[i][t] = mfma32_k16(fa[tap & 1][i], fb[tap & 1][t], acc1[i][t]);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, TM1 + MTW, 0);
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      if (tap + 1 < 9) __builtin_amdgcn_sched_group_barrier(0x100, TM1 + MTW, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, TM1 * MTW, 0);
    }
  };
  // chunk c: loads of chunk c+2 first (the cv2 weights instead, two chunks
  // before the end), then chunk c's MFMAs, then chunk c+1 (loaded during
  // chunk c-1) written to the other stage, one barrier
  auto step1 = [&](int c, u32x4_t (&wl)[WI1], u32x4_t (&xl)[XI], const u32x4_t (&ws)[WI1], const u32x4_t (&xs)[XI]) {
    if (c + 2 < NCH1) load1(c + 2, wl, xl);
    if (c == NCH1 - 2) load_w2();
    compute1(c & 1);
    if (c + 1 < NCH1) store1((c + 1) & 1, ws, xs);
    __syncthreads();
  };

  u32x4_t wa[WI1], xa[XI], wb[WI1], xb[XI];
  load1(0, wa, xa);
  load1(1, wb, xb);
  // the residual this lane adds (4 channels of each cv2 accumulator quad),
  // loaded now so its latency passes under the loops
  int oi[TN2], oj[TN2];
  bool ov[TN2];
#pragma unroll
  for (int j = 0; j < TN2; ++j) {
    const int o = wave * 64 + j * 32 + l32;
    oi[j] = o / TW;
    oj[j] = o - oi[j] * TW;
    ov[j] = y0 + oi[j] < a.H && x0 + oj[j] < a.W;
  }
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.res, a.res ? a.res_bytes : 0);
  u32x2_t rres[TM2][4][TN2];
#pragma unroll
  for (int i = 0; i < TM2; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int j = 0; j < TN2; ++j) {
        const int co = i * 32 + g * 8 + hq * 4;
        const uint32_t ro =
            a.res && ov[j]
                ? ((uint32_t)((b * a.H + y0 + oi[j]) * a.W + x0 + oj[j]) * (uint32_t)a.r_pitch + (uint32_t)co) * 2u
                : kOOB;
        rres[i][g][j] = __builtin_amdgcn_raw_buffer_load_b64(rr, ro, 0, 0);
      }
  store1(0, wa, xa);
  __syncthreads();
  for (int c = 0; c < NCH1; c += 2) {
    step1(c, wa, xa, wb, xb);
    if (c + 1 < NCH1) step1(c + 1, wb, xb, wa, xa);
  }

  // cv1 epilogue -> the middle map (zero outside the image), then the cv2
  // weights into the stage area (every wave is past the last chunk's barrier)
#pragma unroll
  for (int t = 0; t < MTW; ++t) {
    const int p = (wave + 4 * t) * 32 + l32;
    const int pr = p / MW, pc = p - pr * MW;
    const int yy = y0 - 1 + pr, xx = x0 - 1 + pc;
    const bool inside = p < NMP && (unsigned)yy < (unsigned)a.H && (unsigned)xx < (unsigned)a.W;
#pragma unroll
    for (int i = 0; i < TM1; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int cl = i * 32 + g * 8 + hq * 4;
        const f32x4_t sc = *reinterpret_cast<const f32x4_t*>(&cst[cl]);
        const f32x4_t sh = *reinterpret_cast<const f32x4_t*>(&cst[CH + cl]);
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = inside ? silu_fast(acc1[i][t][g * 4 + r] * sc[r] + sh[r]) : 0.f;
        if (p < NMP)
          *reinterpret_cast<u32x2_t*>(sM + p * MROW + cl) = (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      }
  }
#pragma unroll
  for (int i = 0; i < WI2; ++i) {
    const int q = tid + i * NT;
    *reinterpret_cast<u32x4_t*>(smem + (q / W2P) * W2ROW + (q % W2P) * 8) = w2r[i];
  }
  __syncthreads();

  // cv2 from LDS: 16-channel chunk of the middle map outer, tap inner
  int mbase[TN2];   // middle-map position of tap (0, 0) for this lane's output pixels
#pragma unroll
  for (int j = 0; j < TN2; ++j) mbase[j] = oi[j] * MW + oj[j];
  f32x16_t acc2[TM2][TN2];
#pragma unroll
  for (int i = 0; i < TM2; ++i)
#pragma unroll
    for (int j = 0; j < TN2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc2[i][j][r] = 0.f;
#pragma unroll
  for (int c2 = 0; c2 < NCH2; ++c2) {
    G fa[2][TM2], fb[2][TN2];
    auto read_tap = [&](int tap, G (&ra)[TM2], G (&rb)[TN2]) {
      const int toff = (tap / 3) * MW + (tap % 3);
#pragma unroll
      for (int i = 0; i < TM2; ++i) ra[i] = E::load(smem + (i * 32 + l32) * W2ROW + tap * CH + c2 * 16 + hq * 8);
#pragma unroll
      for (int j = 0; j < TN2; ++j) rb[j] = E::load(sM + (mbase[j] + toff) * MROW + c2 * 16 + hq * 8);
    };
    read_tap(0, fa[0], fb[0]);
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      if (tap + 1 < 9) read_tap(tap + 1, fa[(tap + 1) & 1], fb[(tap + 1) & 1]);
#pragma unroll
      for (int i = 0; i < TM2; ++i)
#pragma unroll
        for (int j = 0; j < TN2; ++j) acc2[i][j] = mfma32_k16(fa[tap & 1][i], fb[tap & 1][j], acc2[i][j]);
    }
  }
  __syncthreads();   // every wave is done with the cv2 weights: the staging reuses their LDS

  // cv2 epilogue: register g*4 + r of tile (i, j) is channel i*32 + g*8 +
  // hq*4 + r of pixel slot wave*64 + j*32 + l32
  bf16_t* stg = smem + wave * 64 * SROW;
#pragma unroll
  for (int i = 0; i < TM2; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int cl = i * 32 + g * 8 + hq * 4;
      const f32x4_t sc = *reinterpret_cast<const f32x4_t*>(&cst[2 * CH + cl]);
      const f32x4_t sh = *reinterpret_cast<const f32x4_t*>(&cst[2 * CH + C + cl]);
#pragma unroll
      for (int j = 0; j < TN2; ++j) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = silu_fast(acc2[i][j][g * 4 + r] * sc[r] + sh[r]);
        if (a.res) {
          const u32x2_t rv = rres[i][g][j];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            v[r] += __uint_as_float((r & 1) ? (rv[r >> 1] & 0xffff0000u) : (rv[r >> 1] << 16));
        }
        *reinterpret_cast<u32x2_t*>(stg + (j * 32 + l32) * SROW + cl) =
            (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      }
    }
  __builtin_amdgcn_wave_barrier();   // this wave reads back only its own staging
  constexpr int CPP = C / 8;         // 16-byte chunks per pixel
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y, a.y_bytes);
#pragma unroll
  for (int s = 0; s < CPP; ++s) {
    const int c = lane + 64 * s;
    const int pl = c / CPP, part = c % CPP;
    const int o = wave * 64 + pl;
    const int yy = y0 + o / TW, xx = x0 + o % TW;
    const uint32_t off = yy < a.H && xx < a.W
                             ? ((uint32_t)((b * a.H + yy) * a.W + xx) * (uint32_t)a.y_pitch + (uint32_t)(part * 8)) * 2u
                             : kOOB;
    __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const u32x4_t*>(stg + pl * SROW + part * 8), ry, off, 0, 0);
  }
}

}  // namespace

// vrs_bpair_bf16_c<C>_h<CH>_w<TW>: LDS = the larger of two cv1 stages, the
// cv2 weights and the staging, plus the middle map (C 64, CH 32, TW 32:
// 47 + 27 KB, two workgroups per CU).
extern "C" __global__ __launch_bounds__(256, 2) void vrs_bpair_bf16_c64_h32_w32(vrs_bpair_args a) {
  bpair_body<64, 32, 32>(a);
}

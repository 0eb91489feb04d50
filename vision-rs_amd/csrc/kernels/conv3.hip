// Halo-tiled 3x3 stride-1 Conv2d + folded BN (+SiLU) (+residual), bfloat16,
// for gfx950 (blocks/conv.rs:31-46 as the bottleneck convs of
// blocks/bottleneck.rs:37-63 and the Detect box branch use it).
//
// The implicit-GEMM kernels (conv.hip) stage one (pixels x 32 channels) B
// tile per filter tap, so every input pixel is fetched and written to LDS
// nine times.  Here a workgroup owns BM output channels x 256 output pixels
// -- a run of 256 consecutive pixels of one vertical strip of the image,
// TW pixels wide -- and per 16-channel chunk of the input stages
//   * the strip rows the run touches plus a one-pixel halo: at most
//     (256/TW + 3) x (TW + 2) positions x 16 channels, the two 16-byte
//     halves of a position swapped on every other group of 8 positions
//     (16 consecutive positions -- one 16-lane group of an operand read --
//     then cover the 64 banks once), and
//   * the chunk's weights for all nine taps (BM x 9 x 16, rows padded by
//     16 bytes),
// then runs the nine taps' MFMAs from LDS: the B fragment of tap (ky, kx)
// for output pixel (y, x) is halo position (y - y_first + ky) * (TW + 2) +
// x + kx.  Two LDS stages (~33 KB each, two workgroups per CU) and two
// register sets: chunk c+2's global loads are issued before chunk c's MFMAs
// and written to LDS after chunk c+1's, so loads have two chunks' MFMAs to
// land and each chunk costs one barrier.  4 waves, each BM channels x 64
// pixels (32x32x16 bf16 MFMAs).  The residual is loaded with the first two
// chunks (its latency passes under the K loop).  Epilogue as the
// implicit-GEMM kernels: scale*acc + shift, SiLU, residual, staged through
// LDS for 16-byte NHWC stores.
#include "common.h"

namespace {

constexpr int H3_NP = 256;                   // output pixels per workgroup
constexpr int H3_CK = 16;                    // input channels per stage
constexpr int H3_TW_MIN = 8, H3_TW_MAX = 40; // strip widths the host may choose
// halo positions: rows (256/TW + 3) x cols (TW + 2), largest over TW in [8, 40]
constexpr int h3_hpos_max() {
  int m = 0;
  for (int tw = H3_TW_MIN; tw <= H3_TW_MAX; ++tw) {
    const int v = ((H3_NP + tw - 1) / tw + 3) * (tw + 2);
    m = v > m ? v : m;
  }
  return m;
}
constexpr int H3_HPOS = h3_hpos_max();
constexpr int H3_WROW = 9 * H3_CK + 8;       // weight row (elements): 9 taps x 16 + 16-byte pad

// element offset of 16-byte half `half` of halo position `pos`
__device__ __forceinline__ int h3_swz(int pos, int half) { return pos * H3_CK + ((half ^ ((pos >> 3) & 1)) << 3); }

template <int BM>
__device__ __forceinline__ void conv3h_body(const vrs_conv_args& a) {
  using E = Elt<bf16_t>;
  using G = E::group;
  constexpr int NT = 256;
  constexpr int TM = BM / 32, TN = 2;        // wave tile BM x 64
  constexpr int SW_ELEMS = BM * H3_WROW, SH_ELEMS = H3_HPOS * H3_CK;
  constexpr int STAGE = SW_ELEMS + SH_ELEMS;  // one LDS stage (elements)
  constexpr int SROW = BM + 8;               // epilogue staging row (channels + pad)
  constexpr int ST_ELEMS = 4 * 64 * SROW;
  constexpr int MAIN = 2 * STAGE > ST_ELEMS ? 2 * STAGE : ST_ELEMS;
  __shared__ __attribute__((aligned(16))) bf16_t smem[MAIN];
  constexpr int WI = (BM * 18 + NT - 1) / NT;             // weight chunks per thread (9 taps x 2 halves)
  constexpr int HI = (H3_HPOS * 2 + NT - 1) / NT;         // halo chunks per thread
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hq = lane >> 5;
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int tile_m = logical % a.tiles_m;
  int rest = logical / a.tiles_m;
  const int chunk = rest % a.h3_chunks;
  rest /= a.h3_chunks;
  const int strip = rest % a.h3_strips;
  const int b = rest / a.h3_strips;
  const int m0 = tile_m * BM;
  const int TW = a.h3_tw, HCW = TW + 2;
  const int x0 = strip * TW;                 // first image column of the strip
  const int q0 = chunk * H3_NP;              // first pixel of the run within the strip
  const int y_first = q0 / TW - 1;           // first halo row (image row)
  const int hrows = (q0 + H3_NP - 1) / TW - q0 / TW + 3;
  const int hpos = hrows * HCW;              // <= H3_HPOS (host: TW in [8, 40])

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w, a.w_bytes);
  const uint32_t xrow = (uint32_t)a.x_pitch * 2u;   // bytes per input pixel
  // folded-BN constants of the BM channels, in LDS for the epilogue (visible
  // after the first stage's barrier): one 16-byte read per channel quad
  __shared__ __attribute__((aligned(16))) float s_scale[BM];
  __shared__ __attribute__((aligned(16))) float s_shift[BM];
  for (int c = tid; c < BM; c += NT) {
    const bool ok = m0 + c < a.Cout;
    s_scale[c] = ok ? a.scale[m0 + c] : 0.f;
    s_shift[c] = ok ? a.shift[m0 + c] : 0.f;
  }

  // this thread's staging items (fixed over the chunks; the channel offset
  // moves): weight chunk -> (row, tap, 8-channel group); halo chunk ->
  // (position, 8-channel group)
  uint32_t w_off[WI], h_off[HI];
  int w_lds[WI], h_lds[HI];
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    const int it = tid + i * NT;
    const int row = it / 18, r18 = it % 18, tap = r18 >> 1, g = r18 & 1;
    const int co = m0 + row;
    const bool ok = it < BM * 18 && co < a.Cout;
    w_off[i] = ok ? (uint32_t)(((co * 9 + tap) * a.Cin + g * 8) * 2) : kOOB;
    w_lds[i] = it < BM * 18 ? row * H3_WROW + tap * H3_CK + g * 8 : -1;
  }
#pragma unroll
  for (int i = 0; i < HI; ++i) {
    const int it = tid + i * NT;
    const int pos = it >> 1, g = it & 1;
    const int hr = pos / HCW, hc = pos - hr * HCW;
    const int yy = y_first + hr, xx = x0 - 1 + hc;
    const bool ok = pos < hpos && (unsigned)yy < (unsigned)a.H && (unsigned)xx < (unsigned)a.W;
    h_off[i] = ok ? (uint32_t)((b * a.H + yy) * a.W + xx) * xrow + (uint32_t)(g * 16) : kOOB;
    h_lds[i] = pos < hpos ? h3_swz(pos, g) : -1;
  }
  // chunk c lives in register set c & 1 between its loads and its LDS write,
  // and in LDS stage c & 1 while its MFMAs run
  u32x4_t wreg0[WI], hreg0[HI], wreg1[WI], hreg1[HI];
  auto load_stage = [&](int c, u32x4_t (&wr)[WI], u32x4_t (&hr)[HI]) {
    const uint32_t ci0 = (uint32_t)(c * H3_CK * 2);
#pragma unroll
    for (int i = 0; i < WI; ++i) wr[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_off[i], ci0, 0);
#pragma unroll
    for (int i = 0; i < HI; ++i) hr[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, h_off[i], ci0, 0);
  };
  auto store_stage = [&](int buf, const u32x4_t (&wr)[WI], const u32x4_t (&hr)[HI]) {
    bf16_t* sW = smem + buf * STAGE;
    bf16_t* sH = sW + SW_ELEMS;
#pragma unroll
    for (int i = 0; i < WI; ++i)
      if (w_lds[i] >= 0) *reinterpret_cast<u32x4_t*>(sW + w_lds[i]) = wr[i];
#pragma unroll
    for (int i = 0; i < HI; ++i)
      if (h_lds[i] >= 0) *reinterpret_cast<u32x4_t*>(sH + h_lds[i]) = hr[i];
  };

  // this lane's output pixels (B fragment columns): slot wave*64 + j*32 + l32
  int hbase[TN];   // halo position of tap (0, 0)
  bool pv[TN];
  int py[TN], px[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int q = q0 + wave * 64 + j * 32 + l32;
    const int yy = q / TW, xl = q - yy * TW;
    py[j] = yy;
    px[j] = x0 + xl;
    pv[j] = yy < a.H && x0 + xl < a.W;
    hbase[j] = (yy - y_first - 1) * HCW + xl;   // tap (ky, kx) adds ky*HCW + kx
  }

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nst = a.Cin / H3_CK;   // >= 2 (host: Cin % 32 == 0)
  // one tap's operands are read while the previous tap's MFMAs run (two
  // fragment register sets, the order pinned with scheduling groups)
  auto compute = [&](int buf) {
    const bf16_t* sW = smem + buf * STAGE;
    const bf16_t* sH = sW + SW_ELEMS;
    G fa[2][TM], fb[2][TN];
    auto read_tap = [&](int tap, G (&ra)[TM], G (&rb)[TN]) {
      const int toff = (tap / 3) * HCW + (tap % 3);
#pragma unroll
      for (int i = 0; i < TM; ++i) ra[i] = E::load(sW + (i * 32 + l32) * H3_WROW + tap * H3_CK + hq * 8);
#pragma unroll
      for (int j = 0; j < TN; ++j) rb[j] = E::load(sH + h3_swz(hbase[j] + toff, hq));
    };
    read_tap(0, fa[0], fb[0]);
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      if (tap + 1 < 9) read_tap(tap + 1, fa[(tap + 1) & 1], fb[(tap + 1) & 1]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32_k16(fa[tap & 1][i], fb[tap & 1][j], acc[i][j]);
    }
    // schedule: tap 0's reads, then per tap the next tap's reads ahead of
    // this tap's MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      if (tap + 1 < 9) __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, TM * TN, 0);
    }
  };
  // chunk c: loads of chunk c+2 go out first, then chunk c's MFMAs, then
  // chunk c+1 (loaded during chunk c-1) is written to the other stage -- it
  // was last read by chunk c-1, before the previous barrier -- and one
  // barrier publishes it
  auto step = [&](int c, u32x4_t (&wl)[WI], u32x4_t (&hl)[HI], const u32x4_t (&ws)[WI], const u32x4_t (&hs)[HI]) {
    if (c + 2 < nst) load_stage(c + 2, wl, hl);
    compute(c & 1);
    if (c + 1 < nst) store_stage((c + 1) & 1, ws, hs);
    __syncthreads();
  };
  load_stage(0, wreg0, hreg0);
  load_stage(1, wreg1, hreg1);
  // the residual this lane adds (4 channels of each accumulator quad), loaded
  // now so that its latency passes under the K loop instead of the epilogue
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.res, a.res ? a.res_bytes : 0);
  u32x2_t rres[TM][4][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int co = m0 + i * 32 + g * 8 + hq * 4;
        const uint32_t ro = a.res && pv[j] && co < a.Cout
                                ? (uint32_t)((b * a.r_sb + (int64_t)py[j] * a.Wo * a.r_sp + (int64_t)px[j] * a.r_sp + co) * 2)
                                : kOOB;
        rres[i][g][j] = __builtin_amdgcn_raw_buffer_load_b64(rr, ro, 0, 0);
      }
  store_stage(0, wreg0, hreg0);
  __syncthreads();
  for (int c = 0; c < nst; c += 2) {
    step(c, wreg0, hreg0, wreg1, hreg1);
    if (c + 1 < nst) step(c + 1, wreg1, hreg1, wreg0, hreg0);
  }

  // epilogue: register g*4 + r of tile (i, j) is channel m0 + i*32 + g*8 +
  // hq*4 + r of pixel slot wave*64 + j*32 + l32
  // (the last chunk's barrier: every wave is done with the stage buffers,
  // which the staging reuses)
  bf16_t* stg = smem + wave * 64 * SROW;
  // instantiated per activation: no per-value SiLU select
  auto epilogue = [&](auto silu_on) {
    constexpr bool SILU = decltype(silu_on)::value;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int cl = i * 32 + g * 8 + hq * 4;
        const f32x4_t sc = *reinterpret_cast<const f32x4_t*>(&s_scale[cl]);
        const f32x4_t sh = *reinterpret_cast<const f32x4_t*>(&s_shift[cl]);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float t = acc[i][j][g * 4 + r] * sc[r] + sh[r];
            if constexpr (SILU) t = silu_fast(t);
            v[r] = t;
          }
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
  };
  if (a.act == VRS_ACT_SILU) epilogue(std::true_type{});
  else epilogue(std::false_type{});
  __builtin_amdgcn_wave_barrier();   // this wave reads back only its own staging
  // 16-byte raw-buffer stores at 32-bit offsets (the host bounds the view by
  // y_bytes < 2^31); the pixel's row in the strip by float-reciprocal divmod
  constexpr int CPP = BM / 8;        // 16-byte chunks per pixel
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y, a.y_bytes);
  const float inv_tw = 1.0f / (float)TW;
#pragma unroll
  for (int s = 0; s < CPP; ++s) {
    const int c = lane + 64 * s;
    const int pl = c / CPP, part = c % CPP;
    int xl;
    const int yy = fdivmod(q0 + wave * 64 + pl, TW, inv_tw, xl);
    const int xx = x0 + xl;
    const int co = m0 + part * 8;
    const uint32_t off = yy < a.H && xx < a.W && co < a.Cout
                             ? ((uint32_t)b * (uint32_t)a.y_sb + (uint32_t)(yy * a.Wo + xx) * (uint32_t)a.y_sp +
                                (uint32_t)co) * 2u
                             : kOOB;
    __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const u32x4_t*>(stg + pl * SROW + part * 8), ry, off, 0,
                                           0);
  }
}

}  // namespace

// Two workgroups per CU (~65 KB LDS each).
extern "C" __global__ __launch_bounds__(256, 2) void vrs_conv3h_bf16_64(vrs_conv_args a) { conv3h_body<64>(a); }
extern "C" __global__ __launch_bounds__(256, 2) void vrs_conv3h_bf16_32(vrs_conv_args a) { conv3h_body<32>(a); }

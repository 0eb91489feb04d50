// Halo-tiled 3x3 stride-1 Conv2d + folded BN (+SiLU) (+residual), bfloat16,
// for gfx950 (blocks/conv.rs:31-46 as the bottleneck convs of
// blocks/bottleneck.rs:37-63 and the Detect box branch use it).
//
// The implicit-GEMM kernels (conv.hip) stage one (pixels x 32 channels) B
// tile per filter tap, so every input pixel is fetched and written to LDS
// nine times.  Here a workgroup owns BM output channels x 256 output pixels
// -- a run of 256 consecutive pixels of one vertical strip of the image,
// TW pixels wide -- and per 32-channel chunk of the input stages
//   * the strip rows the run touches plus a one-pixel halo: at most
//     (256/TW + 3) x (TW + 2) positions x 32 channels, 16-byte chunks
//     XOR-swizzled by position (conflict-free 16-byte fragment reads), and
//   * the chunk's weights for all nine taps (BM x 9 x 32, rows padded by
//     16 bytes),
// then runs all nine taps x two 16-deep k slices from LDS: the B fragment of
// tap (ky, kx) for output pixel (y, x) is halo position (y - y_first + ky) *
// (TW + 2) + x + kx.  One LDS stage per chunk (~65 KB, two workgroups per CU);
// the next chunk's global loads are in flight during the MFMAs.  4 waves, each
// BM channels x 64 pixels (32x32x16 bf16 MFMAs).  Epilogue as the implicit-GEMM
// kernels: scale*acc + shift, SiLU, residual, staged through LDS for 16-byte
// NHWC stores.
#include "common.h"

namespace {

constexpr int H3_NP = 256;                   // output pixels per workgroup
constexpr int H3_CK = 32;                    // input channels per stage
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
constexpr int H3_WROW = 9 * H3_CK + 8;       // weight row (elements): 9 taps x 32 + 16-byte pad

__device__ __forceinline__ int h3_swz(int pos, int chunk) { return pos * H3_CK + ((chunk ^ ((pos >> 2) & 3)) << 3); }

template <int BM>
__device__ __forceinline__ void conv3h_body(const vrs_conv_args& a) {
  using E = Elt<bf16_t>;
  using G = E::group;
  constexpr int NT = 256;
  constexpr int TM = BM / 32, TN = 2;        // wave tile BM x 64
  constexpr int SW_ELEMS = BM * H3_WROW, SH_ELEMS = H3_HPOS * H3_CK;
  constexpr int SROW = BM + 8;               // epilogue staging row (channels + pad)
  constexpr int ST_ELEMS = 4 * 64 * SROW;
  constexpr int MAIN = SW_ELEMS + SH_ELEMS > ST_ELEMS ? SW_ELEMS + SH_ELEMS : ST_ELEMS;
  __shared__ __attribute__((aligned(16))) bf16_t smem[MAIN];
  bf16_t* sW = smem;
  bf16_t* sH = smem + SW_ELEMS;
  constexpr int WI = (BM * 9 * 4 + NT - 1) / NT;          // weight chunks per thread
  constexpr int HI = (H3_HPOS * 4 + NT - 1) / NT;         // halo chunks per thread

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
    const int row = it / 36, r36 = it % 36, tap = r36 >> 2, g = r36 & 3;
    const int co = m0 + row;
    const bool ok = it < BM * 36 && co < a.Cout;
    w_off[i] = ok ? (uint32_t)(((co * 9 + tap) * a.Cin + g * 8) * 2) : kOOB;
    w_lds[i] = it < BM * 36 ? row * H3_WROW + tap * H3_CK + g * 8 : -1;
  }
#pragma unroll
  for (int i = 0; i < HI; ++i) {
    const int it = tid + i * NT;
    const int pos = it >> 2, g = it & 3;
    const int hr = pos / HCW, hc = pos - hr * HCW;
    const int yy = y_first + hr, xx = x0 - 1 + hc;
    const bool ok = pos < hpos && (unsigned)yy < (unsigned)a.H && (unsigned)xx < (unsigned)a.W;
    h_off[i] = ok ? (uint32_t)((b * a.H + yy) * a.W + xx) * xrow + (uint32_t)(g * 16) : kOOB;
    h_lds[i] = pos < hpos ? h3_swz(pos, g) : -1;
  }
  u32x4_t wreg[WI], hreg[HI];
  auto load_stage = [&](int ci0) {
#pragma unroll
    for (int i = 0; i < WI; ++i) wreg[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_off[i], ci0 * 2, 0);
#pragma unroll
    for (int i = 0; i < HI; ++i) hreg[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, h_off[i], ci0 * 2, 0);
  };
  auto store_stage = [&]() {
#pragma unroll
    for (int i = 0; i < WI; ++i)
      if (w_lds[i] >= 0) *reinterpret_cast<u32x4_t*>(sW + w_lds[i]) = wreg[i];
#pragma unroll
    for (int i = 0; i < HI; ++i)
      if (h_lds[i] >= 0) *reinterpret_cast<u32x4_t*>(sH + h_lds[i]) = hreg[i];
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

  const int nst = a.Cin / H3_CK;
  load_stage(0);
  for (int st = 0; st < nst; ++st) {
    if (st > 0) __syncthreads();   // the previous chunk's fragments have been read
    store_stage();
    __syncthreads();
    if (st + 1 < nst) load_stage((st + 1) * H3_CK);   // in flight during the MFMAs
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      const int toff = (tap / 3) * HCW + (tap % 3);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        G fa[TM], fb[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
          fa[i] = E::load(sW + (i * 32 + l32) * H3_WROW + tap * H3_CK + kk * 16 + hq * 8);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[j] = E::load(sH + h3_swz(hbase[j] + toff, kk * 2 + hq));
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma32_k16(fa[i], fb[j], acc[i][j]);
      }
    }
  }

  // epilogue: register g*4 + r of tile (i, j) is channel m0 + i*32 + g*8 +
  // hq*4 + r of pixel slot wave*64 + j*32 + l32
  __syncthreads();   // every wave is done with the stage buffers (reused for staging)
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.res, a.res ? a.res_bytes : 0);
  bf16_t* stg = smem + wave * 64 * SROW;
  // instantiated per activation: no per-value SiLU select
  auto epilogue = [&](auto silu_on) {
    constexpr bool SILU = decltype(silu_on)::value;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int cl = i * 32 + g * 8 + hq * 4;
        const int co = m0 + cl;
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
            const uint32_t ro = pv[j] && co < a.Cout
                                    ? (uint32_t)((b * a.r_sb + (int64_t)py[j] * a.Wo * a.r_sp + (int64_t)px[j] * a.r_sp +
                                                  co) * 2)
                                    : kOOB;
            const u32x2_t rv = __builtin_amdgcn_raw_buffer_load_b64(rr, ro, 0, 0);
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
  constexpr int CPP = BM / 8;        // 16-byte chunks per pixel
  for (int c = lane; c < 64 * CPP; c += 64) {
    const int pl = c / CPP, part = c % CPP;
    const int q = q0 + wave * 64 + pl;
    const int yy = q / TW, xx = x0 + (q - yy * TW);
    const int co = m0 + part * 8;
    if (yy >= a.H || xx >= a.W || co >= a.Cout) continue;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(stg + pl * SROW + part * 8);
    *reinterpret_cast<u32x4_t*>(reinterpret_cast<bf16_t*>(a.y) + b * a.y_sb + ((int64_t)yy * a.Wo + xx) * a.y_sp + co) = v;
  }
}

}  // namespace

// Two workgroups per CU (~65 KB LDS each).
extern "C" __global__ __launch_bounds__(256, 2) void vrs_conv3h_bf16_64(vrs_conv_args a) { conv3h_body<64>(a); }
extern "C" __global__ __launch_bounds__(256, 2) void vrs_conv3h_bf16_32(vrs_conv_args a) { conv3h_body<32>(a); }

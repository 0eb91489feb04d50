// Implicit-GEMM Conv2d + folded BatchNorm + SiLU (+ residual) for gfx950: the
// bf16 and float32 kernels (the shared body is in conv_body.h; the fp8
// kernels are in conv8.hip), the persistent variant, the layout
// conversions and the stem.
#include "conv_body.h"

namespace {

// Persistent variant for the memory-bound shapes (bf16, Cin % BK == 0, even
// K-step count, no residual, staged 16-byte stores).  A workgroup takes tiles
// xcd_remap(blockIdx.x) + i*gridDim.x and runs one continuous load stream
// over its (tile, K step) sequence: the two steps in flight at the end of a
// tile are the next tile's first two, so the epilogue -- which stages through
// its own LDS area, not the pipeline buffers -- runs while they land.  Stores
// are raw buffer stores with a fixed count per lane (out-of-range chunks use
// out-of-range offsets), so waiting for the next loads never waits for them.
// DIRECT (the 8-wave 256x256 tile, whose two pipeline stages leave no LDS
// for a staging area): the epilogue stores each lane's 4 channels of a pixel
// as one 8-byte raw-buffer store straight from the accumulators.
template <int BM, int BN, int BK, int WGM, int WGN, bool DIRECT = false>
__device__ __forceinline__ void conv_persist_body(const vrs_conv_args& a) {
  using T = bf16_t;
  using E = Elt<T>;
  using G = E::group;
  constexpr bool SWZ = BK == 32;                        // same LDS layout as conv_body
  constexpr int PAD = 8, LDK = BK + (SWZ ? 0 : PAD), GPR = BK / 8;
  constexpr int NT = 64 * WGM * WGN;
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int A_IT = BM * GPR / NT, B_IT = BN * GPR / NT;
  static_assert(BM * GPR % NT == 0 && BN * GPR % NT == 0, "whole chunks per thread");
  constexpr int TILE_ELEMS = (BM + BN) * LDK;
  constexpr int SPAD = 8, SROW = WTM + SPAD;           // staging row: WTM channels + pad
  constexpr int EPC = 8, CPP = WTM / EPC;               // 16-byte chunks per staged pixel
  constexpr int NST = WTN * CPP / 64;                   // stores per lane per tile
  static_assert(WTN * CPP % 64 == 0, "whole store rounds");
  __shared__ __attribute__((aligned(16))) T smem0[TILE_ELEMS];
  __shared__ __attribute__((aligned(16))) T smem1[TILE_ELEMS];
  __shared__ __attribute__((aligned(16))) T sstage[DIRECT ? 8 : WGM * WGN * WTN * SROW];
  auto sbuf = [&](int b) -> T* { return b ? smem1 : smem0; };
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  static_assert(!SWZ || (NT / GPR) % 4 == 0, "swizzle period");
  const int st_row = tid / GPR, st_chunk = tid % GPR;
  const int st_off = st_row * LDK + (SWZ ? st_chunk ^ ((st_row >> 2) & 3) : st_chunk) * 8;
  const int wm = wave / WGN, wn = wave % WGN, hq = lane >> 5;
  const int HWo = a.Ho * a.Wo;
  const float inv_hwo = 1.0f / (float)HWo, inv_wo = 1.0f / (float)a.Wo;
  const int total = a.tiles_m * a.tiles_n;
  const int nk = a.K / BK;                              // even, >= 2 (host)
  int tile = xcd_remap(blockIdx.x, gridDim.x);
  if (tile >= total) return;

  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w, a.w_bytes);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y, a.y_bytes);

  // load stream state: tile being loaded, its next K step, chunk geometry
  int ld_tile = tile, ld_k = 0, t_ky = 0, t_kx = 0, t_ci = 0;
  uint32_t a_off[A_IT], b_off[B_IT];
  int b_iy0[B_IT], b_ix0[B_IT];
  bool b_ok[B_IT];
  auto geometry = [&](int t) {
    const int m0 = (t % a.tiles_m) * BM, n0 = (t / a.tiles_m) * BN;
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
      const int c = tid + i * NT, co = m0 + c / GPR;
      a_off[i] = co < a.Cout ? (uint32_t)((co * a.K + (c % GPR) * 8) * 2) : kOOB;
    }
#pragma unroll
    for (int i = 0; i < B_IT; ++i) {
      const int c = tid + i * NT, m = n0 + c / GPR;
      b_ok[i] = m < a.M;
      int rr, ox;
      const int bb = fdivmod(b_ok[i] ? m : 0, HWo, inv_hwo, rr);
      const int oy = fdivmod(rr, a.Wo, inv_wo, ox);
      b_iy0[i] = oy * a.stride - a.pad;
      b_ix0[i] = ox * a.stride - a.pad;
      b_off[i] = (uint32_t)((((int64_t)bb * a.H + b_iy0[i]) * a.W + b_ix0[i]) * a.x_pitch + (c % GPR) * 8) * 2u;
    }
  };
  geometry(ld_tile);
  auto load_set = [&](G (&ra)[A_IT], G (&rb)[B_IT]) {
    if (ld_k == nk) {   // the stream moves on to the next tile
      ld_tile += gridDim.x;
      ld_k = 0;
      t_ky = t_kx = t_ci = 0;
      if (ld_tile < total) geometry(ld_tile);
    }
    const uint32_t dead = ld_tile < total ? 0u : kOOB;
#pragma unroll
    for (int i = 0; i < A_IT; ++i)
      ra[i] = E::bload(rw, a_off[i] | dead, (uint32_t)((t_ky * a.kw + t_kx) * a.Cin + t_ci) * 2u);
    const int ky = t_ky, kx = t_kx;
    const uint32_t off = (uint32_t)((ky * a.W + kx) * a.x_pitch + t_ci) * 2u;
    if (++t_kx == a.kw) {
      t_kx = 0;
      if (++t_ky == a.kh) { t_ky = 0; t_ci += BK; }
    }
#pragma unroll
    for (int i = 0; i < B_IT; ++i) {
      const int iy = b_iy0[i] + ky, ix = b_ix0[i] + kx;
      const bool ok = b_ok[i] && (unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W;
      rb[i] = E::bload(rx, (ok ? b_off[i] + off : kOOB) | dead, 0);
    }
    ++ld_k;
  };
  auto store_set = [&](int buf, const G (&ra)[A_IT], const G (&rb)[B_IT]) {
    T* sA = sbuf(buf);
    T* sB = sA + BM * LDK;
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
      const int c = tid + i * NT;
      E::store(&sA[st_off + i * (NT / GPR) * LDK], ra[i]);
    }
#pragma unroll
    for (int i = 0; i < B_IT; ++i) {
      const int c = tid + i * NT;
      E::store(&sB[st_off + i * (NT / GPR) * LDK], rb[i]);
    }
  };

  f32x16_t acc[TM][TN];
  const int frag_row = lane & 31;
  const int frag_swz = SWZ ? (frag_row >> 2) & 3 : 0;
  auto frag_off = [&](int kk) { return ((kk * 2 + hq) ^ frag_swz) * 8; };
  auto step = [&](int cur, const G (&wa)[A_IT], const G (&wb)[B_IT], G (&la)[A_IT], G (&lb)[B_IT]) {
    load_set(la, lb);
    store_set(cur ^ 1, wa, wb);
    const T* sA = sbuf(cur);
    const T* sB = sA + BM * LDK;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      G fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = E::load(&sA[(wm * WTM + i * 32 + frag_row) * LDK + frag_off(kk)]);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = E::load(&sB[(wn * WTN + j * 32 + frag_row) * LDK + frag_off(kk)]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32_k16(fa[i], fb[j], acc[i][j]);
    }
    pipe_schedule<BK / 16 * TM * TN, TM + TN, TM * TN, A_IT + B_IT>();
    __syncthreads();
  };

  G ra0[A_IT], rb0[B_IT], ra1[A_IT], rb1[B_IT];
  load_set(ra0, rb0);
  load_set(ra1, rb1);
  store_set(0, ra0, rb0);
  __syncthreads();
  const ChanConst c_scale(a.scale, a.Cout), c_shift(a.shift, a.Cout);
  const uint32_t hmask = upper_half_mask();
  T* st = sstage + wave * WTN * SROW;
  for (; tile < total; tile += gridDim.x) {
    const int m0 = (tile % a.tiles_m) * BM, n0 = (tile / a.tiles_m) * BN;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    for (int kt = 0; kt < nk; kt += 2) {
      step(0, ra1, rb1, ra0, rb0);
      step(1, ra0, rb0, ra1, rb1);
    }
    if constexpr (DIRECT) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float sc[4], sh[4];
          c_scale.quad(m0 + wm * WTM + i * 32 + g * 8, hmask, sc);
          c_shift.quad(m0 + wm * WTM + i * 32 + g * 8, hmask, sh);
          const int co = m0 + wm * WTM + i * 32 + g * 8 + hq * 4;
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float t = acc[i][j][g * 4 + r] * sc[r] + sh[r];
              if (a.act == VRS_ACT_SILU) t = silu_fast(t);
              v[r] = t;
            }
            const int m = n0 + wn * WTN + j * 32 + (lane & 31);
            const uint32_t off = m < a.M && co < a.Cout ? ((uint32_t)m * (uint32_t)a.y_sp + (uint32_t)co) * 2u : kOOB;
            __builtin_amdgcn_raw_buffer_store_b64((u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])}, ry,
                                                  off, 0, 0);
          }
        }
      continue;
    }
    // epilogue: this wave's (WTN pixel x WTM channel) tile -> its staging
    // area -> 16-byte NHWC chunks.  Register g*4 + r of MFMA tile (i, j) is
    // channel i*32 + g*8 + hq*4 + r of pixel j*32 + (lane & 31).
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int cl = i * 32 + g * 8 + hq * 4;
        float sc[4], sh[4];
        c_scale.quad(m0 + wm * WTM + i * 32 + g * 8, hmask, sc);
        c_shift.quad(m0 + wm * WTM + i * 32 + g * 8, hmask, sh);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float t = acc[i][j][g * 4 + r] * sc[r] + sh[r];
            if (a.act == VRS_ACT_SILU) t = silu_fast(t);
            v[r] = t;
          }
          *reinterpret_cast<u32x2_t*>(st + (j * 32 + (lane & 31)) * SROW + cl) =
              (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        }
      }
    __builtin_amdgcn_wave_barrier();   // the staging is read back by this wave only
#pragma unroll
    for (int s = 0; s < NST; ++s) {
      const int c = lane + s * 64;
      const int pl = c / CPP, part = c % CPP;
      const int m = n0 + wn * WTN + pl;
      const int co = m0 + wm * WTM + part * EPC;
      const uint32_t off = m < a.M && co < a.Cout ? ((uint32_t)m * (uint32_t)a.y_sp + (uint32_t)co) * 2u : kOOB;
      __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const u32x4_t*>(st + pl * SROW + part * EPC), ry, off,
                                             0, 0);
    }
    __builtin_amdgcn_wave_barrier();   // staging reads done before the next tile's writes
  }
}
}  // namespace

// Two workgroups' worth of waves per SIMD: the 256x128 and 128x256 tiles then
// keep their accumulators in VGPRs and fit two groups per CU (measured 10-30%
// faster on memory-bound shapes, neutral elsewhere).
#define VRS_CONV_KERNEL(NAME, T, BM, BN, BK, WGM, WGN, AL)                                        \
  extern "C" __global__ __launch_bounds__(64 * WGM * WGN, 2) void NAME(vrs_conv_args a) {        \
    conv_body<T, BM, BN, BK, WGM, WGN, AL>(a);                                                    \
  }

// Kernel names: vrs_conv_<type>_<BM>x<BN>_k<BK>_<a|g>.  Wave tiles: 128x128
// and 64x256 -> 64x64, 256x128 -> 128x64, 128x256 -> 64x128, 32x256 -> 32x64,
// 64x64 -> 32x32 (in 32x32 MFMA tiles).
VRS_CONV_KERNEL(vrs_conv_bf16_128x128_k32_a, bf16_t, 128, 128, 32, 2, 2, true)
VRS_CONV_KERNEL(vrs_conv_bf16_128x128_k32_g, bf16_t, 128, 128, 32, 2, 2, false)
VRS_CONV_KERNEL(vrs_conv_bf16_128x128_k64_a, bf16_t, 128, 128, 64, 2, 2, true)
VRS_CONV_KERNEL(vrs_conv_bf16_256x128_k32_a, bf16_t, 256, 128, 32, 2, 2, true)
VRS_CONV_KERNEL(vrs_conv_bf16_256x128_k64_a, bf16_t, 256, 128, 64, 2, 2, true)
VRS_CONV_KERNEL(vrs_conv_bf16_128x256_k32_a, bf16_t, 128, 256, 32, 2, 2, true)
VRS_CONV_KERNEL(vrs_conv_bf16_128x256_k64_a, bf16_t, 128, 256, 64, 2, 2, true)
VRS_CONV_KERNEL(vrs_conv_bf16_64x256_k32_a, bf16_t, 64, 256, 32, 1, 4, true)
VRS_CONV_KERNEL(vrs_conv_bf16_64x256_k32_g, bf16_t, 64, 256, 32, 1, 4, false)
VRS_CONV_KERNEL(vrs_conv_bf16_64x256_k64_a, bf16_t, 64, 256, 64, 1, 4, true)
VRS_CONV_KERNEL(vrs_conv_bf16_32x256_k32_a, bf16_t, 32, 256, 32, 1, 4, true)
// 64x64 (wave tiles 32x32): small maps, where the larger tiles leave CUs idle
VRS_CONV_KERNEL(vrs_conv_bf16_64x64_k32_a, bf16_t, 64, 64, 32, 2, 2, true)
VRS_CONV_KERNEL(vrs_conv_bf16_64x64_k64_a, bf16_t, 64, 64, 64, 2, 2, true)
VRS_CONV_KERNEL(vrs_conv_bf16_32x256_k32_g, bf16_t, 32, 256, 32, 1, 4, false)
// 8 waves (512 threads), wave tile 128x64: half the global loads per MFMA of
// the 4-wave tiles, for the large layers with Cout >= 256 and Cin % 64 == 0.
VRS_CONV_KERNEL(vrs_conv_bf16_256x256_k64_a, bf16_t, 256, 256, 64, 2, 4, true)
// Fused nearest-2x upsample (_u): the 1x1 convs that read an upsampled concat
#define VRS_CONV_KERNEL_U(NAME, T, BM, BN, BK, WGM, WGN)                                          \
  extern "C" __global__ __launch_bounds__(64 * WGM * WGN, 2) void NAME(vrs_conv_args a) {        \
    conv_body<T, BM, BN, BK, WGM, WGN, true, false, true>(a);                                     \
  }
VRS_CONV_KERNEL_U(vrs_conv_bf16_128x128_k32_u, bf16_t, 128, 128, 32, 2, 2)
VRS_CONV_KERNEL_U(vrs_conv_bf16_128x128_k64_u, bf16_t, 128, 128, 64, 2, 2)
VRS_CONV_KERNEL_U(vrs_conv_bf16_256x128_k32_u, bf16_t, 256, 128, 32, 2, 2)
VRS_CONV_KERNEL_U(vrs_conv_bf16_256x128_k64_u, bf16_t, 256, 128, 64, 2, 2)
VRS_CONV_KERNEL_U(vrs_conv_bf16_128x256_k32_u, bf16_t, 128, 256, 32, 2, 2)
VRS_CONV_KERNEL_U(vrs_conv_bf16_128x256_k64_u, bf16_t, 128, 256, 64, 2, 2)
VRS_CONV_KERNEL_U(vrs_conv_bf16_256x256_k64_u, bf16_t, 256, 256, 64, 2, 4)
VRS_CONV_KERNEL_U(vrs_conv_f32_128x128_k32_u, float, 128, 128, 32, 2, 2)
VRS_CONV_KERNEL_U(vrs_conv_f32_64x256_k32_u, float, 64, 256, 32, 1, 4)
#define VRS_CONV_P(NAME, BM, BN, BK, WGM, WGN)                                                   \
  extern "C" __global__ __launch_bounds__(64 * WGM * WGN, 2) void NAME(vrs_conv_args a) {        \
    conv_persist_body<BM, BN, BK, WGM, WGN>(a);                                                   \
  }
// persistent (memory-bound shapes): vrs_conv_bf16_<BM>x<BN>_k<BK>_p
VRS_CONV_P(vrs_conv_bf16_128x128_k32_p, 128, 128, 32, 2, 2)
VRS_CONV_P(vrs_conv_bf16_64x256_k32_p, 64, 256, 32, 1, 4)
VRS_CONV_P(vrs_conv_bf16_128x128_k64_p, 128, 128, 64, 2, 2)
// 8 waves of 128x64 (as the 256x256 tile), epilogue stored from the accumulators
extern "C" __global__ __launch_bounds__(512, 2) void vrs_conv_bf16_256x256_k64_p(vrs_conv_args a) {
  conv_persist_body<256, 256, 64, 2, 4, true>(a);
}

// f32 (parity path, fp32 MFMA)
VRS_CONV_KERNEL(vrs_conv_f32_128x128_k32_a, float, 128, 128, 32, 2, 2, true)
VRS_CONV_KERNEL(vrs_conv_f32_128x128_k32_g, float, 128, 128, 32, 2, 2, false)
VRS_CONV_KERNEL(vrs_conv_f32_64x256_k32_a, float, 64, 256, 32, 1, 4, true)
VRS_CONV_KERNEL(vrs_conv_f32_64x256_k32_g, float, 64, 256, 32, 1, 4, false)
VRS_CONV_KERNEL(vrs_conv_f32_32x256_k32_a, float, 32, 256, 32, 1, 4, true)
VRS_CONV_KERNEL(vrs_conv_f32_32x256_k32_g, float, 32, 256, 32, 1, 4, false)

// ---------------------------------------------------------------------------
// NCHW float32 image batch -> NHWC (element type) with zero channel padding.
// One thread per output pixel; the c_pad (<= 8) channels go out as one group.
template <typename T>
__device__ __forceinline__ void pack_body(const vrs_pack_args& a) {
  const int64_t HW = (int64_t)a.H * a.W;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.N * HW) return;
  const int64_t b = i / HW, p = i - b * HW;
  T* y = reinterpret_cast<T*>(a.y) + i * a.c_pad;
  for (int c = 0; c < a.c_pad; ++c) {
    const float v = c < a.C ? a.x[(b * a.C + c) * HW + p] : 0.f;
    y[c] = Elt<T>::from_f(v);
  }
}

extern "C" __global__ __launch_bounds__(256) void vrs_pack_nchw_bf16(vrs_pack_args a) { pack_body<bf16_t>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_pack_nchw_f32(vrs_pack_args a) { pack_body<float>(a); }

// NHWC view (element type) -> NCHW float32, one thread per output element.
template <typename T>
__device__ __forceinline__ void unpack_body(const vrs_pack_args& a) {
  // reuse of vrs_pack_args: x = source view base (pre-offset), y = float32 NCHW,
  // N, C (channels of the view), H, W, c_pad = source pitch
  const int64_t HW = (int64_t)a.H * a.W;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.N * a.C * HW) return;
  const int64_t p = i % HW, bc = i / HW;
  const int64_t c = bc % a.C, b = bc / a.C;
  const T* src = reinterpret_cast<const T*>(a.x);
  reinterpret_cast<float*>(a.y)[i] = Elt<T>::to_f(src[(b * HW + p) * a.c_pad + c]);
}

extern "C" __global__ __launch_bounds__(256) void vrs_unpack_nchw_bf16(vrs_pack_args a) { unpack_body<bf16_t>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_unpack_nchw_f32(vrs_pack_args a) { unpack_body<float>(a); }

// ---------------------------------------------------------------------------
// Stem (model.0 = conv(3, c, 3, 2), yolo26/mod.rs:126-195) fused with the
// input layout change: 3x3 stride-2 pad-1 conv straight from the NCHW float32
// image, folded BN + activation, NHWC output of the element type.
//
// Work item: 2 output rows x 64 output pixels of one image.  The grid is
// persistent (a few workgroups per CU, each taking items blockIdx.x,
// +gridDim.x, ...), and an item's 3 channels x 5 input rows x 132 columns are
// loaded into registers while the previous item is computed and stored.
// Per item: the rows go to LDS; each wave takes one 32-pixel tile and builds
// its MFMA operand straight from those rows (k = c*9 + ky*3 + kx, 27 taps + 5
// zero); the [CT*32][32] weights sit in LDS for the whole kernel; results are
// staged in LDS (aliasing the input rows) and written as 16-byte channel
// chunks.  Every global load and store is a raw buffer access with a fixed
// count per item (out-of-range chunks use out-of-range offsets), so the only
// wait on vector memory -- for the prefetched rows -- leaves the previous
// item's stores in flight.  VEC: image width a multiple of 4 (float4 rows).
template <typename T, int CT, bool VEC>
__device__ __forceinline__ void stem_body(const vrs_stem_args& a) {
  using E = Elt<T>;
  using G = typename E::group;
  constexpr int PX = 64, RO = 2, RI = 2 * RO + 1;      // pixels per row, output rows, input rows
  constexpr int CW = 2 * PX + 4, NQ = CW / 4;           // staged columns (float4 aligned)
  constexpr int CP = CT * 32;                           // padded output channels
  constexpr int EPC = 16 / (int)sizeof(T);              // elements per 16-byte chunk
  constexpr int OP = CP + EPC;                          // output staging row (channels + pad)
  constexpr int WP = 32 + EPC;                          // weight row in LDS (k + pad)
  constexpr int IN_BYTES = 3 * RI * CW * 4;
  constexpr int SO_BYTES = RO * PX * OP * (int)sizeof(T);
  constexpr int A_BYTES = IN_BYTES > SO_BYTES ? IN_BYTES : SO_BYTES;   // input and output staging alias
  constexpr int W_BYTES = CP * WP * (int)sizeof(T);
  __shared__ __attribute__((aligned(16))) unsigned char lds[A_BYTES + W_BYTES];
  float (*sin_)[RI][CW] = reinterpret_cast<float (*)[RI][CW]>(lds);
  T* so = reinterpret_cast<T*>(lds);
  T* sw = reinterpret_cast<T*>(lds + A_BYTES);
  const int tid = threadIdx.x, lane = tid & 63, hq = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // weights -> LDS, once
  for (int i = tid; i < CP * 32 / EPC; i += 256) {
    const int row = i / (32 / EPC), part = i % (32 / EPC);
    *reinterpret_cast<u32x4_t*>(sw + row * WP + part * EPC) =
        reinterpret_cast<const u32x4_t*>(a.w)[i];
  }
  // accumulator lane l holds channel j*32 + (l & 31) of tile j
  float sc[CT], sh[CT];
#pragma unroll
  for (int j = 0; j < CT; ++j) {
    const int c = j * 32 + (lane & 31), cc = c < a.cout ? c : a.cout - 1;
    sc[j] = a.scale[cc];
    sh[j] = a.shift[cc];
  }

  const int rp = (a.Ho + RO - 1) / RO;
  const int total = a.N * rp * a.segs;                  // work items (< 2^31, checked on the host)
  const int plane = a.H * a.W;                          // 3 * plane * 4 < 2^31 (host)
  constexpr int NIN = 3 * RI * NQ, NPT = (NIN + 255) / 256;   // float4 chunks of one item's input
  f32x4_t pre[NPT];
  auto fetch = [&](int item) {
    const int seg = item % a.segs, rest = item / a.segs;
    const int oy0 = (rest % rp) * RO, b = rest / rp;
    const int x0 = 2 * seg * PX - 4;                    // staged column 0 (multiple of 4)
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (int64_t)b * 3 * plane, 3 * plane * 4);
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int i = tid + j * 256;
      const int c = i / (RI * NQ), r = (i / NQ) % RI, q = i % NQ;
      const int iy = 2 * oy0 - 1 + r, ix = x0 + 4 * q;
      const bool row_ok = i < NIN && (unsigned)iy < (unsigned)a.H;
      const uint32_t base = (uint32_t)((c * a.H + iy) * a.W + ix) * 4u;
      if constexpr (VEC) {   // a chunk is wholly inside or wholly outside the row
        pre[j] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rx, row_ok && ix >= 0 && ix < a.W ? base : kOOB, 0, 0));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          pre[j][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                    rx, row_ok && (unsigned)(ix + e) < (unsigned)a.W ? base + 4u * e : kOOB, 0, 0));
      }
    }
  };

  // MFMA B operand: lane l feeds pixel (l & 31) of its wave's tile and
  // k = ks*16 + hq*8 + e; tap_off(k) is the tap's float offset from the
  // pixel's window origin (k >= 27, zero weights: offset 0, zeroed after).
  constexpr auto tap_off = [](int k) { return k < 27 ? (k / 9 * RI + k % 9 / 3) * CW + k % 3 : 0; };
  // window origin of this lane's pixel (ro, p): input row 2*(oy0+ro) - 1 is
  // staged row 2*ro, column 2*(ox0+p) - 1 is staged column 2*p + 3
  const int mpx = wave * 32 + (lane & 31);
  const float* org = &sin_[0][2 * (mpx / PX)][2 * (mpx % PX) + 3];

  constexpr int CPPM = CP / EPC, NST = RO * PX * CPPM / 256;   // store chunks per pixel, per thread
  static_assert(RO * PX * CPPM % 256 == 0, "whole store rounds");
  const int cpp = a.cout / EPC;                         // chunks per pixel (cout % 8 == 0, checked)

  int item = blockIdx.x;
  if (item >= total) return;
  fetch(item);
  for (; item < total; item += gridDim.x) {
    const int seg = item % a.segs, rest = item / a.segs;
    const int oy0 = (rest % rp) * RO, b = rest / rp;
    __syncthreads();   // the previous item's staged output has been read
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int i = tid + j * 256;
      if (i < NIN) {
        const int c = i / (RI * NQ), r = (i / NQ) % RI, q = i % NQ;
        *reinterpret_cast<f32x4_t*>(&sin_[c][r][4 * q]) = pre[j];
      }
    }
    if (item + (int)gridDim.x < total) fetch(item + gridDim.x);
    __syncthreads();
    f32x16_t acc[CT];
    {
      G fb[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = org[hq ? tap_off(ks * 16 + 8 + e) : tap_off(ks * 16 + e)];
        if (ks == 1 && hq) {
#pragma unroll
          for (int e = 3; e < 8; ++e) v[e] = 0.f;   // k = 27..31
        }
        fb[ks] = E::from_f8(v);
      }
#pragma unroll
      for (int j = 0; j < CT; ++j) {   // pixels as the A operand: a lane's accumulators share one channel
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          acc[j] = mfma32_k16(fb[ks], E::load(sw + (j * 32 + (lane & 31)) * WP + ks * 16 + hq * 8), acc[j]);
      }
    }
    __syncthreads();   // every wave is done with the input rows (the staging overwrites them)
    // accumulator register r of tile j: channel j*32 + (lane & 31), pixel
    // wave*32 + (r/4)*8 + hq*4 + r%4
    auto epilogue = [&](auto silu_on) {
#pragma unroll
      for (int j = 0; j < CT; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float u = acc[j][r] * sc[j] + sh[j];
          if constexpr (decltype(silu_on)::value) u = silu_t<T>(u);
          so[(wave * 32 + (r >> 2) * 8 + hq * 4 + (r & 3)) * OP + j * 32 + (lane & 31)] = E::from_f(u);
        }
    };
    if (a.act == VRS_ACT_SILU) epilogue(std::true_type{});
    else epilogue(std::false_type{});
    __syncthreads();
    const __amdgpu_buffer_rsrc_t ry =
        make_rsrc(reinterpret_cast<T*>(a.y) + (int64_t)b * a.Ho * a.Wo * a.y_pitch, a.Ho * a.Wo * a.y_pitch * (int)sizeof(T));
#pragma unroll
    for (int s = 0; s < NST; ++s) {
      const int i = tid + s * 256;
      const int px = i / CPPM, part = i % CPPM;
      const int oy = oy0 + px / PX, ox = seg * PX + px % PX;
      const bool ok = part < cpp && oy < a.Ho && ox < a.Wo;
      const uint32_t off = ok ? (uint32_t)(((oy * a.Wo + ox) * a.y_pitch + part * EPC) * (int)sizeof(T)) : kOOB;
      __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const u32x4_t*>(so + px * OP + part * EPC), ry, off, 0, 0);
    }
  }
}

#define VRS_STEM(DT, T, CT, LB)                                                                          \
  extern "C" __global__ __launch_bounds__(256, LB) void vrs_stem_##DT##_c##CT(vrs_stem_args a) {        \
    stem_body<T, CT, true>(a);                                                                           \
  }                                                                                                      \
  extern "C" __global__ __launch_bounds__(256, LB) void vrs_stem_##DT##_c##CT##_u(vrs_stem_args a) {    \
    stem_body<T, CT, false>(a);                                                                          \
  }
// kernel names: vrs_stem_<type>_c<cout_pad/32>[_u: image width not a multiple of 4]
VRS_STEM(bf16, bf16_t, 1, 4)
VRS_STEM(bf16, bf16_t, 2, 4)
VRS_STEM(bf16, bf16_t, 3, 4)
VRS_STEM(bf16, bf16_t, 4, 4)
VRS_STEM(f32, float, 1, 2)
VRS_STEM(f32, float, 2, 2)
VRS_STEM(f32, float, 3, 2)
VRS_STEM(f32, float, 4, 2)

// Implicit-GEMM Conv2d + folded BatchNorm + SiLU (+ residual) for gfx950: the
// body shared by the bf16/float32 kernels (conv.hip) and the fp8 kernels
// (conv8.hip).
//
// Semantics (blocks/conv.rs:31-99, fused as Graph::optimise() does at
// examples/yolo26.rs:3021): y = act(scale[co] * sum_k W[co,k] x_col[k,p] + shift[co]) + res.
//
// GEMM view: rows = output channels (Cout), cols = output pixels (N*Ho*Wo),
// K = kh*kw*Cin taken in NHWC order (tap-major, channel-minor), so one group of
// 8 consecutive k is 8 consecutive channels of one input pixel: a single
// 16-byte load.  Weights are the MFMA A operand and pixels the B operand, so
// each lane's accumulator quad is 4 consecutive output channels of one pixel
// and the NHWC store is a vector store.
//
// Workgroup: 256 threads = 4 wave64, tile BM (Cout) x BN (pixels), BK = 32.
// Tiles are staged through double-buffered LDS (one barrier per K step) with
// the next step's global loads in flight during the MFMAs.
#pragma once
#include "common.h"

namespace {

// Instruction interleave of one pipelined K step (NM MFMAs, NRK fragment
// reads per 16-deep k slice of NMK MFMAs, NX global loads and as many LDS
// writes): the fragment reads of slice kk+1 ride on the MFMAs of slice kk,
// the global loads of step k+2 go out during the first half of the MFMAs and
// the LDS writes of step k+1 (whose loads then had a whole step to land)
// during the second half.
template <int I, int NM, int NRK, int NMK, int NX>
__device__ __forceinline__ void pipe_schedule_at() {
  if constexpr (I < NM) {
    constexpr int KS = NM / NMK, kk = I / NMK, j = I % NMK, H = NM / 2;
    constexpr int nr = kk + 1 < KS ? (j + 1) * NRK / NMK - j * NRK / NMK : 0;
    constexpr int nv = I < H ? (I + 1) * NX / H - I * NX / H : 0;
    constexpr int nw = I >= H ? (I - H + 1) * NX / (NM - H) - (I - H) * NX / (NM - H) : 0;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    if constexpr (nr > 0) __builtin_amdgcn_sched_group_barrier(0x100, nr, 0);  // DS read
    if constexpr (nv > 0) __builtin_amdgcn_sched_group_barrier(0x020, nv, 0);  // VMEM read
    if constexpr (nw > 0) __builtin_amdgcn_sched_group_barrier(0x200, nw, 0);  // DS write
    pipe_schedule_at<I + 1, NM, NRK, NMK, NX>();
  }
}
template <int NM, int NRK, int NMK, int NX>
__device__ __forceinline__ void pipe_schedule() {
  __builtin_amdgcn_sched_group_barrier(0x100, NRK, 0);  // slice 0 fragments
  pipe_schedule_at<0, NM, NRK, NMK, NX>();
}

// BM output channels x BN pixels per workgroup, BK reduction elements per
// pipeline step, WGM x WGN waves (wave tile (BM/WGM) x (BN/WGN)).
// ALIGNED: Cin % BK == 0, so a K step never straddles two filter taps.
// F8: weights are e4m3 bytes (A operand, 16-byte chunks of 16 k), the bf16
// activations are quantised to e4m3 while staged into LDS (8 k per 16-byte
// group -> 8 bytes), and the 32x32x64 fp8 MFMA consumes 64-byte LDS rows.
// UP: input channels [0, a.c_split) come from the half-resolution a.x2 at
// (y/2, x/2) (fused nearest-2x upsample; 1x1 stride-1 convs, checked on the
// host); the K steps of those channels come first and switch the B source.
// XF8 (fp8 tiles): the activations (x, and x2 of UP) are already e4m3 bytes
// on the input step, staged into LDS as read (16 k per 16-byte chunk, no
// conversion).  YF8 (fp8 tiles): the output is e4m3 on a.out_step (staged
// 16-byte chunks of 16 channels).  A residual is bf16, or e4m3 on a.res_step
// when a.res_f8 (fp8 tiles).
template <typename T, int BM, int BN, int BK, int WGM, int WGN, bool ALIGNED, bool F8 = false, bool UP = false,
          bool XF8 = false, bool YF8 = false>
__device__ __forceinline__ void conv_body(const vrs_conv_args& a) {
  using E = Elt<T>;
  using G = typename E::group;
  static_assert(!F8 || (sizeof(T) == 2 && (BK == 64 || BK == 128) && ALIGNED), "fp8: 64- or 128-deep steps");
  static_assert(F8 || (!XF8 && !YF8), "e4m3 activations only on the fp8 tiles");
  // LDS rows of BK + 8 elements: the 32 rows a half-wave reads with
  // ds_read_b128 (row stride 144 B for BK=64 bf16) start on distinct 4-bank
  // groups of the 64 banks (measured: 4% conflict cycles vs 34% at +16).
  constexpr int PAD = 8;
  // bf16 with 32-deep steps: 64-byte rows, no padding, 16-byte chunk j of
  // row r stored at chunk j ^ ((r >> 2) & 3): the 16 rows a quarter-wave
  // reads (one chunk each) and the 4 rows x 4 chunks it writes both cover
  // the 64 banks once (padded rows left the writes 2-way conflicted: 39 %
  // conflict cycles on the 32x256 tile).
  // (Wave tiles above 64x64 keep the padded rows: their register budget
  // has no room for the swizzled addressing.)
  constexpr bool SWZ = !F8 && sizeof(T) == 2 && BK == 32 && (BM / WGM) * (BN / WGN) <= 64 * 64;
  constexpr int LDK = BK + (SWZ ? 0 : PAD);  // LDS row stride in elements
  constexpr int GPR = BK / 8;                // 8-element groups per tile row (B, and A when !F8)
  constexpr int GPRA = F8 ? BK / 16 : GPR;   // 16-byte weight chunks per row
  constexpr int GPRB = XF8 ? BK / 16 : GPR;  // 16-byte activation chunks per row
  constexpr int CEB = XF8 ? 16 : 8;          // activation elements per chunk
  constexpr int XS = XF8 ? 1 : (int)sizeof(T);   // bytes per activation element
  constexpr int AEL = F8 ? 16 : 8;           // weight elements per chunk
  constexpr int LDKB = BK + 16;              // F8: LDS row stride in bytes (80 or 144: the 16 rows a
                                             // quarter-wave reads start on distinct 4-bank groups)
  constexpr int NT = 64 * WGM * WGN;         // threads per workgroup
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int TM = WTM / 32, TN = WTN / 32;   // 32x32 MFMA tiles per wave
  constexpr int A_IT = (BM * GPRA + NT - 1) / NT;
  constexpr int B_IT = (BN * GPRB + NT - 1) / NT;
  constexpr bool A_FULL = (BM * GPRA) % NT == 0;   // every thread owns A_IT chunks
  constexpr bool B_FULL = (BN * GPRB) % NT == 0;
  // Branch-free software pipeline (two register sets, interleaved schedule)
  // when every thread loads whole chunks; otherwise the plain loop.
  constexpr bool PIPE = ALIGNED && A_FULL && B_FULL;
  constexpr int TILE_ELEMS = F8 ? (BM + BN) * LDKB / 2 : (BM + BN) * LDK;   // one pipeline stage
  // epilogue staging: per wave WTN pixels x (WTM + SPAD) channels
  constexpr int SPAD = 16 / (int)sizeof(T);
  constexpr int STAGE2 = (WGM * WGN / 2) * WTN * (WTM + SPAD);   // half the waves' staging
  constexpr int BUF_ELEMS = TILE_ELEMS > STAGE2 ? TILE_ELEMS : STAGE2;
  static_assert(TM >= 1 && TN >= 1 && BK % 32 == 0, "tile");
  static_assert(!F8 || PIPE, "fp8 needs whole-chunk loads (the pipelined loop)");

  // The two pipeline buffers are separate objects so the compiler can move
  // LDS writes of one past reads of the other.  Epilogue staging: the first
  // half of the waves
  // use buffer 0, the other half buffer 1.
  __shared__ __attribute__((aligned(16))) T smem0[BUF_ELEMS];
  __shared__ __attribute__((aligned(16))) T smem1[BUF_ELEMS];
  auto sbuf = [&](int b) -> T* { return b ? smem1 : smem0; };
  // element offset of 8-element chunk `chunk` of LDS row `row`
  const int tid = threadIdx.x;
  // LDS slot of this thread's staged chunks: chunk i of the thread is row
  // tid / GPR + i * NT / GPR (a multiple of 4 further down: same swizzle)
  static_assert(!SWZ || (NT / GPR) % 4 == 0, "swizzle period");
  const int st_row = tid / GPR, st_chunk = tid % GPR;
  const int st_off = st_row * LDK + (SWZ ? st_chunk ^ ((st_row >> 2) & 3) : st_chunk) * 8;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  static_assert(WGM * WGN == 4 || WGM * WGN == 8, "4 or 8 waves");

  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int tile_m = logical % a.tiles_m, tile_n = a.n_tile0 + logical / a.tiles_m;
  const int m0 = tile_m * BM;   // first output channel
  const int n0 = tile_n * BN;   // first output pixel
  // folded-BN constants of the tile's BM channels, staged in LDS for the
  // epilogue (visible after the K loop's first barrier): each lane then reads
  // its 4 channels as one 16-byte LDS load instead of selecting them from
  // scalar registers per value
  // (bf16 tiles; the fp8 tiles, whose registers are tighter, and the float32
  // ones, whose two workgroups per CU leave no LDS for it, select them from
  // the scalar cache)
  constexpr bool LDS_CONST = !F8 && sizeof(T) == 2;
  __shared__ __attribute__((aligned(16))) float s_scale[LDS_CONST ? BM : 4];
  __shared__ __attribute__((aligned(16))) float s_shift[LDS_CONST ? BM : 4];
  if (LDS_CONST)
  for (int c = threadIdx.x; c < BM; c += 64 * WGM * WGN) {
    const bool ok = m0 + c < a.Cout;
    s_scale[c] = ok ? a.scale[m0 + c] : 0.f;
    s_shift[c] = ok ? a.shift[m0 + c] : 0.f;
  }

  const T* __restrict__ x = reinterpret_cast<const T*>(a.x);
  const T* __restrict__ w = reinterpret_cast<const T*>(a.w);
  const int HWo = a.Ho * a.Wo;
  // pixel index -> (image, position): float-reciprocal divmod (M < 2^24 is
  // checked on the host)
  const float inv_hwo = 1.0f / (float)HWo, inv_wo = 1.0f / (float)a.Wo;

  // Per-thread chunk geometry, fixed over the K loop: the A pointer advances
  // by k0; the B (pixel) pointer is the tap-(0,0) input pixel and each K step
  // adds a wave-uniform tap offset, so the loop body does one 64-bit add and
  // two range checks per chunk.
  const T* a_ptr[A_IT];
  bool a_ok[A_IT];
#pragma unroll
  for (int i = 0; i < A_IT; ++i) {
    const int c = tid + i * NT;
    const int co = m0 + c / GPRA;
    a_ok[i] = (A_FULL || c < BM * GPRA) && (co < a.Cout);
    a_ptr[i] = w + (int64_t)(a_ok[i] ? co : 0) * a.K + (c % GPRA) * 8;
  }
  int b_iy0[B_IT], b_ix0[B_IT];
  int64_t b_el[B_IT];   // element offset of the chunk's tap-(0,0) position in x
  bool b_ok[B_IT];
  uint32_t b_off2[B_IT];   // fused upsample: byte offset of the pixel's source in x2
#pragma unroll
  for (int i = 0; i < B_IT; ++i) {
    const int c = tid + i * NT;
    const int m = n0 + c / GPRB;
    b_ok[i] = (B_FULL || c < BN * GPRB) && (m < a.M);
    const int mm = b_ok[i] ? m : 0;
    int rr, ox;
    const int bb = fdivmod(mm, HWo, inv_hwo, rr);
    const int oy = fdivmod(rr, a.Wo, inv_wo, ox);
    b_iy0[i] = oy * a.stride - a.pad;
    b_ix0[i] = ox * a.stride - a.pad;
    b_el[i] = (((int64_t)bb * a.H + b_iy0[i]) * a.W + b_ix0[i]) * a.x_pitch + (c % GPRB) * CEB;
    if constexpr (UP)
      b_off2[i] = b_ok[i] ? (uint32_t)((((int64_t)bb * a.H2 + (oy >> 1)) * a.W2 + (ox >> 1)) * a.x2_pitch +
                                       (c % GPRB) * CEB) * (uint32_t)XS
                          : kOOB;
  }

  G ra[A_IT], rb[B_IT];

  // ALIGNED path: raw buffer loads.  Weight rows: per-lane byte offset, the
  // K step as the scalar offset.  Pixels: per-lane byte offset of the
  // tap-(0,0) position plus a wave-uniform tap offset; lanes whose tap falls
  // in the zero padding (or past the last pixel/row) use kOOB and read zeros.
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w, a.w_bytes);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t rx2 = UP ? make_rsrc(a.x2, a.x2_bytes) : rx;
  uint32_t a_off[A_IT], b_off[B_IT];
  if (ALIGNED) {
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
      if constexpr (F8) {   // weights are bytes: row co * K, chunk * 16
        const int c = tid + i * NT;
        a_off[i] = a_ok[i] ? (uint32_t)((m0 + c / GPRA) * a.K + (c % GPRA) * AEL) : kOOB;
      } else {
        a_off[i] = a_ok[i] ? (uint32_t)((a_ptr[i] - w) * (int)sizeof(T)) : kOOB;
      }
    }
#pragma unroll
    for (int i = 0; i < B_IT; ++i) b_off[i] = (uint32_t)(b_el[i] * XS);
  }

  // (ky, kx, ci0) of the next step to load, advanced incrementally (ALIGNED:
  // a step never crosses a tap).  Steps run channel-chunk-outer, tap-inner:
  // the kh*kw taps of one BK-channel chunk are consecutive steps, so the
  // input rows a tile reads stay in L1/L2 across its taps instead of being
  // fetched again per tap; the weight offset of a step is
  // (ky*kw + kx)*Cin + ci0 in the [Cout][kh][kw][Cin] packing.
  // float32 kernels (the 1e-4 parity path) keep the tap-outer order, whose
  // float32 summation order the network-level tolerance was set against.
  constexpr bool TAP_INNER = sizeof(T) == 2;
  int t_ky = 0, t_kx = 0, t_ci = 0;
  auto advance = [&]() {
    if constexpr (TAP_INNER) {
      if (++t_kx == a.kw) {
        t_kx = 0;
        if (++t_ky == a.kh) { t_ky = 0; t_ci += BK; }
      }
    } else {
      t_ci += BK;
      if (t_ci == a.Cin) {
        t_ci = 0;
        if (++t_kx == a.kw) { t_kx = 0; ++t_ky; }
      }
    }
  };
  auto load_tiles = [&](int k0) {
    if (ALIGNED) {
#pragma unroll
      for (int i = 0; i < A_IT; ++i)
        ra[i] = E::bload(rw, a_off[i], (TAP_INNER ? (uint32_t)((t_ky * a.kw + t_kx) * a.Cin + t_ci) : (uint32_t)k0) *
                                           sizeof(T));
      const int ky = t_ky, kx = t_kx;
      const uint32_t off = (uint32_t)((ky * a.W + kx) * a.x_pitch + t_ci) * sizeof(T);
      const bool lo = UP && t_ci < a.c_split;   // fused upsample: this chunk comes from x2 (uniform)
      const uint32_t off2 = (uint32_t)t_ci * sizeof(T);
      advance();
#pragma unroll
      for (int i = 0; i < B_IT; ++i) {
        const int iy = b_iy0[i] + ky, ix = b_ix0[i] + kx;
        const bool ok = b_ok[i] && (unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W;
        if constexpr (UP)
          rb[i] = E::bload(lo ? rx2 : rx, lo ? b_off2[i] + off2 : (ok ? b_off[i] + off : kOOB), 0);
        else
          rb[i] = E::bload(rx, ok ? b_off[i] + off : kOOB, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < A_IT; ++i) {
        const int k = k0 + ((tid + i * NT) % GPR) * 8;
        ra[i] = (a_ok[i] && k < a.K) ? E::load(a_ptr[i] + k0) : E::zero();
      }
#pragma unroll
      for (int i = 0; i < B_IT; ++i) {
        const int grp = (tid + i * NT) % GPR;
        const int k = k0 + grp * 8;
        const int t = k / a.Cin, ci = k - t * a.Cin;
        const int ky = t / a.kw, kx = t - ky * a.kw;
        const int iy = b_iy0[i] + ky, ix = b_ix0[i] + kx;
        const bool ok = b_ok[i] && (k < a.K) && (unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W;
        rb[i] = ok ? E::load(x + b_el[i] - grp * 8 + ((int64_t)ky * a.W + kx) * a.x_pitch + ci) : E::zero();
      }
    }
  };

  auto store_tiles = [&](int buf) {
    T* sA = sbuf(buf);
    T* sB = sA + BM * LDK;
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
      const int c = tid + i * NT;
      if (A_FULL || c < BM * GPR) E::store(&sA[st_off + i * (NT / GPR) * LDK], ra[i]);
    }
#pragma unroll
    for (int i = 0; i < B_IT; ++i) {
      const int c = tid + i * NT;
      if (B_FULL || c < BN * GPR) E::store(&sB[st_off + i * (NT / GPR) * LDK], rb[i]);
    }
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = (a.K + BK - 1) / BK;
  const int frag_row = lane & 31;
  // fragment rows are frag_row plus multiples of 32, so their swizzle term is
  // (frag_row >> 2) & 3 for every tile row
  const int frag_swz = SWZ ? (frag_row >> 2) & 3 : 0;
  auto frag_off = [&](int kk) { return ((kk * 2 + (lane >> 5)) ^ frag_swz) * 8; };

  if constexpr (PIPE) {
    // Step k: LDS buffer k&1 holds step k; register set (k+1)&1 holds step
    // k+1 (loaded during step k-1) and is written to buffer (k+1)&1 while
    // the MFMAs of step k run; set k&1 receives the loads of step k+2.  Loads
    // at k0 >= K read zeros (out-of-range buffer offsets), so the body has no
    // branches; an odd step count ends with one more copy of the step (the
    // 8-wave tile, which has no registers to spare for it, runs one all-zero
    // step instead).
    G ra0[A_IT], rb0[B_IT], ra1[A_IT], rb1[B_IT];
    auto load_set = [&](int k0, G (&ra)[A_IT], G (&rb)[B_IT]) {
      const uint32_t dead = k0 < a.K ? 0u : kOOB;
#pragma unroll
      for (int i = 0; i < A_IT; ++i)
        ra[i] = E::bload(rw, a_off[i] | dead,
                         (TAP_INNER ? (uint32_t)((t_ky * a.kw + t_kx) * a.Cin + t_ci) : (uint32_t)k0) *
                             (F8 ? 1u : (uint32_t)sizeof(T)));
      const int ky = t_ky, kx = t_kx;
      const uint32_t off = (uint32_t)((ky * a.W + kx) * a.x_pitch + t_ci) * (uint32_t)XS;
      const bool lo = UP && t_ci < a.c_split;   // fused upsample: this chunk comes from x2 (uniform)
      const uint32_t off2 = (uint32_t)t_ci * (uint32_t)XS;
      advance();
#pragma unroll
      for (int i = 0; i < B_IT; ++i) {
        const int iy = b_iy0[i] + ky, ix = b_ix0[i] + kx;
        const bool ok = b_ok[i] && (unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W;
        if constexpr (UP)
          rb[i] = E::bload(lo ? rx2 : rx, (lo ? b_off2[i] + off2 : (ok ? b_off[i] + off : kOOB)) | dead, 0);
        else
          rb[i] = E::bload(rx, (ok ? b_off[i] + off : kOOB) | dead, 0);
      }
    };
    auto store_set = [&](int buf, const G (&ra)[A_IT], const G (&rb)[B_IT]) {
      if constexpr (F8) {
        unsigned char* sA = reinterpret_cast<unsigned char*>(sbuf(buf));
        unsigned char* sB = sA + BM * LDKB;
#pragma unroll
        for (int i = 0; i < A_IT; ++i) {
          const int c = tid + i * NT;
          *reinterpret_cast<u32x4_t*>(sA + (c / GPRA) * LDKB + (c % GPRA) * 16) =
              *reinterpret_cast<const u32x4_t*>(&ra[i]);
        }
#pragma unroll
        for (int i = 0; i < B_IT; ++i) {
          const int c = tid + i * NT;
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&rb[i]);
          if constexpr (XF8) {   // 16 e4m3 activations: stored as read
            *reinterpret_cast<u32x4_t*>(sB + (c / GPRB) * LDKB + (c % GPRB) * 16) = v;
          } else {
            const u32x2_t q = {bf16x2_to_fp8x2(v[0], a.clamp_bits, a.in_scale) |
                                   (bf16x2_to_fp8x2(v[1], a.clamp_bits, a.in_scale) << 16),
                               bf16x2_to_fp8x2(v[2], a.clamp_bits, a.in_scale) |
                                   (bf16x2_to_fp8x2(v[3], a.clamp_bits, a.in_scale) << 16)};
            *reinterpret_cast<u32x2_t*>(sB + (c / GPR) * LDKB + (c % GPR) * 8) = q;
          }
        }
      } else {
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
      }
    };
    auto step = [&](int cur, const G (&wa)[A_IT], const G (&wb)[B_IT], G (&la)[A_IT], G (&lb)[B_IT], int k_load) {
      load_set(k_load, la, lb);
      store_set(cur ^ 1, wa, wb);
      if constexpr (F8) {
        const unsigned char* sA = reinterpret_cast<const unsigned char*>(sbuf(cur));
        const unsigned char* sB = sA + BM * LDKB;
        const int fk = (lane >> 5) * 32;
        auto ld32 = [&](const unsigned char* p) {
          const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(p);
          const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(p + 16);
          return (i32x8_t){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        };
        // one 64-deep k slice per fp8 MFMA: fragment bytes [kk*64, kk*64+64)
        // of each staged row
#pragma unroll
        for (int kk = 0; kk < BK / 64; ++kk) {
          i32x8_t fa[TM], fb[TN];
#pragma unroll
          for (int i = 0; i < TM; ++i) fa[i] = ld32(sA + (wm * WTM + i * 32 + frag_row) * LDKB + kk * 64 + fk);
#pragma unroll
          for (int j = 0; j < TN; ++j) fb[j] = ld32(sB + (wn * WTN + j * 32 + frag_row) * LDKB + kk * 64 + fk);
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = mfma32_fp8_k64(fa[i], fb[j], acc[i][j]);
        }
        pipe_schedule<BK / 64 * TM * TN, 2 * (TM + TN), TM * TN, A_IT + B_IT>();
        __syncthreads();
        return;
      }
      const T* sA = sbuf(cur);
      const T* sB = sA + BM * LDK;
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        G fa[TM], fb[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
          fa[i] = E::load(&sA[(wm * WTM + i * 32 + frag_row) * LDK + frag_off(kk)]);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          fb[j] = E::load(&sB[(wn * WTN + j * 32 + frag_row) * LDK + frag_off(kk)]);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma32_k16(fa[i], fb[j], acc[i][j]);
      }
      pipe_schedule<BK / 16 * TM * TN, TM + TN, TM * TN, A_IT + B_IT>();
      __syncthreads();
    };
    load_set(0, ra0, rb0);
    load_set(BK, ra1, rb1);
    store_set(0, ra0, rb0);
    __syncthreads();
    constexpr bool TAIL = WGM * WGN == 4;
    for (int kt = 0; TAIL ? kt + 1 < nk : kt < nk; kt += 2) {
      step(0, ra1, rb1, ra0, rb0, (kt + 2) * BK);
      step(1, ra0, rb0, ra1, rb1, (kt + 3) * BK);
    }
    if (TAIL && (nk & 1)) step(0, ra1, rb1, ra0, rb0, (nk + 1) * BK);
  } else {
  load_tiles(0);
  store_tiles(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tiles((kt + 1) * BK);
    const T* sA = sbuf(cur);
    const T* sB = sA + BM * LDK;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      G fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[i] = E::load(&sA[(wm * WTM + i * 32 + frag_row) * LDK + frag_off(kk)]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[j] = E::load(&sB[(wn * WTN + j * 32 + frag_row) * LDK + frag_off(kk)]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32_k16(fa[i], fb[j], acc[i][j]);
    }
    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }
  }

  // Epilogue: folded BN, activation, residual.  Accumulator register
  // g*4 + r of MFMA tile (i, j) is channel i*32 + g*8 + hq*4 + r of pixel
  // j*32 + (lane & 31), hq = lane >> 5.  Instantiated per activation so the
  // identity layers carry no SiLU and the SiLU layers no per-value select.
  const int hq = lane >> 5;
  const ChanConst c_scale(a.scale, a.Cout), c_shift(a.shift, a.Cout);
  const uint32_t hmask = upper_half_mask();
  auto chan4 = [&](const float* s, int i, int g) {
    if constexpr (!LDS_CONST) {
      float q[4];
      (s == s_scale ? c_scale : c_shift).quad(m0 + wm * WTM + i * 32 + g * 8, hmask, q);
      return (f32x4_t){q[0], q[1], q[2], q[3]};
    } else {
      return *reinterpret_cast<const f32x4_t*>(&s[wm * WTM + i * 32 + g * 8 + hq * 4]);
    }
  };
  // MODE 0: identity, 1: SiLU, 2: chosen per value at run time (the fp8
  // tiles: a second epilogue copy costs them registers)
  auto epilogue = [&](auto mode_tag) {
    constexpr int MODE = decltype(mode_tag)::value;
    if constexpr (sizeof(T) == 2 && !F8) {
      if (a.stage == 2) {
        // Channel-major float32 output (the Detect heads' flat layout:
        // element (b, p, co) at y + b*y_sb + p + co*y_sc): the wave tile goes
        // through LDS as [channel][pixel] rows, CH channels per pass, and
        // each lane stores 4 consecutive pixels of one channel as one 16-byte
        // raw-buffer store (the host checks that 4 pixels never straddle two
        // images and the 16-byte alignment of y, y_sb and y_sc).  Each wave
        // reads back only what it wrote, so the passes need no barrier.
        constexpr int HW_ = WGM * WGN / 2;              // waves per pipeline buffer
        constexpr int PR = WTN + 8;                     // staging row (floats): the
                                                        // two half-waves' rows 32 banks apart
        constexpr int WB = TILE_ELEMS * (int)sizeof(T) / HW_ / 4;   // floats per wave
        constexpr int FIT = WB / PR;
        constexpr int CH = (FIT >= 128 && WTM >= 128) ? 128
                           : (FIT >= 64 && WTM >= 64) ? 64
                           : FIT >= 32 ? 32 : FIT >= 16 ? 16 : 8;
        static_assert(FIT >= 8 && WTM % CH == 0, "flat staging fits the pipeline buffers");
        constexpr int QPR = WTN / 4;                    // pixel quads per staged row
        constexpr int NSQ = CH * QPR / 64;              // stores per lane per pass
        static_assert(CH * QPR % 64 == 0, "whole store rounds");
        float* st = reinterpret_cast<float*>(sbuf(wave / HW_)) + (wave % HW_) * WB;
        const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y, a.y_bytes);
#pragma unroll
        for (int pass = 0; pass < WTM / CH; ++pass) {
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const int cb = i * 32 + g * 8;
              if (cb < pass * CH || cb >= (pass + 1) * CH) continue;
              const int cl = cb - pass * CH + hq * 4;
              const f32x4_t sc = chan4(s_scale, i, g), sh = chan4(s_shift, i, g);
#pragma unroll
              for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  float t = acc[i][j][g * 4 + r] * sc[r] + sh[r];
                  if constexpr (MODE == 1) t = silu_t<T>(t);
                  st[(cl + r) * PR + j * 32 + (lane & 31)] = t;
                }
            }
#pragma unroll
          for (int q = 0; q < NSQ; ++q) {
            const int c = lane + q * 64, cl = c / QPR, pq = c % QPR;
            const int co = m0 + wm * WTM + pass * CH + cl;
            const int m = n0 + wn * WTN + pq * 4;
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&st[cl * PR + pq * 4]);
            uint32_t off = kOOB;
            if (m < a.M && co < a.Cout) {
              int p;
              const int b = fdivmod(m, HWo, inv_hwo, p);
              off = (uint32_t)(((int64_t)b * a.y_sb + p + (int64_t)co * a.y_sc) * 4);
            }
            __builtin_amdgcn_raw_buffer_store_b128(v, ry, off, 0, 0);
          }
        }
        return;
      }
    }
    if (YF8 || a.stage) {
      // Staged store: every wave writes its (WTN pixel x WTM channel) tile to
      // LDS, then stores whole 16-byte channel chunks per lane, so consecutive
      // lanes write contiguous bytes of a pixel's NHWC row.  YF8: the tile is
      // staged in bfloat16 like a bf16 output, and each 16-byte store takes 16
      // staged channels rounded to e4m3 on out_step (the output is the e4m3
      // rounding of the bf16 value; converting while staging instead held
      // twice the registers through the epilogue).  The host stages YF8
      // outputs only, 16-channel aligned.
      constexpr int HW_ = WGM * WGN / 2;
      constexpr int OB = YF8 ? 1 : (int)sizeof(T);        // bytes per output element
      constexpr int SROW = (WTM + SPAD) * (int)sizeof(T);  // bytes per staged pixel row
      unsigned char* st = reinterpret_cast<unsigned char*>(sbuf(wave / HW_)) + (wave % HW_) * WTN * SROW;
      // the host stages only views addressable with 32-bit byte offsets
      // (y_bytes, res_bytes): pixel m of an NHWC view starts at m * pitch
      const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y, a.y_bytes);
      const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.res, a.res ? a.res_bytes : 0);
      const bool res_f8 = F8 && a.res_f8;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int cl = i * 32 + g * 8 + hq * 4;   // channel within the wave tile
          const int co = m0 + wm * WTM + cl;
          const f32x4_t sc = chan4(s_scale, i, g), sh = chan4(s_shift, i, g);
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int pl = j * 32 + (lane & 31);
            const int m = n0 + wn * WTN + pl;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float t = acc[i][j][g * 4 + r] * sc[r] + sh[r];
              if constexpr (MODE == 1) t = silu_t<T>(t);
              if constexpr (MODE == 2) if (a.act == VRS_ACT_SILU) t = silu_t<T>(t);
              v[r] = t;
            }
            if (a.res) {   // NHWC view: pixel m at m * pitch (raw buffer, out-of-range lanes read 0)
              const bool in = m < a.M && co < a.Cout;
              const uint32_t re = (uint32_t)m * (uint32_t)a.r_sp + (uint32_t)co;   // element offset
              if (res_f8) {   // 4 e4m3 channels on the residual's step
                const uint32_t rv = __builtin_amdgcn_raw_buffer_load_b32(rr, in ? re : kOOB, 0, 0);
                float d[4];
                fp8x4_to_f32(rv, a.res_step, d);
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] += d[r];
              } else if constexpr (sizeof(T) == 2) {
                const u32x2_t rv = __builtin_amdgcn_raw_buffer_load_b64(rr, in ? re * 2u : kOOB, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                  v[r] += __uint_as_float((r & 1) ? (rv[r >> 1] & 0xffff0000u) : (rv[r >> 1] << 16));
              } else {
                const u32x4_t rv = __builtin_amdgcn_raw_buffer_load_b128(rr, in ? re * 4u : kOOB, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] += __uint_as_float(rv[r]);
              }
            }
            unsigned char* sp = st + pl * SROW + cl * (int)sizeof(T);
            if constexpr (sizeof(T) == 2) {
              *reinterpret_cast<u32x2_t*>(sp) = (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            } else {
              *reinterpret_cast<f32x4_t*>(sp) = (f32x4_t){v[0], v[1], v[2], v[3]};
            }
          }
        }
      __syncthreads();
      constexpr int EPC = 16 / OB;              // elements per 16-byte chunk
      constexpr int CPP = WTM / EPC;            // chunks per pixel row
      const int co_w = m0 + wm * WTM;
      static_assert((WTN * CPP) % 64 == 0, "whole store rounds");
      uint32_t lim = 0;   // YF8: bfloat16 bits of 448 * out_step in both halves (exact)
      if constexpr (YF8) {
        lim = __float_as_uint(448.f * a.out_step) >> 16;
        lim |= lim << 16;
      }
#pragma unroll
      for (int s = 0; s < WTN * CPP / 64; ++s) {
        const int c = lane + s * 64;
        const int pl = c / CPP, part = c % CPP;
        const int m = n0 + wn * WTN + pl;
        const int co = co_w + part * EPC;
        u32x4_t v;
        if constexpr (YF8) {
          const u32x4_t h0 = *reinterpret_cast<const u32x4_t*>(st + pl * SROW + part * 32);
          const u32x4_t h1 = *reinterpret_cast<const u32x4_t*>(st + pl * SROW + part * 32 + 16);
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            v[q] = bf16x2_to_fp8x2(h0[2 * q], lim, a.out_step) | (bf16x2_to_fp8x2(h0[2 * q + 1], lim, a.out_step) << 16);
            v[q + 2] = bf16x2_to_fp8x2(h1[2 * q], lim, a.out_step) | (bf16x2_to_fp8x2(h1[2 * q + 1], lim, a.out_step) << 16);
          }
        } else {
          v = *reinterpret_cast<const u32x4_t*>(st + pl * SROW + part * 16);
        }
        const uint32_t off = m < a.M && co < a.Cout
                                 ? ((uint32_t)m * (uint32_t)a.y_sp + (uint32_t)co) * (uint32_t)OB
                                 : kOOB;
        __builtin_amdgcn_raw_buffer_store_b128(v, ry, off, 0, 0);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int co = m0 + wm * WTM + i * 32 + g * 8 + hq * 4;
        const f32x4_t sc = chan4(s_scale, i, g), sh = chan4(s_shift, i, g);
        if (co >= a.Cout) continue;
        const bool full4 = (co + 3 < a.Cout);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int m = n0 + wn * WTN + j * 32 + (lane & 31);
          if (m >= a.M) continue;
          int pp;
          const int bb = fdivmod(m, HWo, inv_hwo, pp);
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float t = acc[i][j][g * 4 + r] * sc[r] + sh[r];
            if constexpr (MODE == 1) t = silu_t<T>(t);
            if constexpr (MODE == 2) if (a.act == VRS_ACT_SILU) t = silu_t<T>(t);
            v[r] = t;
          }
          if (a.res) {
            const T* rp = reinterpret_cast<const T*>(a.res) + bb * a.r_sb + pp * a.r_sp + (int64_t)co * a.r_sc;
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (co + r < a.Cout) v[r] += E::to_f(rp[r * a.r_sc]);
          }
          const int64_t yo = bb * a.y_sb + pp * a.y_sp + (int64_t)co * a.y_sc;
          if (a.y_f32) {
            float* yp = reinterpret_cast<float*>(a.y) + yo;
            if (a.y_sc == 1 && full4) {
              *reinterpret_cast<f32x4_t*>(yp) = (f32x4_t){v[0], v[1], v[2], v[3]};
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (co + r < a.Cout) yp[r * a.y_sc] = v[r];
            }
          } else {
            T* yp = reinterpret_cast<T*>(a.y) + yo;
            if (sizeof(T) == 2 && a.y_sc == 1 && full4) {
              *reinterpret_cast<u32x2_t*>(yp) = (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (co + r < a.Cout) yp[r * a.y_sc] = E::from_f(v[r]);
            }
          }
        }
      }
  };
  if constexpr (F8) epilogue(std::integral_constant<int, 2>{});
  else if (a.act == VRS_ACT_SILU) epilogue(std::integral_constant<int, 1>{});
  else epilogue(std::integral_constant<int, 0>{});
}

}  // namespace

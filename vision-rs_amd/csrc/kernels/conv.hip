// Implicit-GEMM Conv2d + folded BatchNorm + SiLU (+ residual) for gfx950.
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
template <typename T, int BM, int BN, int BK, int WGM, int WGN, bool ALIGNED, bool F8 = false, bool UP = false>
__device__ __forceinline__ void conv_body(const vrs_conv_args& a) {
  using E = Elt<T>;
  using G = typename E::group;
  static_assert(!F8 || (sizeof(T) == 2 && BK == 64 && ALIGNED), "fp8: bf16 activations, 64-deep steps");
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
  constexpr int AEL = F8 ? 16 : 8;           // weight elements per chunk
  constexpr int LDKB = BK + 16;              // F8: LDS row stride in bytes (80: conflict-free)
  constexpr int NT = 64 * WGM * WGN;         // threads per workgroup
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int TM = WTM / 32, TN = WTN / 32;   // 32x32 MFMA tiles per wave
  constexpr int A_IT = (BM * GPRA + NT - 1) / NT;
  constexpr int B_IT = (BN * GPR + NT - 1) / NT;
  constexpr bool A_FULL = (BM * GPRA) % NT == 0;   // every thread owns A_IT chunks
  constexpr bool B_FULL = (BN * GPR) % NT == 0;
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
  const T* b_ptr[B_IT];
  bool b_ok[B_IT];
  uint32_t b_off2[B_IT];   // fused upsample: byte offset of the pixel's source in x2
#pragma unroll
  for (int i = 0; i < B_IT; ++i) {
    const int c = tid + i * NT;
    const int m = n0 + c / GPR;
    b_ok[i] = (B_FULL || c < BN * GPR) && (m < a.M);
    const int mm = b_ok[i] ? m : 0;
    int rr, ox;
    const int bb = fdivmod(mm, HWo, inv_hwo, rr);
    const int oy = fdivmod(rr, a.Wo, inv_wo, ox);
    b_iy0[i] = oy * a.stride - a.pad;
    b_ix0[i] = ox * a.stride - a.pad;
    b_ptr[i] = x + (((int64_t)bb * a.H + b_iy0[i]) * a.W + b_ix0[i]) * a.x_pitch + (c % GPR) * 8;
    if constexpr (UP)
      b_off2[i] = b_ok[i] ? (uint32_t)((((int64_t)bb * a.H2 + (oy >> 1)) * a.W2 + (ox >> 1)) * a.x2_pitch + (c % GPR) * 8) *
                                (uint32_t)sizeof(T)
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
    for (int i = 0; i < B_IT; ++i) b_off[i] = (uint32_t)((b_ptr[i] - x) * (int64_t)sizeof(T));
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
        rb[i] = ok ? E::load(b_ptr[i] - grp * 8 + ((int64_t)ky * a.W + kx) * a.x_pitch + ci) : E::zero();
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
      const uint32_t off = (uint32_t)((ky * a.W + kx) * a.x_pitch + t_ci) * sizeof(T);
      const bool lo = UP && t_ci < a.c_split;   // fused upsample: this chunk comes from x2 (uniform)
      const uint32_t off2 = (uint32_t)t_ci * sizeof(T);
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
          const u32x2_t q = {bf16x2_to_fp8x2(v[0], a.clamp_bits, a.in_scale) |
                                 (bf16x2_to_fp8x2(v[1], a.clamp_bits, a.in_scale) << 16),
                             bf16x2_to_fp8x2(v[2], a.clamp_bits, a.in_scale) |
                                 (bf16x2_to_fp8x2(v[3], a.clamp_bits, a.in_scale) << 16)};
          *reinterpret_cast<u32x2_t*>(sB + (c / GPR) * LDKB + (c % GPR) * 8) = q;
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
        i32x8_t fa[TM], fb[TN];
        auto ld32 = [&](const unsigned char* p) {
          const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(p);
          const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(p + 16);
          return (i32x8_t){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        };
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[i] = ld32(sA + (wm * WTM + i * 32 + frag_row) * LDKB + fk);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[j] = ld32(sB + (wn * WTN + j * 32 + frag_row) * LDKB + fk);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma32_fp8_k64(fa[i], fb[j], acc[i][j]);
        pipe_schedule<TM * TN, 2 * (TM + TN), TM * TN, A_IT + B_IT>();
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
    if (a.stage) {
      // Staged store: every wave writes its (WTN pixel x WTM channel) tile to
      // LDS, then stores whole 16-byte channel chunks per lane, so consecutive
      // lanes write contiguous bytes of a pixel's NHWC row.
      constexpr int HW_ = WGM * WGN / 2;
      T* st = sbuf(wave / HW_) + (wave % HW_) * WTN * (WTM + SPAD);
      // the host stages only views addressable with 32-bit byte offsets
      // (y_bytes, res_bytes): pixel m of an NHWC view starts at m * pitch
      const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y, a.y_bytes);
      const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.res, a.res ? a.res_bytes : 0);
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
              const uint32_t ro = m < a.M && co < a.Cout
                                      ? ((uint32_t)m * (uint32_t)a.r_sp + (uint32_t)co) * (uint32_t)sizeof(T)
                                      : kOOB;
              if constexpr (sizeof(T) == 2) {
                const u32x2_t rv = __builtin_amdgcn_raw_buffer_load_b64(rr, ro, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                  v[r] += __uint_as_float((r & 1) ? (rv[r >> 1] & 0xffff0000u) : (rv[r >> 1] << 16));
              } else {
                const u32x4_t rv = __builtin_amdgcn_raw_buffer_load_b128(rr, ro, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] += __uint_as_float(rv[r]);
              }
            }
            T* sp = st + pl * (WTM + SPAD) + cl;
            if constexpr (sizeof(T) == 2) {
              *reinterpret_cast<u32x2_t*>(sp) = (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            } else {
              *reinterpret_cast<f32x4_t*>(sp) = (f32x4_t){v[0], v[1], v[2], v[3]};
            }
          }
        }
      __syncthreads();
      constexpr int EPC = 16 / (int)sizeof(T);  // elements per 16-byte chunk
      constexpr int CPP = WTM / EPC;            // chunks per pixel row
      const int co_w = m0 + wm * WTM;
      static_assert((WTN * CPP) % 64 == 0, "whole store rounds");
#pragma unroll
      for (int s = 0; s < WTN * CPP / 64; ++s) {
        const int c = lane + s * 64;
        const int pl = c / CPP, part = c % CPP;
        const int m = n0 + wn * WTN + pl;
        const int co = co_w + part * EPC;
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(st + pl * (WTM + SPAD) + part * EPC);
        const uint32_t off = m < a.M && co < a.Cout
                                 ? ((uint32_t)m * (uint32_t)a.y_sp + (uint32_t)co) * (uint32_t)sizeof(T)
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
// fp8 e4m3 weights + e4m3-quantised bf16 activations (32x32x64 fp8 MFMA),
// 64-deep steps (Cin % 64 == 0), bf16 outputs
#define VRS_CONV_F8(NAME, BM, BN, WGM, WGN)                                                       \
  extern "C" __global__ __launch_bounds__(64 * WGM * WGN) void NAME(vrs_conv_args a) {          \
    conv_body<bf16_t, BM, BN, 64, WGM, WGN, true, true>(a);                                      \
  }
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

VRS_CONV_F8(vrs_conv_fp8_128x128_k64_a, 128, 128, 2, 2)
VRS_CONV_F8(vrs_conv_fp8_256x128_k64_a, 256, 128, 2, 2)
VRS_CONV_F8(vrs_conv_fp8_128x256_k64_a, 128, 256, 2, 2)
VRS_CONV_F8(vrs_conv_fp8_64x256_k64_a, 64, 256, 1, 4)
// 8 waves (512 threads) of 128x64, as the bf16 256x256 tile
VRS_CONV_F8(vrs_conv_fp8_256x256_k64_a, 256, 256, 2, 4)
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

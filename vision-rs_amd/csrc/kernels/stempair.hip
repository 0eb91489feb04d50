// Stem pair for gfx950: the first two layers of YOLO26 at the m and l widths
// in one kernel -- model.0 = conv(3, 64, 3, 2) and model.1 = conv(64, 128, 3,
// 2) (yolo26/mod.rs:126-195; each blocks/conv.rs:31-46: conv, folded BN,
// SiLU):
//
//   s = bf16(silu(scale0 * conv3x3s2(x, w0) + shift0))     64 channels
//   y = bf16(silu(scale1 * conv3x3s2(s, w1) + shift1))     128 channels
//
// s is the largest activation of the network (four times the pixels of y)
// and here never leaves the chip.  A workgroup (512 threads, one per CU)
// walks a contiguous run of steps; a step is 2 output rows x 32 output
// columns of one image strip, and consecutive steps of a strip move down it.
//
// * ring: the 5 stem rows a step reads (2*32+1 columns x 64 channels, bf16)
//   sit in one of two LDS buffers; during a step the other buffer receives
//   the next step's 4 new stem rows (all 5 at the start of a strip) and a
//   copy of the one row the two steps share.  Columns are stored even ones
//   first, then the odd ones 16 bytes further on, so the stride-2 columns of
//   one model.1 tap are consecutive entries and the stem's row writes do not
//   pair up on banks.
// * The waves split by role, one of each per SIMD, so that one's MFMAs run
//   under the other's VALU work (this kernel has about twice as much VALU
//   work -- two SiLUs per stem value -- as MFMA work):
//   - waves 0-3, model.1: wave cb owns output channels 32cb..32cb+31 of the
//     step's 64 pixels.  Its 32 x 576 weights stay in registers for the whole
//     run (36 bf16x8 A fragments); B fragments are 16-byte LDS reads of the
//     ring; 72 v_mfma_f32_32x32x16_bf16 per step (two 32-pixel rows) in the
//     tap-major, channel-minor K order of the dense conv kernel, so y equals
//     vrs_conv_stem + vrs_conv2d bit for bit.  They also copy the shared
//     ring row.
//   - waves 4-7, stem: the next step's 4 new rows x 64 own columns are 8
//     tiles of 32 pixels, two per wave, on the MFMA (K = 27 taps padded to
//     32, k = c*9 + ky*3 + kx, as in vrs_stem).  These waves also stage the
//     image: 3 channels x 11 rows x 132 columns of float32 per step, loaded
//     two steps ahead into registers and written to LDS one step ahead, and
//     run at a raised wave priority: theirs is the longer dependency chain.
//   - the strip's left halo column is one more stem tile, pixels as rows,
//     split over model.1 waves 2 and 3.
// * One barrier per step.
//
// Out-of-range stem pixels (model.1's zero padding) are stored as zeros;
// image reads outside the picture (the stem's padding) and output stores
// outside y use offsets the buffer resource rejects.
#include "common.h"

namespace {

using E = Elt<bf16_t>;
using G = E::group;

constexpr int NT = 512, NH = 256;       // threads; threads per role
constexpr int C0 = 64, C1 = 128;
constexpr int SW = 32;                  // output columns per strip
constexpr int SC = 2 * SW + 1;          // stem columns a strip reads (65)
constexpr int NR = 5;                   // stem rows a step reads
constexpr int IR = 2 * NR + 1;          // image rows staged for one step (11)
constexpr int IQ = SW + 1;              // float4 chunks per staged image row (33)
constexpr int IC = 4 * IQ;              // image columns staged (132)
constexpr int EP = C0 + 8;              // LDS stem pixel: 64 channels + pad (144 bytes)
constexpr int ODD = 33 * EP + 8;        // first odd column (16 bytes past the even ones)
constexpr int ROW = SC * EP + 8;        // LDS stem row (elements)
constexpr int RING = NR * ROW;          // one ring buffer (elements)
constexpr int IMG = 3 * IR * IC;        // one image buffer (floats)
constexpr int WP = 32 + 8;              // stem weight row in LDS (k + pad)
constexpr int KS = 9 * C0 / 16;         // model.1 K slices of 16 (36)
constexpr int NIMG = 3 * IR * IQ;       // image chunks per step (1089)
constexpr int NLD = (NIMG + NH - 1) / NH;   // image chunks per stem-wave thread (5)
constexpr int NCP = SC * C0 / 8;        // 16-byte chunks of one stem row (520)
static_assert(RING * 2 + IMG * 4 + C0 * WP * 2 + (C0 + C1) * 8 <= 160 * 1024, "LDS");

// LDS element offset of stem column j (0..64) within a ring row
__device__ __forceinline__ int col_off(int j) { return (j & 1) ? ODD + (j >> 1) * EP : (j >> 1) * EP; }

// image buffer offset of tap k of a stem pixel, from the pixel's window origin
// (k >= 27 is padding: offset 0, the value zeroed by the caller)
__device__ constexpr int tap_off(int k) { return k < 27 ? (k / 9 * IR + k % 9 / 3) * IC + k % 3 : 0; }

struct Pos {
  int b, sx, t;
};

// a copy of v the optimiser cannot see through: per-thread values derived
// from it are recomputed where used instead of being hoisted out of the step
// loop (where each would hold a register for the whole run)
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

__device__ __forceinline__ void stem_pair_body(const vrs_stem_pair_args& a) {
  __shared__ __attribute__((aligned(16))) bf16_t ring[2 * RING];
  __shared__ __attribute__((aligned(16))) float img[2 * IMG];
  __shared__ __attribute__((aligned(16))) bf16_t sw0[C0 * WP];
  __shared__ __attribute__((aligned(16))) float bn0[2 * C0];
  __shared__ __attribute__((aligned(16))) float bn1[2 * C1];

  const int tid = threadIdx.x, lane = tid & 63, hq = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q0 = (int)((int64_t)a.total * blockIdx.x / gridDim.x);
  const int n = (int)((int64_t)a.total * (blockIdx.x + 1) / gridDim.x) - q0;
  if (n <= 0) return;   // uniform, before any barrier

  // stem weights and both layers' folded-BN constants -> LDS
  for (int i = tid; i < C0 * 4; i += NT)
    *reinterpret_cast<u32x4_t*>(&sw0[(i >> 2) * WP + (i & 3) * 8]) = reinterpret_cast<const u32x4_t*>(a.w0)[i];
  if (tid < C0) {
    bn0[tid] = a.scale0[tid];
    bn0[C0 + tid] = a.shift0[tid];
  }
  if (tid < C1) {
    bn1[tid] = a.scale1[tid];
    bn1[C1 + tid] = a.shift1[tid];
  }

  auto pos = [&](int s) {
    const int q = q0 + s, r = q / a.sps;
    return Pos{r / a.strips, r % a.strips, q % a.sps};
  };
  // the next step's position without divisions (wave-uniform, scalar)
  auto advance = [&](Pos& p) {
    if (++p.t == a.sps) {
      p.t = 0;
      if (++p.sx == a.strips) {
        p.sx = 0;
        ++p.b;
      }
    }
  };
  // Fragment of stem pixel (ring row rho, column j): lane k group hq,
  // k = ks*16 + hq*8 + e -> image buffer row c*IR + 2rho + ky, column
  // 2j + 1 + kx.
  auto gather = [&](const float* im, int rho, int j, G (&f)[2]) {
    const float* org = im + 2 * rho * IC + 2 * j + 1;
    // offset lo + hz*(hi - lo): lo folds into the LDS instruction's offset,
    // hz (an opaque copy of hq) keeps the product from being hoisted out of
    // the step loop, where a select between two constants per tap would hold
    // registers for the whole run
    const int hz = opaque(hq);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int lo = tap_off(ks * 16 + e), hi = tap_off(ks * 16 + 8 + e);
        v[e] = org[lo + hz * (hi - lo)];
      }
      if (ks == 1 && hz) {
#pragma unroll
        for (int e = 3; e < 8; ++e) v[e] = 0.f;   // k = 27..31
      }
      f[ks] = E::from_f8(v);
    }
  };
  auto wfrag = [&](int ct, int ks) { return E::load(sw0 + (ct * 32 + l32) * WP + ks * 16 + hq * 8); };
  // Left halo column (j = 0) of the stem rows of step u (rows 1..4, or 0..4
  // at the start of a strip), 32-channel half ct: pixels as rows (as
  // vrs_stem), so register r < 4 of lane l is pixel hq*4 + r, channel
  // ct*32 + l32.  Run by model.1 waves 2 and 3.
  auto halo = [&](int u, const Pos& p, int ct) {
    const bool first = u == 0 || p.t == 0;
    const float* im = img + (u & 1) * IMG;
    bf16_t* rg = ring + (u & 1) * RING;
    const int rho0 = first ? 0 : 1, nh = first ? 5 : 4, y0 = 4 * p.t - 1;
    const bool col_ok = p.sx > 0;
    G f[2];
    gather(im, rho0 + (l32 < nh ? l32 : nh - 1), 0, f);
    f32x16_t acc = {};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) acc = mfma32_k16(f[ks], wfrag(ct, ks), acc);
    const int ch = ct * 32 + l32;
    const float sc = bn0[ch], sh = bn0[C0 + ch];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int px = hq * 4 + r;
      if (px < nh) {
        const bool ok = col_ok && (unsigned)(y0 + rho0 + px) < (unsigned)a.H0;
        rg[(rho0 + px) * ROW + ch] = f2bf(ok ? silu_fast(acc[r] * sc + sh) : 0.f);   // col_off(0) = 0
      }
    }
  };
  // positions of steps s (model.1), s + 1 (stem rows) and s + 3 (image loads)
  Pos pc = pos(0), pn = pos(0), pl = pos(n > 2 ? 2 : 0);

  if (wave < 4) {
    // ===================== model.1 role (waves 0-3) ========================
    const int cb = wave;
    // A fragments: output channel 32cb + l32, k = kk*16 + hq*8 .. +7
    G w1[KS];
    {
      const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w1, C1 * 9 * C0 * 2);
      const uint32_t base = (uint32_t)(((cb * 32 + l32) * 9 * C0 + hq * 8) * 2);
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) w1[kk] = E::bload(rw, base, (uint32_t)(kk * 32));
    }
    // ring buffer s & 1, row 4 -> ring buffer (s + 1) & 1, row 0
    auto copy_row = [&](int s) {
      const bf16_t* src = ring + (s & 1) * RING + 4 * ROW;
      bf16_t* dst = ring + ((s + 1) & 1) * RING;
      for (int i = opaque(tid); i < NCP; i += NH) {
        const int o = col_off(i >> 3) + (i & 7) * 8;
        *reinterpret_cast<u32x4_t*>(dst + o) = *reinterpret_cast<const u32x4_t*>(src + o);
      }
    };
    // B fragment of k slice kk = tap*4 + cc for output pixel p of step row
    // pr: ring row 2pr + ky, stem column 2p + kx, channels cc*16 + hq*8 ..
    // +7.  Accumulator register 4g + r: output channel 32cb + g*8 + hq*4 + r
    // of pixel l32 of row pr; stored as 8-byte chunks of 4 channels.
    auto m1_step = [&](int s, const Pos& p) {
      const bf16_t* rb = ring + (s & 1) * RING + l32 * EP + hq * 8;
      f32x16_t acc[2] = {};
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const int tap = kk >> 2, ky = tap / 3, kx = tap % 3;
        const int off = ky * ROW + (kx == 1 ? ODD : kx == 2 ? EP : 0) + (kk & 3) * 16;
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) acc[pr] = mfma32_k16(w1[kk], E::load(rb + 2 * pr * ROW + off), acc[pr]);
      }
      // schedule: PD reads ahead of the MFMAs, then one read per MFMA
      constexpr int PD = 4;
      __builtin_amdgcn_sched_group_barrier(0x100, PD, 0);
#pragma unroll
      for (int m = 0; m < 2 * KS; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (m + PD < 2 * KS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      const int per_image = a.H1 * a.W1 * a.y_pitch;
      const __amdgpu_buffer_rsrc_t ry =
          make_rsrc(reinterpret_cast<bf16_t*>(a.y) + (int64_t)p.b * per_image, per_image * 2);
      const int x1 = SW * p.sx + opaque(l32);
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        const int y1 = 2 * p.t + pr;
        const bool ok = y1 < a.H1 && x1 < a.W1;
        const uint32_t pix = (uint32_t)((y1 * a.W1 + x1) * a.y_pitch + cb * 32 + hq * 4) * 2u;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int co = cb * 32 + g * 8 + hq * 4;
          const f32x4_t sc = *reinterpret_cast<const f32x4_t*>(&bn1[co]);
          const f32x4_t sh = *reinterpret_cast<const f32x4_t*>(&bn1[C1 + co]);
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = silu_fast(acc[pr][g * 4 + r] * sc[r] + sh[r]);
          __builtin_amdgcn_raw_buffer_store_b64((u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])}, ry,
                                                ok ? pix + (uint32_t)g * 16u : kOOB, 0, 0);
        }
      }
    };

    __syncthreads();   // prologue: the stem waves stage step 0's image rows
    for (int s = -1; s < n; ++s) {
      if (s + 1 < n && wave >= 2) halo(s + 1, pn, wave - 2);
      if (s >= 0) {
        if (s + 1 < n && pn.t != 0) copy_row(s);
        m1_step(s, pc);
        advance(pc);
      }
      __syncthreads();
      advance(pn);
    }
    return;
  }

  // ======================= stem role (waves 4-7) ===========================
  // image rows: buffer row ri is image row 8t - 3 + ri, buffer column
  // 4cq..4cq+3 is image column 128sx - 4 + 4cq (W % 4 == 0: a chunk is wholly
  // inside or outside the picture).  Steps after a strip's first need rows
  // 2..10 only.  Chunk i of a step is floats 4i..4i+3 of its buffer.
  f32x4_t pre[NLD];
  auto load_img = [&](int s, const Pos& p) {
    const bool first = s == 0 || p.t == 0;
    const int plane = a.H * a.W;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (int64_t)p.b * 3 * plane, 3 * plane * 4);
    const int iy0 = 8 * p.t - 3, ix0 = 128 * p.sx - 4, t0 = opaque(tid - NH);
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      const int i = t0 + j * NH;
      const int r = i / IQ, cq = i % IQ, c = r / IR, ri = r % IR;
      const int iy = iy0 + ri, ix = ix0 + 4 * cq;
      const bool ok = i < NIMG && (first || ri >= 2) && (unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W;
      const uint32_t off = ok ? (uint32_t)((c * a.H + iy) * a.W + ix) * 4u : kOOB;
      pre[j] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
    }
  };
  auto store_img = [&](int s) {
    float* im = img + (s & 1) * IMG;
    const int t0 = opaque(tid - NH);
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      const int i = t0 + j * NH;
      if (i < NIMG) *reinterpret_cast<f32x4_t*>(&im[4 * i]) = pre[j];
    }
  };

  // the stem's A fragments and this lane's folded-BN constants (channels
  // ct*32 + g*8 + hq*4 .. +3), read from LDS after the prologue's barrier and
  // kept in registers (these waves hold no model.1 weights)
  G wf[2][2];
  f32x4_t bsc[2][4], bsh[2][4];

  // NTL tiles of 32 own columns each, in rows rho, rho + 2, ... of the same
  // columns: weights as rows, so accumulator register 4g + r of lane l is
  // channel ct*32 + g*8 + hq*4 + r of pixel l32.  The tiles go through each
  // phase together (their LDS reads, MFMAs and SiLUs are independent work for
  // one wave).  Stores: the two lanes l and l + 32 of a pixel exchange halves
  // with one v_permlane32_swap per register so that each writes 8 whole
  // channels (16 bytes) -- lane l group 2q + 1, lane l + 32 group 2q.
  auto stem_tiles = [&](auto ntl, const float* im, bf16_t* rg, int rho, int j, int y0, bool col_ok) {
    constexpr int NTL = decltype(ntl)::value;
    G f[NTL][2];
    bool ok[NTL];
#pragma unroll
    for (int t = 0; t < NTL; ++t) {
      gather(im, rho + 2 * t, j, f[t]);
      ok[t] = col_ok && (unsigned)(y0 + rho + 2 * t) < (unsigned)a.H0;
    }
    bf16_t* dst = rg + rho * ROW + col_off(j) + (1 - hq) * 8;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      f32x16_t acc[NTL];
#pragma unroll
      for (int t = 0; t < NTL; ++t) acc[t] = (f32x16_t){};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int t = 0; t < NTL; ++t) acc[t] = mfma32_k16(wf[ct][ks], f[t][ks], acc[t]);
#pragma unroll
      for (int t = 0; t < NTL; ++t)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          uint32_t pk[2][2];   // [g - 2q][half]: 4 channels of group g as two bf16 pairs
#pragma unroll
          for (int gg = 0; gg < 2; ++gg) {
            const int g = 2 * q + gg;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
              v[r] = ok[t] ? silu_fast(acc[t][g * 4 + r] * bsc[ct][g][r] + bsh[ct][g][r]) : 0.f;
            pk[gg][0] = pack_bf16x2(v[0], v[1]);
            pk[gg][1] = pack_bf16x2(v[2], v[3]);
          }
          const auto x0 = __builtin_amdgcn_permlane32_swap(pk[1][0], pk[0][0], false, false);
          const auto x1 = __builtin_amdgcn_permlane32_swap(pk[1][1], pk[0][1], false, false);
          *reinterpret_cast<u32x4_t*>(dst + 2 * t * ROW + ct * 32 + q * 16) = (u32x4_t){x0[0], x1[0], x0[1], x1[1]};
        }
    }
  };
  // the stem rows of step u into ring buffer u & 1 (ring row rho is stem row
  // 4t - 1 + rho): rows 1..4, or 0..4 at the start of a strip
  auto stem_rows = [&](int u, const Pos& p) {
    const bool first = u == 0 || p.t == 0;
    const float* im = img + (u & 1) * IMG;
    bf16_t* rg = ring + (u & 1) * RING;
    const int y0 = 4 * p.t - 1, x0 = 64 * p.sx - 1;
    const int rho0 = first ? 0 : 1, sw = wave - 4;
    // this wave's tiles: sw, sw + 4 (and sw + 8) of the 8 (10) row halves,
    // i.e. rows rho0 + (sw >> 1) + 0, 2 (, 4) of column half sw & 1
    const int j = 1 + 32 * (sw & 1) + opaque(l32), rho = rho0 + (sw >> 1);
    const bool col_ok = (unsigned)(x0 + j) < (unsigned)a.W0;
    if (first && sw < 2) stem_tiles(std::integral_constant<int, 3>{}, im, rg, rho, j, y0, col_ok);
    else stem_tiles(std::integral_constant<int, 2>{}, im, rg, rho, j, y0, col_ok);
  };

  // prologue: step 0's image rows in LDS, step 1's in registers.  These
  // waves' latency chains set the pace: they issue ahead of the model.1
  // waves on their SIMD, whose MFMAs fill the gaps.
  __builtin_amdgcn_s_setprio(3);
  load_img(0, pc);
  store_img(0);
  if (n > 1) {
    Pos p1 = pc;
    advance(p1);
    load_img(1, p1);
  }
  __syncthreads();
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) wf[ct][ks] = wfrag(ct, ks);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      bsc[ct][g] = *reinterpret_cast<const f32x4_t*>(&bn0[ct * 32 + g * 8 + hq * 4]);
      bsh[ct][g] = *reinterpret_cast<const f32x4_t*>(&bn0[C0 + ct * 32 + g * 8 + hq * 4]);
    }
  }
  // iteration s: the stem rows of step s + 1; step s + 2's image rows to LDS,
  // step s + 3's loads issued (the model.1 waves run step s meanwhile)
  for (int s = -1; s < n; ++s) {
    if (s + 1 < n) stem_rows(s + 1, pn);
    if (s + 2 < n) store_img(s + 2);
    if (s + 3 < n) load_img(s + 3, pl);
    __syncthreads();
    advance(pn);
    advance(pl);
  }
}

}  // namespace

extern "C" __global__ __launch_bounds__(NT, 1) void vrs_stem_pair_bf16(vrs_stem_pair_args a) { stem_pair_body(a); }

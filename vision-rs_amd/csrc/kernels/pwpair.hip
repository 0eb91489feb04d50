// Fused pointwise pair for gfx950 (bfloat16 in, float32 out): the last two
// 1x1 convs of a Detect class branch (blocks/detect.rs:117-155: the second
// DWConv -> Conv pair's Conv, then the conv_plain that writes the class
// logits; each blocks/conv.rs:31-46 / :90-99) in one kernel, so the CM-channel
// map between them never goes to memory:
//   m   = bf16(silu(s1 * (W1 . x) + b1))          (C -> CM channels)
//   out = s2 * (W2 . m) + b2                       (CM -> NC channels, float32,
//                                                   channel-major flat layout)
// out[b * sb + p * sp + co * sc] for pixel p of image b, as the flat-output
// conv stores the Detect head's scores.
//
// A workgroup (4 waves) owns 64 consecutive pixels (of the N*H*W pixel rows):
//   * W1 . x: the K loop over C in 32-channel steps, two LDS stages (the
//     W1 slab of all CM rows and the 64 pixel rows of the step's channels,
//     rows padded by 16 bytes) and one register set: step k+1's global loads
//     are issued before step k's MFMAs and written to the other stage after
//     them, one barrier per step.  Wave w computes channels 64w..64w+63 of
//     all 64 pixels (2 x 2 blocks of v_mfma_f32_32x32x16_bf16);
//   * its epilogue (scale, shift, SiLU, bfloat16 rounding as in the conv
//     kernels) writes m as [pixel][CM + 8] rows into the LDS the stages used;
//   * W2 . m: waves 0-2 each own 32 output channels (rows past NC read as
//     zero and are not stored) of both 32-pixel halves; their W2 fragments
//     (32 x CM bf16) are loaded into registers at the start and the B
//     fragments are 16-byte reads of m.  Channel-major stores: the 32 lanes
//     of a half-wave write 32 consecutive pixels of one channel.
// Both K loops take 16-channel slices in increasing order into one
// accumulator per output, as the tiled and weight-stationary 1x1 kernels do,
// and the epilogues round the same way, so the output equals the two
// separate launches bit for bit.  52 KB of LDS: two workgroups per CU.
// Maps of many tiles run the weight-stationary persistent form below
// (vrs_pwpair_w_*), whose W1 never leaves the registers.
#include "common.h"

namespace {

template <int C, int CM>
__device__ __forceinline__ void pwpair_body(const vrs_pwpair_args& a) {
  using E = Elt<bf16_t>;
  using G = E::group;
  constexpr int NT = 256, NP = 64;                 // threads, pixels per workgroup
  constexpr int KS = C / 32;                       // K steps of GEMM 1
  constexpr int ROW1 = 32 + 8;                     // LDS row of a 32-channel slab (elements)
  constexpr int SW = CM * ROW1, SX = NP * ROW1;    // W1 slab, pixel slab (elements)
  constexpr int STAGE = SW + SX;
  constexpr int MROW = CM + 8;                     // LDS row of m (elements)
  constexpr int AREA = 2 * STAGE > NP * MROW ? 2 * STAGE : NP * MROW;
  constexpr int WL = CM * 4 / NT;                  // 16-byte W1 chunks per thread and step
  static_assert(C % 32 == 0 && CM == 256 && KS >= 2 && CM * 4 % NT == 0, "shape");
  static_assert(NP * 4 == NT, "one 16-byte pixel chunk per thread and step");
  static_assert(AREA * 2 + 2 * CM * 4 <= 64 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) bf16_t smem[AREA];
  __shared__ float s1s[CM], b1s[CM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hq = lane >> 5;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int m0 = tile * NP;   // M < 2^31 (host check)

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t rw1 = make_rsrc(a.w1, CM * C * 2);
  const __amdgpu_buffer_rsrc_t rw2 = make_rsrc(a.w2, a.NC * CM * 2);

  // W2 fragments of this wave's 32 output channels (waves 0-2), all K slices:
  // lane row 32w + l32, k = 16s + 8hq .. +7; rows at or past NC read zero
  const bool g2 = wave < 3;
  G w2f[CM / 16];
  if (g2) {
    const uint32_t base = (uint32_t)((wave * 32 + l32) * CM + hq * 8) * 2u;
#pragma unroll
    for (int s = 0; s < CM / 16; ++s) w2f[s] = E::bload(rw2, base, (uint32_t)(s * 32));
  }
  for (int i = tid; i < CM; i += NT) {
    s1s[i] = a.s1[i];
    b1s[i] = a.b1[i];
  }

  // step k's global loads: W1 rows r = tid / 4 + 64j (chunk tid % 4), and
  // pixel tid / 4 (chunk tid % 4); pixels past M read zero
  const int pr = tid >> 2, pc = tid & 3;
  const bool pin = m0 + pr < a.M;
  const uint32_t xoff = pin ? (uint32_t)((m0 + pr) * a.x_pitch + pc * 8) * 2u : kOOB;
  G wreg[WL], xreg;
  auto gload = [&](int k) {
#pragma unroll
    for (int j = 0; j < WL; ++j)
      wreg[j] = E::bload(rw1, (uint32_t)(((pr + 64 * j) * C + k * 32 + pc * 8) * 2), 0);
    xreg = E::bload(rx, xoff, (uint32_t)(k * 64));   // kOOB + k * 64 stays out of range
  };
  auto lstore = [&](int buf) {
    bf16_t* st = smem + buf * STAGE;
#pragma unroll
    for (int j = 0; j < WL; ++j) E::store(st + (pr + 64 * j) * ROW1 + pc * 8, wreg[j]);
    E::store(st + SW + pr * ROW1 + pc * 8, xreg);
  };

  // GEMM 1: wave w, channel blocks cb (rows 64w + 32cb), pixel blocks pb
  f32x16_t acc[2][2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) acc[cb][pb] = (f32x16_t){};
  auto compute = [&](int buf) {
    const bf16_t* st = smem + buf * STAGE;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      G af[2], bfr[2];
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) af[cb] = E::load(st + (wave * 64 + cb * 32 + l32) * ROW1 + s * 16 + hq * 8);
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) bfr[pb] = E::load(st + SW + (pb * 32 + l32) * ROW1 + s * 16 + hq * 8);
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int pb = 0; pb < 2; ++pb) acc[cb][pb] = mfma32_k16(af[cb], bfr[pb], acc[cb][pb]);
    }
  };
  gload(0);
  lstore(0);
  __syncthreads();
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    if (k + 1 < KS) gload(k + 1);
    compute(k & 1);
    if (k + 1 < KS) lstore((k + 1) & 1);
    __syncthreads();
  }

  // GEMM 1 epilogue -> m in LDS ([pixel][CM + 8], bf16): accumulator register
  // 4g + r of lane l is channel 64w + 32cb + 8g + 4hq + r of pixel 32pb + l32
  bf16_t* mid = smem;
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int ch = wave * 64 + cb * 32 + g * 8 + hq * 4;
      float sc[4], sh[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[r] = s1s[ch + r];
        sh[r] = b1s[ch + r];
      }
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = silu_fast(acc[cb][pb][g * 4 + r] * sc[r] + sh[r]);
        *reinterpret_cast<u32x2_t*>(mid + (pb * 32 + l32) * MROW + ch) =
            (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      }
    }
  __syncthreads();
  if (!g2) return;   // after the workgroup's last barrier

  // GEMM 2: output channels 32w + 8g + 4hq + r of pixels 32pb + l32
  f32x16_t o[2] = {};
#pragma unroll
  for (int s = 0; s < CM / 16; ++s)
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) o[pb] = mfma32_k16(w2f[s], E::load(mid + (pb * 32 + l32) * MROW + s * 16 + hq * 8), o[pb]);

  // channel-major float32 stores through a raw buffer over the output
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y, a.y_bytes);
#pragma unroll
  for (int pb = 0; pb < 2; ++pb) {
    const int m = m0 + pb * 32 + l32;
    const bool ok = m < a.M;
    const int b = ok ? m / a.HW : 0, p = ok ? m - b * a.HW : 0;
    const int64_t pix = (int64_t)b * a.y_sb + (int64_t)p * a.y_sp;
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int co = wave * 32 + g * 8 + hq * 4 + r;
        const bool st = ok && co < a.NC;
        const float v = o[pb][g * 4 + r] * a.s2[st ? co : 0] + a.b2[st ? co : 0];
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ry,
                                              st ? (uint32_t)((pix + (int64_t)co * a.y_sc) * 4) : kOOB, 0, 0);
      }
  }
}

typedef __attribute__((address_space(3))) void lds_void_t;

// Weight-stationary persistent form (maps of many tiles): one workgroup of
// 8 waves per CU loops over the tiles t = blockIdx.x + i * gridDim.x.  W1
// stays in registers for the whole run (wave w: rows 32w..32w+31, all 256 k
// -- its A fragments, 64 VGPRs), as do the W2 fragments of the six waves
// that run the second GEMM (output channel block w % 3 of the 32-pixel half
// w / 3; rows past NC read zero), two waves per SIMD so that one's epilogue
// runs under the other's MFMAs.  Each tile's 64 pixel rows are staged one
// tile ahead by direct-to-LDS buffer loads (LDS address M0 + 16 * lane,
// out-of-range offsets fill zeros), chunk c of pixel p at slot 32p + (c ^ (p
// & 31)) so that the B fragment reads of 32 consecutive pixels hit distinct
// banks.  These loads are issued by inline assembly, which the compiler does
// not count: the waits for them are explicit (vmcnt before the stores, the
// only other vector memory operations in the loop), and the barriers are
// bare s_barriers, since the fence of __syncthreads would wait for the loads
// of the next tile too.  Two barriers per tile: after the GEMM 1 epilogue (m
// complete) and after the stores (m read, the next tile staged).
template <int C, int CM>
__device__ __forceinline__ void pwpair_w_body(const vrs_pwpair_args& a) {
  using E = Elt<bf16_t>;
  using Gr = E::group;
  constexpr int NP = 64, NT = 512, NW = NT / 64;
  constexpr int XB = NP * C;                 // one x tile (elements, swizzled chunks)
  constexpr int MROW = CM + 8;
  constexpr int NQ = NP * C / 8 / NT;        // direct-to-LDS loads per lane and tile (4)
  static_assert(C == 256 && CM == 256 && NW * 32 == CM, "shape");
  __shared__ __attribute__((aligned(16))) bf16_t xs[2 * XB];
  __shared__ __attribute__((aligned(16))) bf16_t mid[NP * MROW];
  __shared__ float s1s[CM], b1s[CM], s2s[96], b2s[96];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hq = lane >> 5;
  const int tiles = (a.M + NP - 1) / NP, G = gridDim.x;   // the host launches at most one group per tile

  // W1 fragments: wave rows 32w + l32, k = 16s + 8hq .. +7
  Gr w1f[C / 16];
  {
    const __amdgpu_buffer_rsrc_t rw1 = make_rsrc(a.w1, CM * C * 2);
#pragma unroll
    for (int s = 0; s < C / 16; ++s)
      w1f[s] = E::bload(rw1, (uint32_t)(((wave * 32 + l32) * C + hq * 8) * 2), (uint32_t)(s * 32));
  }
  // GEMM 2 roles: waves 0-5 own output channel block cb2 = w % 3 (rows past
  // NC read zero) of the 32-pixel half pb2 = w / 3; their W2 fragments
  const bool g2 = wave < 6;
  const int cb2 = wave % 3, pb2 = wave / 3;
  Gr w2f[CM / 16];
  if (g2) {
    const __amdgpu_buffer_rsrc_t rw2 = make_rsrc(a.w2, a.NC * CM * 2);
#pragma unroll
    for (int s = 0; s < CM / 16; ++s)
      w2f[s] = E::bload(rw2, (uint32_t)(((cb2 * 32 + l32) * CM + hq * 8) * 2), (uint32_t)(s * 32));
  }
  for (int i = tid; i < CM; i += NT) { s1s[i] = a.s1[i]; b1s[i] = a.b1[i]; }
  for (int i = tid; i < 96; i += NT) {
    s2s[i] = i < a.NC ? a.s2[i] : 0.f;
    b2s[i] = i < a.NC ? a.b2[i] : 0.f;
  }
  const uint64_t xbase = (uint64_t)(uintptr_t)a.x;
  const int base_lo = __builtin_amdgcn_readfirstlane((int)(uint32_t)xbase);
  const int base_hi = __builtin_amdgcn_readfirstlane((int)(uint32_t)(xbase >> 32) & 0xffff);
  const int xbytes = __builtin_amdgcn_readfirstlane(a.x_bytes);
  typedef int i4_t __attribute__((ext_vector_type(4)));
  const i4_t rd = {base_lo, base_hi, xbytes, 0x00020000};
  auto stage = [&](int t, int b) {
    const int m0 = t * NP;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int slot = (wave * NQ + q) * 64 + lane;
      const int p = slot >> 5, c = (slot & 31) ^ (p & 31);
      const uint32_t off = m0 + p < a.M ? (uint32_t)(((m0 + p) * a.x_pitch + c * 8) * 2) : kOOB;
      const uint32_t la = __builtin_amdgcn_readfirstlane(
          (uint32_t)(uintptr_t)(lds_void_t*)(xs + b * XB + (wave * NQ + q) * 64 * 8));
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" :: "s"(la), "v"(off), "s"(rd)
                   : "memory", "m0");
    }
  };
  int t = blockIdx.x;
  stage(t, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y, a.y_bytes);
  for (int it = 0; t < tiles; ++it, t += G) {
    const int cur = it & 1;
    if (t + G < tiles) stage(t + G, cur ^ 1);
    const bf16_t* xb = xs + cur * XB;
    f32x16_t acc[2] = {};
#pragma unroll
    for (int s = 0; s < C / 16; ++s)
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) {
        const int p = pb * 32 + l32, c = 2 * s + hq;
        acc[pb] = mfma32_k16(w1f[s], E::load(xb + (p * 32 + (c ^ (p & 31))) * 8), acc[pb]);
      }
    // GEMM 1 epilogue -> mid: register 4g + r is channel 32w + 8g + 4hq + r
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int ch = wave * 32 + g * 8 + hq * 4;
      float sc[4], sh[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) { sc[r] = s1s[ch + r]; sh[r] = b1s[ch + r]; }
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = silu_fast(acc[pb][g * 4 + r] * sc[r] + sh[r]);
        *reinterpret_cast<u32x2_t*>(mid + (pb * 32 + l32) * MROW + ch) =
            (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (g2) {
      f32x16_t o = {};
#pragma unroll
      for (int s = 0; s < CM / 16; ++s)
        o = mfma32_k16(w2f[s], E::load(mid + (pb2 * 32 + l32) * MROW + s * 16 + hq * 8), o);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the next tile's staging (and earlier stores)
      const int m = t * NP + pb2 * 32 + l32;
      const bool ok = m < a.M;
      const int b = ok ? m / a.HW : 0, p = ok ? m - b * a.HW : 0;
      const int64_t pix = (int64_t)b * a.y_sb + (int64_t)p * a.y_sp;
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int co = cb2 * 32 + g * 8 + hq * 4 + r;
          const bool st = ok && co < a.NC;
          const float v = o[g * 4 + r] * s2s[co] + b2s[co];
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ry,
                                                st ? (uint32_t)((pix + (int64_t)co * a.y_sc) * 4) : kOOB, 0, 0);
        }
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
}

}  // namespace

extern "C" __global__ __launch_bounds__(256, 2) void vrs_pwpair_bf16_c256_m256(vrs_pwpair_args a) {
  pwpair_body<256, 256>(a);
}

extern "C" __global__ __launch_bounds__(512, 1) void vrs_pwpair_w_bf16_c256_m256(vrs_pwpair_args a) {
  pwpair_w_body<256, 256>(a);
}

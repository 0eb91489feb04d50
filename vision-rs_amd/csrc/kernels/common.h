// Device helpers for the gfx950 (CDNA4) kernels: element types, 16-byte
// vector moves, and the 16x16x32 MFMA step shared by conv and attention.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../kargs.h"

typedef uint16_t bf16_t;  // storage type for bfloat16 activations/weights

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2_t;

__device__ __forceinline__ float bf2f(bf16_t v) { return __uint_as_float(((uint32_t)v) << 16); }

typedef __bf16 bf16x2_hw __attribute__((ext_vector_type(2)));
typedef float f32x2_hw __attribute__((ext_vector_type(2)));

// float -> bfloat16, round to nearest even (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }
// Two floats -> packed bfloat16 pair (lo, hi) in one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_hw f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_hw));
}

// q = n / d and r = n % d for 0 <= n < 2^24 and d >= 1 from the float
// reciprocal: n is exact in float and the float quotient is within one of
// the true one, so a single correction step makes it exact.
__device__ __forceinline__ int fdivmod(int n, int d, float inv_d, int& r) {
  int q = (int)((float)n * inv_d);
  r = n - q * d;
  if (r < 0) { --q; r += d; } else if (r >= d) { ++q; r -= d; }
  return q;
}

// SiLU: the bfloat16 path uses the hardware exp2 and reciprocal (v_exp_f32,
// v_rcp_f32, ~1 ulp each -- far below bf16 resolution) instead of an
// IEEE-exact division; the float32 parity path uses expf and a true divide.
__device__ __forceinline__ float silu_fast(float v) {
  const float e = __builtin_amdgcn_exp2f(-v * 1.4426950408889634f);
  return v * __builtin_amdgcn_rcpf(1.0f + e);
}
__device__ __forceinline__ float silu_acc(float v) { return v / (1.0f + expf(-v)); }
template <typename T> __device__ __forceinline__ float silu_t(float v) {
  return sizeof(T) == 4 ? silu_acc(v) : silu_fast(v);
}

// Raw buffer resource over [base, base + bytes): a load whose offset is at or
// past `bytes` returns zeros, so padding/halo lanes need no branch.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
constexpr uint32_t kOOB = 0x80000000u;  // an offset every resource here rejects

// Scalar (SMEM) buffer load of 8 dwords at a wave-uniform byte offset; dwords
// at or past the resource's byte size read 0.
typedef float f32x8_hw __attribute__((ext_vector_type(8)));
typedef int i32x4_hw __attribute__((ext_vector_type(4)));
__device__ f32x8_hw vrs_s_buffer_load_x8(i32x4_hw rsrc, int offset, int aux) __asm("llvm.amdgcn.s.buffer.load.v8f32");

// Per-channel epilogue constants (folded BN scale or shift, n channels) read
// through the scalar cache: one wave-uniform 8-channel group cb..cb+7 per
// load, of which lanes 0-31 keep cb..cb+3 and lanes 32-63 cb+4..cb+7 -- the
// channels of a 32x32 MFMA accumulator quad (hq = lane >> 5).  Channels past
// n read 0.  Per-lane vector loads of the same values cost one vector memory
// instruction per value and made the epilogue the busiest part of the
// memory pipeline.
struct ChanConst {
  i32x4_hw r;
  __device__ __forceinline__ ChanConst(const float* p, int n) {
    const uint64_t b = reinterpret_cast<uint64_t>(p);
    r = (i32x4_hw){(int)(uint32_t)b, (int)(uint32_t)(b >> 32), n * 4, 0x00020000};
  }
  // hi_mask: all ones on lanes 32-63, zero on lanes 0-31 (see upper_half_mask)
  __device__ __forceinline__ void quad(int cb, uint32_t hi_mask, float (&out)[4]) const {
    const f32x8_hw s = vrs_s_buffer_load_x8(r, __builtin_amdgcn_readfirstlane(cb) * 4, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e)   // one v_bfi_b32 per value
      out[e] = __uint_as_float((__float_as_uint(s[4 + e]) & hi_mask) | (__float_as_uint(s[e]) & ~hi_mask));
  }
};
// Lane mask for ChanConst::quad, opaque to the optimiser so the per-lane
// choice stays a bit select (as a known 0/1 choice it is rewritten into a
// dynamic vector index: a compare/select chain per value).
__device__ __forceinline__ uint32_t upper_half_mask() {
  uint32_t m = (threadIdx.x & 32) ? 0xffffffffu : 0u;
  asm volatile("" : "+v"(m));
  return m;
}

// ---- element traits --------------------------------------------------------
// A "group" is 8 consecutive elements along K: the unit one lane feeds into
// the 16x16x32 MFMA step (bf16: one 16-byte register quad; f32: two quads).
template <typename T> struct Elt;

template <> struct Elt<bf16_t> {
  struct group { u32x4_t v; };
  static __device__ __forceinline__ group bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    group g; g.v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0); return g;
  }
  static __device__ __forceinline__ group load(const bf16_t* p) {
    group g; g.v = *reinterpret_cast<const u32x4_t*>(p); return g;
  }
  static __device__ __forceinline__ group zero() { group g; g.v = (u32x4_t){0, 0, 0, 0}; return g; }
  static __device__ __forceinline__ void store(bf16_t* p, const group& g) {
    *reinterpret_cast<u32x4_t*>(p) = g.v;
  }
  static __device__ __forceinline__ float to_f(bf16_t v) { return bf2f(v); }
  static __device__ __forceinline__ bf16_t from_f(float v) { return f2bf(v); }
  static __device__ __forceinline__ group from_f8(const float (&v)[8]) {
    group g;
    g.v = (u32x4_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
    return g;
  }
};

template <> struct Elt<float> {
  struct group { u32x4_t lo, hi; };
  static __device__ __forceinline__ group bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    group g;
    g.lo = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    g.hi = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16u, soff, 0);
    return g;
  }
  static __device__ __forceinline__ group load(const float* p) {
    group g;
    g.lo = *reinterpret_cast<const u32x4_t*>(p);
    g.hi = *reinterpret_cast<const u32x4_t*>(p + 4);
    return g;
  }
  static __device__ __forceinline__ group zero() {
    group g; g.lo = (u32x4_t){0, 0, 0, 0}; g.hi = g.lo; return g;
  }
  static __device__ __forceinline__ group from_f8(const float (&v)[8]) {
    group g;
    g.lo = (u32x4_t){__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
    g.hi = (u32x4_t){__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])};
    return g;
  }
  static __device__ __forceinline__ void store(float* p, const group& g) {
    *reinterpret_cast<u32x4_t*>(p) = g.lo;
    *reinterpret_cast<u32x4_t*>(p + 4) = g.hi;
  }
  static __device__ __forceinline__ float to_f(float v) { return v; }
  static __device__ __forceinline__ float from_f(float v) { return v; }
};

// acc(16x16, fp32) += A(16 x 32) * B(32 x 16).
// Lane l supplies A[row l%16][k (l/16)*8 + j] and B[k (l/16)*8 + j][col l%16],
// j = 0..7, as one group each.  acc lane l holds D[row (l/16)*4 + r][col l%16].
__device__ __forceinline__ f32x4_t mfma_k32(const Elt<bf16_t>::group& a, const Elt<bf16_t>::group& b,
                                            f32x4_t acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a.v),
                                                 __builtin_bit_cast(bf16x8_t, b.v), acc, 0, 0, 0);
}

// f32: eight 16x16x4 steps; step j takes element j of every lane's group, so
// the four lane groups cover k = g*8 + j and all 32 k are summed.
__device__ __forceinline__ f32x4_t mfma_k32(const Elt<float>::group& a, const Elt<float>::group& b,
                                            f32x4_t acc) {
  const float* av0 = reinterpret_cast<const float*>(&a.lo);
  const float* av1 = reinterpret_cast<const float*>(&a.hi);
  const float* bv0 = reinterpret_cast<const float*>(&b.lo);
  const float* bv1 = reinterpret_cast<const float*>(&b.hi);
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av0[j], bv0[j], acc, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av1[j], bv1[j], acc, 0, 0, 0);
  return acc;
}

// 32x32x16 step (the full-rate bf16 MFMA on gfx950: 16x16x32 issues at half
// the flop rate).  Lane l supplies A[row l%32][k (l/32)*8 + j] and
// B[k (l/32)*8 + j][col l%32], j = 0..7, as one group each; accumulator
// register r of lane l holds D[row (r/4)*8 + (l/32)*4 + r%4][col l%32].
__device__ __forceinline__ f32x16_t mfma32_k16(const Elt<bf16_t>::group& a, const Elt<bf16_t>::group& b,
                                               f32x16_t acc) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a.v),
                                                 __builtin_bit_cast(bf16x8_t, b.v), acc, 0, 0, 0);
}

// f32: eight 32x32x2 steps; step j takes element j of every lane's group, so
// the two lane groups cover k = g*8 + j and all 16 k are summed.
__device__ __forceinline__ f32x16_t mfma32_k16(const Elt<float>::group& a, const Elt<float>::group& b,
                                               f32x16_t acc) {
  const float* av0 = reinterpret_cast<const float*>(&a.lo);
  const float* av1 = reinterpret_cast<const float*>(&a.hi);
  const float* bv0 = reinterpret_cast<const float*>(&b.lo);
  const float* bv1 = reinterpret_cast<const float*>(&b.hi);
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av0[j], bv0[j], acc, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av1[j], bv1[j], acc, 0, 0, 0);
  return acc;
}

// 32x32x64 fp8 step: lane l supplies 32 e4m3 bytes of A[row l%32][k (l/32)*32 ..]
// and of B[k ..][col l%32]; block scales fixed at 1.0 (E8M0 0x7f); same
// accumulator layout as the 32x32 bf16 step.
typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8_t;
__device__ __forceinline__ f32x16_t mfma32_fp8_k64(const i32x8_t& a, const i32x8_t& b, f32x16_t acc) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc, 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
}

// Two bfloat16 (one dword) -> two e4m3 bytes: |x| clamped to the bf16 bits
// `lim` (448 * scale), then rne(x / scale) with scale a power of two.
typedef __attribute__((__vector_size__(2 * sizeof(short)))) short i16x2_t;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2_to_fp8x2(uint32_t v, uint32_t lim, float scale) {
  typedef __attribute__((__vector_size__(2 * sizeof(unsigned short)))) unsigned short u16x2_t;
  const u16x2_t mag = __builtin_bit_cast(u16x2_t, v & 0x7fff7fffu);
  const u16x2_t l = __builtin_bit_cast(u16x2_t, lim);
  const u16x2_t m = mag < l ? mag : l;   // v_pk_min_u16
  const uint32_t c = __builtin_bit_cast(uint32_t, m) | (v & 0x80008000u);
  const i16x2_t r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16((i16x2_t){0, 0}, __builtin_bit_cast(bf16x2_t, c), scale, false);
  return (uint32_t)(uint16_t)r[0];
}

// Four e4m3 bytes (element 0 in the low byte) -> floats times step.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void fp8x4_to_f32(uint32_t u, float step, float (&o)[4]) {
  const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(u, false), hi = __builtin_amdgcn_cvt_pk_f32_fp8(u, true);
  o[0] = lo[0] * step; o[1] = lo[1] * step; o[2] = hi[0] * step; o[3] = hi[1] * step;
}

// blockIdx.x -> logical block id so that each XCD (workgroups are dealt
// round-robin over the 8 XCDs) receives a contiguous range of logical ids
// (a bijection on [0, G)): neighbouring tiles -- the Cout tiles of one pixel
// tile, the query blocks of one attention head -- then share that XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int G) {
  const int q = G >> 3, r = G & 7;
  const int xcd = bid & 7, idx = bid >> 3;
  return xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

// Multi-scale deformable attention (RF-DETR decoder cross-attention) for gfx950.
// There is no reference function (the reference has no deformable attention);
// the semantics are the published Deformable-DETR formulation that BASELINE
// config 4 names: for each (b, q, head)
//   out[d] = sum_{l,p} attw[l,p] * bilinear(V_l[:, :, head, d],
//                                           x = (ref_x + off_x) * W_l - 0.5,
//                                           y = (ref_y + off_y) * H_l - 0.5)
// with zero padding outside the map (grid_sample bilinear, zeros,
// align_corners=False).
//
// Gather-bound.  The value tensor [B, S, heads, 32] keeps each (pixel, head)
// row of 32 floats (128 bytes) contiguous; 8 lanes own one head and fetch a
// corner row as 8 x 16-byte loads, so one wave64 serves all 8 heads of one
// query and every corner fetch is a full 128-byte segment per head.  The
// level and point loops are unrolled at compile time (L <= 4, P <= 4 for the
// fast kernel) so all corner fetches of a query are independent loads in
// flight together; sampling locations and weights are read once per lane
// group with 8-byte / 4-byte loads.
#include "common.h"

namespace {

// Sampling coordinate (ref + off) * size - 0.5 as a rounded add, a rounded
// multiply and a rounded subtract -- no fused multiply-add -- so every
// bilinear corner and weight is the one the float32 CPU restatement (built
// with contraction off) computes; a contracted form moves a coordinate by up
// to half an ulp (~4e-6 at the 80-wide level), which shows in the outputs at
// the 1e-4 parity bar.
__device__ __forceinline__ float sample_coord(float r, float o, int n) {
#pragma clang fp contract(off)
  const float loc = r + o;
  const float scaled = loc * (float)n;
  return scaled - 0.5f;
}

template <int L, int P>
__device__ __forceinline__ void msda_body(const vrs_msda_args& a) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int part = (int)(gid & 7);          // which 4 of the 32 channels
  const int64_t bqh = gid >> 3;
  if (bqh >= (int64_t)a.B * a.Q * a.heads) return;
  const int h = (int)(bqh % a.heads);
  const int64_t bq = bqh / a.heads;
  const int b = (int)(bq / a.Q);
  const float rx = a.ref[bq * 2 + 0], ry = a.ref[bq * 2 + 1];
  const int64_t row = (int64_t)a.heads * 32;  // floats per value pixel
  const float* vb = a.value + (int64_t)b * a.S * row + h * 32 + part * 4;
  const int64_t obase = bqh * (L * P);
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int l = 0; l < L; ++l) {
    const int Hl = a.lh[l], Wl = a.lw[l];
    const float* vl = vb + (int64_t)a.lstart[l] * row;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int64_t oi = obase + l * P + p;
      const float2 off = *reinterpret_cast<const float2*>(a.off + 2 * oi);
      const float w = a.attw[oi];
      const float ix = sample_coord(rx, off.x, Wl);
      const float iy = sample_coord(ry, off.y, Hl);
      const float fx = floorf(ix), fy = floorf(iy);
      const int x0 = (int)fx, y0 = (int)fy;
      const float ax1 = ix - fx, ay1 = iy - fy;
      const float ax0 = 1.f - ax1, ay0 = 1.f - ay1;
      const bool xv0 = (unsigned)x0 < (unsigned)Wl, xv1 = (unsigned)(x0 + 1) < (unsigned)Wl;
      const bool yv0 = (unsigned)y0 < (unsigned)Hl, yv1 = (unsigned)(y0 + 1) < (unsigned)Hl;
      const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
      const f32x4_t v00 = (yv0 && xv0) ? *reinterpret_cast<const f32x4_t*>(vl + ((int64_t)y0 * Wl + x0) * row) : z;
      const f32x4_t v01 = (yv0 && xv1) ? *reinterpret_cast<const f32x4_t*>(vl + ((int64_t)y0 * Wl + x0 + 1) * row) : z;
      const f32x4_t v10 = (yv1 && xv0) ? *reinterpret_cast<const f32x4_t*>(vl + ((int64_t)(y0 + 1) * Wl + x0) * row) : z;
      const f32x4_t v11 = (yv1 && xv1) ? *reinterpret_cast<const f32x4_t*>(vl + ((int64_t)(y0 + 1) * Wl + x0 + 1) * row) : z;
      acc += w * (ay0 * (ax0 * v00 + ax1 * v01) + ay1 * (ax0 * v10 + ax1 * v11));
    }
  }
  *reinterpret_cast<f32x4_t*>(a.out + bq * row + h * 32 + part * 4) = acc;
}

// Any L <= 8, P: runtime loops (the shapes the unrolled kernels do not cover).
__device__ __forceinline__ void msda_any(const vrs_msda_args& a) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int part = (int)(gid & 7);
  const int64_t bqh = gid >> 3;
  if (bqh >= (int64_t)a.B * a.Q * a.heads) return;
  const int h = (int)(bqh % a.heads);
  const int64_t bq = bqh / a.heads;
  const int b = (int)(bq / a.Q);
  const float rx = a.ref[bq * 2 + 0], ry = a.ref[bq * 2 + 1];
  const int64_t row = (int64_t)a.heads * 32;
  const float* vb = a.value + (int64_t)b * a.S * row + h * 32 + part * 4;
  const int64_t obase = bqh * a.L * a.P;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int l = 0; l < a.L; ++l) {
    const int Hl = a.lh[l], Wl = a.lw[l];
    const float* vl = vb + (int64_t)a.lstart[l] * row;
    for (int p = 0; p < a.P; ++p) {
      const int64_t oi = obase + l * a.P + p;
      const float ix = sample_coord(rx, a.off[2 * oi], Wl);
      const float iy = sample_coord(ry, a.off[2 * oi + 1], Hl);
      const float w = a.attw[oi];
      const float fx = floorf(ix), fy = floorf(iy);
      const int x0 = (int)fx, y0 = (int)fy;
      const float ax1 = ix - fx, ay1 = iy - fy;
      const float ax0 = 1.f - ax1, ay0 = 1.f - ay1;
      const int xs[2] = {x0, x0 + 1}, ys[2] = {y0, y0 + 1};
      const float wx[2] = {ax0, ax1}, wy[2] = {ay0, ay1};
      for (int cy = 0; cy < 2; ++cy)
        for (int cx = 0; cx < 2; ++cx) {
          if ((unsigned)xs[cx] >= (unsigned)Wl || (unsigned)ys[cy] >= (unsigned)Hl) continue;
          const f32x4_t v = *reinterpret_cast<const f32x4_t*>(vl + ((int64_t)ys[cy] * Wl + xs[cx]) * row);
          acc += (w * wy[cy] * wx[cx]) * v;
        }
    }
  }
  *reinterpret_cast<f32x4_t*>(a.out + bq * row + h * 32 + part * 4) = acc;
}

// L = 4, P = 4 split by level: workgroup = one (b, q), wave = one level, so a
// query's 64 bilinear corner fetches per lane spread over four waves (4x the
// waves in flight of one wave per query); the four partial sums meet in LDS.
// Workgroups are dealt round-robin over the 8 XCDs; the XCD-aware order gives
// each XCD a contiguous run of queries -- whole images at B*Q/8 queries per
// XCD -- so the corner rows one image's queries share are fetched into one
// L2 rather than into all eight.
__device__ __forceinline__ void msda_split_body(const vrs_msda_args& a) {
  constexpr int P = 4;
  __shared__ f32x4_t part[4][64];
  const int lane = threadIdx.x & 63, l = threadIdx.x >> 6;
  const int64_t bq = xcd_remap(blockIdx.x, gridDim.x);
  const int h = lane >> 3, pc = lane & 7;   // head, 4-channel part
  const int b = (int)(bq / a.Q);
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  if (h < a.heads) {
    const float rx = a.ref[bq * 2 + 0], ry = a.ref[bq * 2 + 1];
    const int64_t row = (int64_t)a.heads * 32;
    const float* vl = a.value + ((int64_t)b * a.S + a.lstart[l]) * row + h * 32 + pc * 4;
    const int Hl = a.lh[l], Wl = a.lw[l];
    const int64_t obase = ((bq * a.heads + h) * 4 + l) * P;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int64_t oi = obase + p;
      const float2 off = *reinterpret_cast<const float2*>(a.off + 2 * oi);
      const float w = a.attw[oi];
      const float ix = sample_coord(rx, off.x, Wl);
      const float iy = sample_coord(ry, off.y, Hl);
      const float fx = floorf(ix), fy = floorf(iy);
      const int x0 = (int)fx, y0 = (int)fy;
      const float ax1 = ix - fx, ay1 = iy - fy;
      const float ax0 = 1.f - ax1, ay0 = 1.f - ay1;
      const bool xv0 = (unsigned)x0 < (unsigned)Wl, xv1 = (unsigned)(x0 + 1) < (unsigned)Wl;
      const bool yv0 = (unsigned)y0 < (unsigned)Hl, yv1 = (unsigned)(y0 + 1) < (unsigned)Hl;
      const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
      const f32x4_t v00 = (yv0 && xv0) ? *reinterpret_cast<const f32x4_t*>(vl + ((int64_t)y0 * Wl + x0) * row) : z;
      const f32x4_t v01 = (yv0 && xv1) ? *reinterpret_cast<const f32x4_t*>(vl + ((int64_t)y0 * Wl + x0 + 1) * row) : z;
      const f32x4_t v10 = (yv1 && xv0) ? *reinterpret_cast<const f32x4_t*>(vl + ((int64_t)(y0 + 1) * Wl + x0) * row) : z;
      const f32x4_t v11 =
          (yv1 && xv1) ? *reinterpret_cast<const f32x4_t*>(vl + ((int64_t)(y0 + 1) * Wl + x0 + 1) * row) : z;
      acc += w * (ay0 * (ax0 * v00 + ax1 * v01) + ay1 * (ax0 * v10 + ax1 * v11));
    }
  }
  part[l][lane] = acc;
  __syncthreads();
  if (l == 0 && h < a.heads) {
    const f32x4_t sum = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
    *reinterpret_cast<f32x4_t*>(a.out + bq * (int64_t)a.heads * 32 + h * 32 + pc * 4) = sum;
  }
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void vrs_msda_l4p4_f32(vrs_msda_args a) { msda_body<4, 4>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_msda_l4p4s_f32(vrs_msda_args a) { msda_split_body(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_msda_f32(vrs_msda_args a) { msda_any(a); }

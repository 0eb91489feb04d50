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
// Gather-bound: the value tensor [B, S, heads, 32] keeps each (pixel, head)
// row of 32 floats contiguous, so a corner fetch by the 32 lanes that own a
// head is one 128-byte coalesced segment.  A wave64 serves two heads of the
// same query; the per-sample location/weight loads are wave-uniform per half
// and come from the scalar-broadcast path of the vector cache.
#include "common.h"

extern "C" __global__ __launch_bounds__(256) void vrs_msda_f32(vrs_msda_args a) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int d = (int)(gid & 31);
  const int64_t bqh = gid >> 5;
  if (bqh >= (int64_t)a.B * a.Q * a.heads) return;
  const int h = (int)(bqh % a.heads);
  const int64_t bq = bqh / a.heads;
  const int b = (int)(bq / a.Q);
  const float rx = a.ref[bq * 2 + 0], ry = a.ref[bq * 2 + 1];
  const float* vb = a.value + (int64_t)b * a.S * a.heads * 32 + h * 32 + d;
  const int64_t row = (int64_t)a.heads * 32;  // elements per pixel
  const int64_t obase = bqh * a.L * a.P;
  float acc = 0.f;
  for (int l = 0; l < a.L; ++l) {
    const int Hl = a.lh[l], Wl = a.lw[l];
    const float* vl = vb + (int64_t)a.lstart[l] * row;
    for (int p = 0; p < a.P; ++p) {
      const int64_t oi = obase + l * a.P + p;
      const float lx = rx + a.off[2 * oi + 0];
      const float ly = ry + a.off[2 * oi + 1];
      const float w = a.attw[oi];
      const float ix = lx * (float)Wl - 0.5f;
      const float iy = ly * (float)Hl - 0.5f;
      const float fx = floorf(ix), fy = floorf(iy);
      const int x0 = (int)fx, y0 = (int)fy;
      const float ax1 = ix - fx, ay1 = iy - fy;
      const float ax0 = 1.f - ax1, ay0 = 1.f - ay1;
      const bool xv0 = x0 >= 0 && x0 < Wl, xv1 = x0 + 1 >= 0 && x0 + 1 < Wl;
      const bool yv0 = y0 >= 0 && y0 < Hl, yv1 = y0 + 1 >= 0 && y0 + 1 < Hl;
      float v00 = 0.f, v01 = 0.f, v10 = 0.f, v11 = 0.f;
      if (yv0 && xv0) v00 = vl[((int64_t)y0 * Wl + x0) * row];
      if (yv0 && xv1) v01 = vl[((int64_t)y0 * Wl + x0 + 1) * row];
      if (yv1 && xv0) v10 = vl[((int64_t)(y0 + 1) * Wl + x0) * row];
      if (yv1 && xv1) v11 = vl[((int64_t)(y0 + 1) * Wl + x0 + 1) * row];
      acc += w * (ay0 * (ax0 * v00 + ax1 * v01) + ay1 * (ax0 * v10 + ax1 * v11));
    }
  }
  a.out[bq * row + h * 32 + d] = acc;
}

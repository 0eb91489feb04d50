// fp8 implicit-GEMM conv kernels for gfx950 (BASELINE config 5's second run;
// no reference function -- the layers are blocks/conv.rs:31-99): e4m3
// weights with a per-output-channel step, the 32x32x64 fp8 MFMA, 64-deep K
// steps (Cin % 64 == 0).  Activations in memory are bf16 (quantised to e4m3
// on the layer's step while staged into LDS) or already e4m3 (_x8); outputs
// are bf16 or e4m3 on the output's step (_y8).  The body is conv_body.h's.
#include "conv_body.h"

// LB: workgroups per CU the launch bounds ask for.  Two (2 waves per SIMD)
// for the tiles whose wave tile is 64x64 or whose 8 waves share the CU:
// without it the e4m3-output instances allot a second copy of the
// accumulators on the way out of the K loop.  One for the 128x64 wave tiles
// of 256x128 / 128x256, which spill at two.
#define VRS_CONV_F8(NAME, BM, BN, BK, WGM, WGN, LB, UP, XF8, YF8)                                \
  extern "C" __global__ __launch_bounds__(64 * WGM * WGN, LB) void NAME(vrs_conv_args a) {      \
    conv_body<bf16_t, BM, BN, BK, WGM, WGN, true, true, UP, XF8, YF8>(a);                        \
  }
// kernel names: vrs_conv_fp8_<BM>x<BN>_k<64 | 128: K step>_<a | u: fused
// nearest-2x upsample>[_x8: e4m3 input][_y8: e4m3 output]
#define VRS_CONV_F8_IO(TAG, BM, BN, BK, WGM, WGN, LB, UP, K)                                      \
  VRS_CONV_F8(vrs_conv_fp8_##TAG##_k##BK##_##K, BM, BN, BK, WGM, WGN, LB, UP, false, false)        \
  VRS_CONV_F8(vrs_conv_fp8_##TAG##_k##BK##_##K##_x8, BM, BN, BK, WGM, WGN, LB, UP, true, false)    \
  VRS_CONV_F8(vrs_conv_fp8_##TAG##_k##BK##_##K##_y8, BM, BN, BK, WGM, WGN, LB, UP, false, true)    \
  VRS_CONV_F8(vrs_conv_fp8_##TAG##_k##BK##_##K##_x8_y8, BM, BN, BK, WGM, WGN, LB, UP, true, true)

VRS_CONV_F8_IO(128x128, 128, 128, 64, 2, 2, 2, false, a)
VRS_CONV_F8_IO(256x128, 256, 128, 64, 2, 2, 1, false, a)
VRS_CONV_F8_IO(128x256, 128, 256, 64, 2, 2, 1, false, a)
VRS_CONV_F8_IO(64x256, 64, 256, 64, 1, 4, 2, false, a)
// 8 waves (512 threads) of 128x64, as the bf16 256x256 tile
VRS_CONV_F8_IO(256x256, 256, 256, 64, 2, 4, 1, false, a)
// fused nearest-2x upsample (the neck's Upsample -> Concat -> C3k2 cv1)
VRS_CONV_F8_IO(128x128, 128, 128, 64, 2, 2, 2, true, u)
VRS_CONV_F8_IO(256x128, 256, 128, 64, 2, 2, 1, true, u)
VRS_CONV_F8_IO(128x256, 128, 256, 64, 2, 2, 1, true, u)
VRS_CONV_F8_IO(256x256, 256, 256, 64, 2, 4, 1, true, u)
// 128-deep K steps (Cin % 128 == 0) on the 256x256 tile: two fp8 MFMA k
// slices per LDS stage and barrier (the 3x3/s2 layers: 7-10 % faster than
// 64-deep steps).  e4m3 inputs only (with bf16 inputs the staging registers
// spill).  On 128x128 the 128-deep stages drop the occupancy from three
// workgroups per CU to two and measured equal or slower; 64x256's 92 KB of
// stages leave one workgroup per CU.
VRS_CONV_F8(vrs_conv_fp8_256x256_k128_a_x8, 256, 256, 128, 2, 4, 1, false, true, false)
VRS_CONV_F8(vrs_conv_fp8_256x256_k128_a_x8_y8, 256, 256, 128, 2, 4, 1, false, true, true)

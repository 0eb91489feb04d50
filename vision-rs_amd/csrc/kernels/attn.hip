// PSA attention for gfx950 (blocks/c2psa.rs:61-116 with key_dim 32, head_dim 64).
//
// Reads the qkv conv output directly in NHWC (per head h the channels
// [h*128, +32) are q, [+32, +64) k, [+64, +128) v: the layout psa_pack_qkv
// gathers at kernels/attention/psa.rs:57-94) and writes
//   out[b, n, h*64 + d] = sum_j softmax_j(q_n . k_j * kd^-0.5) v_j[d]
//                        + pe_scale[c] * dw3x3(v)[n, c] + pe_shift[c]
// i.e. flash_attention2_forward (flash_attn2.rs:53-121) for V_lo and V_hi in
// one pass, psa_merge_attn_nchw, psa_extract_v_nchw, the PE depthwise conv_bn
// and the elem_add, fused.
//
// Workgroup = (b, h, block of 64 queries); each wave64 owns 16 queries.
// S^T = K Q^T on MFMA (keys are rows), so each lane holds 4 keys x 1 query and
// softmax row statistics need only two cross-lane steps (xor 16, 32).  The
// probabilities feed O^T += V^T P^T directly from registers: the k-slot order
// of P^T is the lane's natural key order and V^T is read from LDS in that same
// order.  K/V are streamed through LDS 64 keys at a time.
#include "common.h"

namespace {
constexpr int QB = 64;     // queries per workgroup
constexpr int KC = 64;     // keys per LDS chunk
constexpr int KD = 32, VD = 64;

template <typename T>
__device__ __forceinline__ void attn_body(const vrs_attn_args& a) {
  using E = Elt<T>;
  using G = typename E::group;
  constexpr int LDK = KD + 16 / (int)sizeof(T) * 2;   // padded K row
  constexpr int LDV = KC + 16 / (int)sizeof(T);       // padded V^T row
  __shared__ __attribute__((aligned(16))) T sK[KC * LDK];
  __shared__ __attribute__((aligned(16))) T sVt[VD * LDV];

  const int N = a.H * a.W;
  const int qblk = blockIdx.x % a.q_blocks;
  const int bh = blockIdx.x / a.q_blocks;
  const int h = bh % a.heads, b = bh / a.heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lq = lane & 15, lg = lane >> 4;

  const T* qkv = reinterpret_cast<const T*>(a.qkv);
  const int64_t img = (int64_t)b * N;
  const int hc = h * (2 * KD + VD);

  // B operand Q^T: lane holds q[query lq][lg*8 .. +8]
  const int qn = qblk * QB + wave * 16 + lq;
  G qf = qn < N ? E::load(qkv + (img + qn) * a.qkv_pitch + hc + lg * 8) : E::zero();

  f32x4_t o[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) o[t] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_part = 0.f;

  for (int kc = 0; kc < N; kc += KC) {
    __syncthreads();
    {  // K chunk: 64 keys x 4 groups, one group per thread
      const int key = tid >> 2, g = tid & 3;
      const int n = kc + key;
      G v = n < N ? E::load(qkv + (img + n) * a.qkv_pitch + hc + KD + g * 8) : E::zero();
      E::store(&sK[key * LDK + g * 8], v);
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {  // V chunk transposed: 64 keys x 8 groups
      const int c = tid + it * 256;
      const int key = c >> 3, dg = c & 7;
      const int n = kc + key;
      G v = n < N ? E::load(qkv + (img + n) * a.qkv_pitch + hc + 2 * KD + dg * 8) : E::zero();
      const T* ev = reinterpret_cast<const T*>(&v);
#pragma unroll
      for (int j = 0; j < 8; ++j) sVt[(dg * 8 + j) * LDV + key] = ev[j];
    }
    __syncthreads();

    // S^T for 4 key tiles of 16
    f32x4_t s[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      G kf = E::load(&sK[(t * 16 + lq) * LDK + lg * 8]);
      s[t] = mfma_k32(kf, qf, (f32x4_t){0.f, 0.f, 0.f, 0.f});
    }
    float cmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kc + t * 16 + lg * 4 + r;
        float v = s[t][r] * a.scale_log2e;
        v = key < N ? v : -INFINITY;
        s[t][r] = v;
        cmax = fmaxf(cmax, v);
      }
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
    const float m_new = fmaxf(m_run, cmax);
    const float alpha = exp2f(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = exp2f(s[t][r] - m_new);
        s[t][r] = p;
        psum += p;
      }
    l_part = l_part * alpha + psum;
#pragma unroll
    for (int t = 0; t < 4; ++t) o[t] *= alpha;

    // O^T += V^T P^T, two k-steps of 32 keys (tiles 2kk, 2kk+1)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      G pf;
      T* pv = reinterpret_cast<T*>(&pf);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pv[r] = E::from_f(s[2 * kk][r]);
        pv[4 + r] = E::from_f(s[2 * kk + 1][r]);
      }
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const T* vrow = &sVt[(dt * 16 + lq) * LDV + kk * 32 + lg * 4];
        G vf;
        T* vv = reinterpret_cast<T*>(&vf);
#pragma unroll
        for (int r = 0; r < 4; ++r) { vv[r] = vrow[r]; vv[4 + r] = vrow[16 + r]; }
        o[dt] = mfma_k32(vf, pf, o[dt]);
      }
    }
  }

  float l_tot = l_part;
  l_tot += __shfl_xor(l_tot, 16);
  l_tot += __shfl_xor(l_tot, 32);
  if (qn >= N) return;
  const float inv = 1.f / l_tot;

  // Fused PE: depthwise 3x3 on V (pad 1) + folded BN, added to the attention.
  const int qy = qn / a.W, qx = qn - qy * a.W;
  T* out = reinterpret_cast<T*>(a.out) + (img + qn) * a.out_pitch + h * VD;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    const int d0 = dt * 16 + lg * 4;
    const int c0 = h * VD + d0;
    float pe[4] = {0.f, 0.f, 0.f, 0.f};
    for (int ky = 0; ky < 3; ++ky) {
      const int yy = qy + ky - 1;
      if (yy < 0 || yy >= a.H) continue;
      for (int kx = 0; kx < 3; ++kx) {
        const int xx = qx + kx - 1;
        if (xx < 0 || xx >= a.W) continue;
        const T* vp = qkv + (img + yy * a.W + xx) * a.qkv_pitch + hc + 2 * KD + d0;
        const T* wk = reinterpret_cast<const T*>(a.pe_w) + (ky * 3 + kx) * (a.heads * VD) + c0;
#pragma unroll
        for (int r = 0; r < 4; ++r) pe[r] += E::to_f(wk[r]) * E::to_f(vp[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
      out[d0 + r] = E::from_f(o[dt][r] * inv + pe[r] * a.pe_scale[c0 + r] + a.pe_shift[c0 + r]);
  }
}
}  // namespace

extern "C" __global__ __launch_bounds__(256) void vrs_psa_attn_bf16(vrs_attn_args a) { attn_body<bf16_t>(a); }
extern "C" __global__ __launch_bounds__(256) void vrs_psa_attn_f32(vrs_attn_args a) { attn_body<float>(a); }

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
// Workgroup = (b, h, block of QW*16 queries); each wave64 owns 16 queries.
// S^T = K Q^T on MFMA (keys are rows), so each lane holds 4 keys x 1 query and
// softmax row statistics need only two cross-lane steps (xor 16, 32: one
// v_permlane swap each).  The probabilities feed O^T += V^T P^T straight
// from registers: the k-slot order
// of P^T is the lane's natural key order and V^T is read from LDS in that same
// order.  K and V^T are streamed through double-buffered LDS 64 keys at a
// time (one barrier per chunk); V^T is written as packed key pairs so the
// transposing store is free of bank conflicts.
#include "common.h"

namespace {
constexpr int KC = 64;     // keys per LDS chunk
constexpr int KD = 32, VD = 64;

// x combined with the value of lane ^ 16 (SPAN 16) or lane ^ 32 (SPAN 32) by
// one v_permlane16/32_swap (a VALU op; __shfl_xor goes through the LDS
// crossbar).  The swap returns this lane's value and its partner's in an
// order that depends on the lane, so only symmetric combinations are formed:
// fmaxf and + give the same bits whichever operand comes first.
template <int SPAN>
__device__ __forceinline__ float xor_max(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = SPAN == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                            : __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
template <int SPAN>
__device__ __forceinline__ float xor_sum(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = SPAN == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                            : __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <typename T, int QW>
__device__ __forceinline__ void attn_body(const vrs_attn_args& a) {
  using E = Elt<T>;
  using G = typename E::group;
  constexpr int NT = QW * 64;
  constexpr int LDK = KD + 16 / (int)sizeof(T) * 2;   // padded K row (elements)
  constexpr int LDV = KC + 16 / (int)sizeof(T);       // padded V^T row (elements)
  constexpr int BUF = KC * LDK + VD * LDV;
  __shared__ __attribute__((aligned(16))) T smem[2 * BUF];

  const int N = a.H * a.W;
  // the q_blocks workgroups of one (b, h) read the same K and V: keep them
  // on one XCD so the re-reads hit its L2
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int qblk = logical % a.q_blocks;
  const int bh = logical / a.q_blocks;
  const int h = bh % a.heads, b = bh / a.heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lq = lane & 15, lg = lane >> 4;

  const T* qkv = reinterpret_cast<const T*>(a.qkv);
  const int64_t img = (int64_t)b * N;
  const int hc = h * (2 * KD + VD);

  // B operand Q^T: lane holds q[query lq][lg*8 .. +8]
  const int qn = qblk * (QW * 16) + wave * 16 + lq;
  G qf = qn < N ? E::load(qkv + (img + qn) * a.qkv_pitch + hc + lg * 8) : E::zero();

  // Stage one chunk of K (row-major) and V^T (transposed) into buffer `buf`.
  auto stage = [&](int kc, int buf) {
    T* sK = smem + buf * BUF;
    T* sVt = sK + KC * LDK;
    for (int c = tid; c < KC * 4; c += NT) {  // K: 64 keys x 4 groups of 8
      const int key = c >> 2, g = c & 3;
      const int n = kc + key;
      E::store(&sK[key * LDK + g * 8], n < N ? E::load(qkv + (img + n) * a.qkv_pitch + hc + KD + g * 8) : E::zero());
    }
    for (int c = tid; c < (KC / 2) * 8; c += NT) {  // V^T: 32 key pairs x 8 channel groups
      const int kp = c & 31, dg = c >> 5;
      const int n0 = kc + 2 * kp;
      const T* vp = qkv + (img + n0) * a.qkv_pitch + hc + 2 * KD + dg * 8;
      G v0 = n0 < N ? E::load(vp) : E::zero();
      G v1 = n0 + 1 < N ? E::load(vp + a.qkv_pitch) : E::zero();
      const T* e0 = reinterpret_cast<const T*>(&v0);
      const T* e1 = reinterpret_cast<const T*>(&v1);
#pragma unroll
      for (int j = 0; j < 8; ++j) {  // one 4-byte (bf16) / 8-byte (f32) store per key pair
        T* dst = &sVt[(dg * 8 + j) * LDV + 2 * kp];
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<uint32_t*>(dst) =
              (uint32_t)__builtin_bit_cast(uint16_t, e0[j]) | ((uint32_t)__builtin_bit_cast(uint16_t, e1[j]) << 16);
        } else {
          *reinterpret_cast<u32x2_t*>(dst) = (u32x2_t){__builtin_bit_cast(uint32_t, e0[j]), __builtin_bit_cast(uint32_t, e1[j])};
        }
      }
    }
  };

  f32x4_t o[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) o[t] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_part = 0.f;

  const int nchunks = (N + KC - 1) / KC;
  stage(0, 0);
  __syncthreads();
  for (int ci = 0; ci < nchunks; ++ci) {
    const int kc = ci * KC;
    const T* sK = smem + (ci & 1) * BUF;
    const T* sVt = sK + KC * LDK;
    if (ci + 1 < nchunks) stage(kc + KC, (ci + 1) & 1);  // overlaps this chunk's math

    // S^T for 4 key tiles of 16
    f32x4_t s[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      G kf = E::load(&sK[(t * 16 + lq) * LDK + lg * 8]);
      s[t] = mfma_k32(kf, qf, (f32x4_t){0.f, 0.f, 0.f, 0.f});
    }
    float cmax = -INFINITY;
    const bool tail = kc + KC > N;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = s[t][r] * a.scale_log2e;
        if (tail && kc + t * 16 + lg * 4 + r >= N) v = -INFINITY;
        s[t][r] = v;
        cmax = fmaxf(cmax, v);
      }
    cmax = xor_max<16>(cmax);
    cmax = xor_max<32>(cmax);
    const float m_new = fmaxf(m_run, cmax);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = __builtin_amdgcn_exp2f(s[t][r] - m_new);
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
      if constexpr (sizeof(T) == 2) {
        u32x4_t pv = {pack_bf16x2(s[2 * kk][0], s[2 * kk][1]), pack_bf16x2(s[2 * kk][2], s[2 * kk][3]),
                      pack_bf16x2(s[2 * kk + 1][0], s[2 * kk + 1][1]), pack_bf16x2(s[2 * kk + 1][2], s[2 * kk + 1][3])};
        pf = *reinterpret_cast<G*>(&pv);
      } else {
        T* pv = reinterpret_cast<T*>(&pf);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pv[r] = E::from_f(s[2 * kk][r]);
          pv[4 + r] = E::from_f(s[2 * kk + 1][r]);
        }
      }
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const T* vrow = &sVt[(dt * 16 + lq) * LDV + kk * 32 + lg * 4];
        G vf;
        if constexpr (sizeof(T) == 2) {
          const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(vrow);
          const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(vrow + 16);
          u32x4_t vv = {lo[0], lo[1], hi[0], hi[1]};
          vf = *reinterpret_cast<G*>(&vv);
        } else {
          T* vv = reinterpret_cast<T*>(&vf);
#pragma unroll
          for (int r = 0; r < 4; ++r) { vv[r] = vrow[r]; vv[4 + r] = vrow[16 + r]; }
        }
        o[dt] = mfma_k32(vf, pf, o[dt]);
      }
    }
    __syncthreads();  // next chunk staged; this chunk's buffer is free
  }

  float l_tot = xor_sum<16>(l_part);
  l_tot = xor_sum<32>(l_tot);
  if (qn >= N) return;
  const float inv = 1.f / l_tot;

  // Fused PE: depthwise 3x3 on V (pad 1) + folded BN, added to the attention.
  const int qy = qn / a.W, qx = qn - qy * a.W;
  const int C = a.heads * VD;
  T* out = reinterpret_cast<T*>(a.out) + (img + qn) * a.out_pitch + h * VD;
  const T* wpe = reinterpret_cast<const T*>(a.pe_w);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    const int d0 = dt * 16 + lg * 4;
    const int c0 = h * VD + d0;
    // the nine taps' V and weight loads all go out before the sums (taps
    // outside the map load the query's own V and are masked), then the sums
    // run in tap order over the taps inside the map
    using L = typename std::conditional<sizeof(T) == 2, u32x2_t, f32x4_t>::type;
    L vv[9], ww[9];
    bool ok[9];
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      const int yy = qy + t / 3 - 1, xx = qx + t % 3 - 1;
      ok[t] = (unsigned)yy < (unsigned)a.H && (unsigned)xx < (unsigned)a.W;
      const int pix = ok[t] ? yy * a.W + xx : qn;
      vv[t] = *reinterpret_cast<const L*>(qkv + (img + pix) * a.qkv_pitch + hc + 2 * KD + d0);
      ww[t] = *reinterpret_cast<const L*>(wpe + t * C + c0);
    }
    float pe[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      if (!ok[t]) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (sizeof(T) == 2) {
          const uint32_t vw = vv[t][r >> 1] >> (16 * (r & 1)), wwv = ww[t][r >> 1] >> (16 * (r & 1));
          pe[r] += bf2f((bf16_t)wwv) * bf2f((bf16_t)vw);
        } else {
          pe[r] += ww[t][r] * vv[t][r];
        }
      }
    }
    float res[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) res[r] = o[dt][r] * inv + pe[r] * a.pe_scale[c0 + r] + a.pe_shift[c0 + r];
    if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<u32x2_t*>(out + d0) = (u32x2_t){pack_bf16x2(res[0], res[1]), pack_bf16x2(res[2], res[3])};
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) out[d0 + r] = E::from_f(res[r]);
    }
  }
}
}  // namespace

// 5 waves x 16 queries: N = 400 (a 20x20 map) is exactly 5 workgroups per head.
extern "C" __global__ __launch_bounds__(320) void vrs_psa_attn_bf16(vrs_attn_args a) { attn_body<bf16_t, 5>(a); }
extern "C" __global__ __launch_bounds__(320) void vrs_psa_attn_f32(vrs_attn_args a) { attn_body<float, 5>(a); }

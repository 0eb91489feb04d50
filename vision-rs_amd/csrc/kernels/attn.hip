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

// ---------------------------------------------------------------------------
// Resident-head attention, bfloat16, N <= 512 keys (every PSA map of YOLO26 at
// 640: 20x20).  Workgroup = (b, h, QT query tiles of 32), one wave per query
// tile.  The head's K ([key][kd], 80-byte rows) and V ([key][d], 128-byte rows,
// 16-byte chunks XOR-swizzled by key) are staged into LDS once; every wave then
// walks all key tiles with no further barrier:
//   S^T(32 keys x 32 queries) = K_tile Q^T            2 x v_mfma 32x32x16
//   p = exp2(s * c - m * c)   (c = kd^-0.5 log2 e)   one FMA + v_exp per score
//   O^T(64 x 32) += V^T_tile P^T                      4 x v_mfma 32x32x16
//   l(1 x 32)    += 1 P^T                             2 x v_mfma (ones row)
// The next tile's S^T MFMAs are issued before this tile's softmax, so the
// matrix core works while the VALU does the exponentials.  Each lane holds 16
// keys x 1 query of S^T, so a query's running max needs one cross-lane step
// (lanes l, l^32); it is updated lazily: a key tile rescales O only when some
// query's tile max exceeds its running max by more than 2^8 (p <= 256 in
// between), so after the first tile rescales are rare.  l accumulates exactly
// the bf16 probabilities the PV MFMAs consume (a ones row as A operand), so
// the rounding of a dominant probability cancels in O / l.
// P^T's k slots follow the accumulator's key order (lane half hh holds keys
// 4hh..4hh+3 and 8+4hh..8+4hh+3 of each 16); the V^T operand in that order
// comes straight from the row-major V with ds_read_b64_tr_b16 (per 16-lane
// group, lane i receives element i % 4 of the 4 values lane 4j + i / 4 read:
// a 4-key x 16-channel block transposed).
// Epilogue, per piece of the head's channels (32 with 7 waves, else 16): the
// waves park O/l (f32) in the LDS freed by K; each thread then takes (query,
// 8 channels) and computes the PE depthwise 3x3 on V from LDS, two taps per
// v_dot2_f32_bf16 (tap-paired weights staged as bf16 pairs; taps outside the
// map read a zero row), adds O/l and the PE's folded BN and stores 16 bytes.
namespace {
constexpr int RN_MAX = 512;             // keys held in LDS
constexpr int RK_LD = 40;               // K row: 32 kd + 8 pad (80 B: conflict-free 16-byte reads)
constexpr int RV_LD = 64;               // V row (128 B), chunks swizzled by vswz(key)
constexpr float R_TAU = 8.0f;           // lazy rescale threshold (log2 units)

// 16-byte chunk c (channels 8c..8c+7) of V row `key` sits at chunk c ^ vswz(key):
// the four rows one transposed read spans then cover distinct LDS banks.
__device__ __forceinline__ int vswz(int key) { return ((key >> 1) & 1) * 4; }
__device__ __forceinline__ int vidx(int key, int d) { return key * RV_LD + (((d >> 3) ^ vswz(key)) << 3) + (d & 7); }

typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x2_t lds_read_tr16(const bf16_t* p) {
  const v4i16_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16_t*)(p));
  return __builtin_bit_cast(u32x2_t, r);
}
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v_t, a), __builtin_bit_cast(bf16x2v_t, b), c, false);
}

template <int QT>
__device__ __forceinline__ void attn_resident_body(const vrs_attn_args& a) {
  constexpr int NT = QT * 64;
  constexpr int PD = QT <= 8 ? 32 : 16;            // epilogue channel piece
  constexpr int RO_LD = PD + 4;                     // parked O row (f32)
  static_assert(QT * 32 * RO_LD * 4 <= RN_MAX * RK_LD * 2, "parked O must fit the K region");
  __shared__ __attribute__((aligned(16))) bf16_t sK[RN_MAX * RK_LD];       // later: parked O
  __shared__ __attribute__((aligned(16))) bf16_t sV[(RN_MAX + 1) * RV_LD]; // + a zero row
  __shared__ __attribute__((aligned(16))) uint32_t sWp[5 * 64];            // PE tap pairs (bf16 x2)
  __shared__ float sScale[64], sShift[64];
  float* sO = reinterpret_cast<float*>(sK);

  const int N = a.H * a.W;
  const int NK = (N + 31) & ~31;
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int qblk = logical % a.q_blocks;
  const int bh = logical / a.q_blocks;
  const int h = bh % a.heads, b = bh / a.heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  const int64_t img = (int64_t)b * N;
  const int hc = h * 128;
  const int C = a.heads * 64;
  const int q0 = qblk * QT * 32;        // first query of this workgroup

  // ---- stage K, V (zero beyond N) and the PE constants ---------------------
  // Raw buffer loads (offsets past the buffer, used for keys >= N, read 0):
  // every load of a thread is issued before its first LDS store.
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qkv, a.qkv_bytes);
  const uint32_t rowb = (uint32_t)a.qkv_pitch * 2u;
  constexpr int KI = (RN_MAX * 4 + NT - 1) / NT;   // K items (key, 16-byte chunk) per thread
  constexpr int VI = (RN_MAX * 8 + NT - 1) / NT;   // V items per thread
  u32x4_t kreg[KI], vreg[VI];
#pragma unroll
  for (int i = 0; i < KI; ++i) {
    const int it = tid + i * NT, key = it >> 2;
    kreg[i] = __builtin_amdgcn_raw_buffer_load_b128(
        rq, key < N ? (uint32_t)(img + key) * rowb + (uint32_t)(hc + 32 + (it & 3) * 8) * 2u : kOOB, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < VI; ++i) {
    const int it = tid + i * NT, key = it >> 3;
    vreg[i] = __builtin_amdgcn_raw_buffer_load_b128(
        rq, key < N ? (uint32_t)(img + key) * rowb + (uint32_t)(hc + 64 + (it & 7) * 8) * 2u : kOOB, 0, 0);
  }
  {
    const bf16_t* wpe = reinterpret_cast<const bf16_t*>(a.pe_w);   // tap-major [9][C]
    for (int it = tid; it < 5 * 64; it += NT) {
      const int pr = it >> 6, d = it & 63;
      const uint32_t w0 = wpe[(2 * pr) * C + h * 64 + d];
      const uint32_t w1 = pr < 4 ? wpe[(2 * pr + 1) * C + h * 64 + d] : 0u;
      sWp[it] = w0 | (w1 << 16);
    }
    for (int it = tid; it < 64; it += NT) {
      sScale[it] = a.pe_scale[h * 64 + it];
      sShift[it] = a.pe_shift[h * 64 + it];
    }
    for (int it = tid; it < RV_LD / 8; it += NT)   // the zero row read by taps outside the map
      *reinterpret_cast<u32x4_t*>(sV + NK * RV_LD + it * 8) = (u32x4_t){0, 0, 0, 0};
  }
#pragma unroll
  for (int i = 0; i < KI; ++i) {
    const int it = tid + i * NT;
    if (it < NK * 4) *reinterpret_cast<u32x4_t*>(sK + (it >> 2) * RK_LD + (it & 3) * 8) = kreg[i];
  }
#pragma unroll
  for (int i = 0; i < VI; ++i) {
    const int it = tid + i * NT, key = it >> 3;
    if (it < NK * 8) *reinterpret_cast<u32x4_t*>(sV + vidx(key, (it & 7) * 8)) = vreg[i];
  }

  // ---- this wave's 32 queries: Q^T fragments (B operand) ----------------
  const int qn = q0 + wave * 32 + l32;
  Elt<bf16_t>::group qf[2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
    qf[s].v = __builtin_amdgcn_raw_buffer_load_b128(
        rq, qn < N ? (uint32_t)(img + qn) * rowb + (uint32_t)(hc + s * 16 + hh * 8) * 2u : kOOB, 0, 0);
  __syncthreads();

  // o[0], o[1]: O^T channels 0-31, 32-63; o[2] row 0: l (ones-row MFMA)
  f32x16_t o[3];
#pragma unroll
  for (int dt = 0; dt < 3; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
  Elt<bf16_t>::group ones;   // A[row 0][k] = 1 (lanes 0 and 32), other rows 0
  {
    const uint32_t one2 = l32 == 0 ? 0x3f803f80u : 0u;
    ones.v = (u32x4_t){one2, one2, one2, one2};
  }
  // transposed-read sources of this lane for the V^T operand: group G = lane/16
  // covers channels D0 + 0..15 (D0 = (G % 2) * 16 within a 32-channel tile)
  // and keys 4hh + 0..3 (+8 for the second read) of each 16-key step
  const int gi = lane & 15;
  const int vt_key = 4 * hh + (gi >> 2);
  const int vt_d = ((lane >> 4) & 1) * 16 + 4 * (gi & 3);
  float m_run = -INFINITY;
  const float c = a.scale_log2e;
  const float tau = R_TAU / c;              // threshold in raw score units
  const bool active = q0 + wave * 32 < N;   // waves past the last query skip the loop
  const int ntiles = NK / 32;
  auto scores = [&](int kt) {
    f32x16_t s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const Elt<bf16_t>::group kf = Elt<bf16_t>::load(sK + (kt * 32 + l32) * RK_LD + ks * 16 + hh * 8);
      s = mfma32_k16(kf, qf[ks], s);
    }
    return s;
  };
  if (active) {
    f32x16_t s = scores(0);
    for (int kt = 0; kt < ntiles; ++kt) {
      f32x16_t s_next;
      if (kt + 1 < ntiles) s_next = scores(kt + 1);   // in flight during this tile's softmax
      // key of register r: kt*32 + (r/4)*8 + hh*4 + r%4
      if (kt * 32 + 32 > N) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kt * 32 + (r >> 2) * 8 + hh * 4 + (r & 3) >= N) s[r] = -INFINITY;
      }
      float tmax = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) tmax = fmaxf(tmax, s[r]);
      tmax = xor_max<32>(tmax);
      if (kt == 0) {
        m_run = tmax;
      } else if (__any(tmax > m_run + tau)) {   // wave-uniform: rescale every lane (alpha 1 where unchanged)
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c);
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < 3; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
      }
      const float mc = m_run * c;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c, -mc));
      // P^T k-step t (16 keys): registers 8t..8t+7
      Elt<bf16_t>::group pf[2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
        pf[t].v = (u32x4_t){pack_bf16x2(s[8 * t + 0], s[8 * t + 1]), pack_bf16x2(s[8 * t + 2], s[8 * t + 3]),
                            pack_bf16x2(s[8 * t + 4], s[8 * t + 5]), pack_bf16x2(s[8 * t + 6], s[8 * t + 7])};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int key = kt * 32 + t * 16 + vt_key;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          const u32x2_t lo = lds_read_tr16(sV + vidx(key, dt * 32 + vt_d));
          const u32x2_t hi = lds_read_tr16(sV + vidx(key + 8, dt * 32 + vt_d));
          Elt<bf16_t>::group vf;
          vf.v = (u32x4_t){lo[0], lo[1], hi[0], hi[1]};
          o[dt] = mfma32_k16(vf, pf[t], o[dt]);
        }
        o[2] = mfma32_k16(ones, pf[t], o[2]);
      }
      if (kt + 1 < ntiles) s = s_next;
    }
  }
  // row 0 of o[2] (register 0 of lanes 0-31) is l of query l32
  const float l_tot = __shfl(o[2][0], l32);
  const float inv = active ? 1.f / l_tot : 0.f;

  // ---- epilogue, one channel piece of the head at a time -------------------
#pragma unroll
  for (int pc = 0; pc < 64 / PD; ++pc) {
    __syncthreads();   // K (first piece) or the previous piece's parked O no longer read
    // O^T register r of o[dt]: channel dt*32 + (r/4)*8 + hh*4 + r%4, query l32
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = dt * 32 + g * 8;
        if (d < pc * PD || d >= pc * PD + PD) continue;   // compile-time after unrolling
        const f32x4_t v = {o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv,
                           o[dt][4 * g + 3] * inv};
        *reinterpret_cast<f32x4_t*>(sO + (wave * 32 + l32) * RO_LD + (d - pc * PD) + hh * 4) = v;
      }
    __syncthreads();
    // (query, 8-channel) items: PD / 16 per thread
#pragma unroll
    for (int i = 0; i < PD / 16; ++i) {
      const int it = tid + i * NT;
      const int ql = it / (PD / 8), g = it % (PD / 8);
      const int n = q0 + ql;
      const int d0 = pc * PD + g * 8;   // channel within the head
      const int y = n / a.W, x = n - y * a.W;
      u32x4_t tv[9];
#pragma unroll
      for (int t = 0; t < 9; ++t) {
        const int yy = y + t / 3 - 1, xx = x + t % 3 - 1;
        const bool in = n < N && (unsigned)yy < (unsigned)a.H && (unsigned)xx < (unsigned)a.W;
        const int key = in ? yy * a.W + xx : NK;
        tv[t] = *reinterpret_cast<const u32x4_t*>(sV + vidx(key, d0));
      }
      float pe[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int pr = 0; pr < 5; ++pr) {
        const u32x4_t w0 = *reinterpret_cast<const u32x4_t*>(sWp + pr * 64 + d0);
        const u32x4_t w1 = *reinterpret_cast<const u32x4_t*>(sWp + pr * 64 + d0 + 4);
        const u32x4_t va = tv[2 * pr];
        const u32x4_t vb = pr < 4 ? tv[2 * pr + 1] : (u32x4_t){0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          // (tap a, tap b) pairs of channel d0+2k (low halves) and d0+2k+1 (high halves)
          const uint32_t lo = __builtin_amdgcn_perm(va[k], vb[k], 0x01000504u);
          const uint32_t hi = __builtin_amdgcn_perm(va[k], vb[k], 0x03020706u);
          pe[2 * k] = dot2_bf16(lo, k < 2 ? w0[2 * k] : w1[2 * k - 4], pe[2 * k]);
          pe[2 * k + 1] = dot2_bf16(hi, k < 2 ? w0[2 * k + 1] : w1[2 * k - 3], pe[2 * k + 1]);
        }
      }
      if (n >= N) continue;
      const float* op = sO + ql * RO_LD + g * 8;
      float r8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) r8[j] = op[j] + pe[j] * sScale[d0 + j] + sShift[d0 + j];
      *reinterpret_cast<u32x4_t*>(reinterpret_cast<bf16_t*>(a.out) + (img + n) * a.out_pitch + h * 64 + d0) =
          (u32x4_t){pack_bf16x2(r8[0], r8[1]), pack_bf16x2(r8[2], r8[3]), pack_bf16x2(r8[4], r8[5]),
                    pack_bf16x2(r8[6], r8[7])};
    }
  }
}
}  // namespace

// QT = 7: tiles of seven 32-query tiles (two workgroups per 20x20 head, for
// batches with fewer heads than CUs); QT = 13 / 16: one workgroup per head.
extern "C" __global__ __launch_bounds__(448) void vrs_psa_attn_res7_bf16(vrs_attn_args a) { attn_resident_body<7>(a); }
extern "C" __global__ __launch_bounds__(832) void vrs_psa_attn_res13_bf16(vrs_attn_args a) { attn_resident_body<13>(a); }
extern "C" __global__ __launch_bounds__(1024) void vrs_psa_attn_res16_bf16(vrs_attn_args a) { attn_resident_body<16>(a); }

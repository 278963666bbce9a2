// Fused attention forward on the fp32 matrix cores:
//   O[b] = softmax_rows(scale * Q[b] K[b]^T) V[b]
// for every (batch, head) b, without writing the [Sq, Sk] score matrix.
//
// This is the lowering target of the reference graph
//   scores = q.batched_dot(k^T) * scale;  attn = scores.softmax();
//   ctx = attn.batched_dot(v)
// (include/array.h:1360-1403, 1677-1709): unfused it writes and re-reads the
// scores twice (48 x 512 x 512 fp32 = 50 MB at the encoder configuration)
// in three launches; fused, each workgroup keeps its 64 query rows' scores
// in registers and LDS while it walks the keys.
//
// Workgroup: 4 wavefronts over 32 query rows of one (batch, head): wavefront
// w takes row group w % 2 (16 rows) and key half w / 2 of every 64-key
// block, so 768 workgroups cover the encoder's 48 x 512 rows (three per CU,
// all resident) and each wavefront's running softmax covers half the keys;
// the two halves of a row group are merged through LDS at the end
// (m = max(m0, m1), l and O rescaled by exp(m_h - m)).  The block's K
// (row-major, pitch D + 4) and V (transposed, Vt[d][key], pitch 68) are
// staged in LDS; the next block's loads are issued before the current block
// is multiplied.  Per block and wavefront:
//   S (16 x 32) = Q_w K^T on v_mfma_f32_16x16x4f32, the head dim in groups
//     of 16 whose k values go to the lane's k slot q as 16 g + 4 q + j at
//     step j (any assignment of k to slots adds the same products), so Q
//     sits in registers as float4 per group and K is read with one
//     ds_read_b128 per 16-key block and group;
//   online softmax: s = acc * scale (the unfused product's rounding),
//     masked keys -inf, row max and sum over the 16 lanes that share a row
//     (DPP row reductions), exponentials on v_exp_f32, running max m and
//     sum l, O rescaled by exp(m - m');
//   P goes to the wavefront's LDS rows, is read back in the A-operand
//     layout and O (16 x D) += P V on MFMA, V read as ds_read_b128 from Vt.
// O is divided by l at the end and stored through the output strides (the
// head-merged [B*S, H*D] layout included).
#include <hip/hip_runtime.h>

#include <cmath>

#include "internal.h"

namespace silgpu {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kAttnWaves = 4;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kBQ = 32;       // query rows per workgroup (two row groups of 16)
constexpr int kBKey = 64;     // keys per block (two halves of 32)
constexpr int kHalf = kBKey / 2;
constexpr int kPadA = 4;      // LDS row padding (floats), keeps rows 16-byte aligned

template <int D>
struct attn_cfg {
  static_assert(D % 16 == 0 && D >= 16 && D <= 128, "head dim");
  static constexpr int kG = D / 16;                  // 16-deep groups of D = 16-column blocks of O
  static constexpr int kKPitch = D + kPadA;          // Ks[key][d]
  static constexpr int kVPitch = kBKey + kPadA;      // Vt[d][key]
  static constexpr int kPPitch = kHalf + kPadA;      // Ps[row][key]
  static constexpr int kKs = kBKey * kKPitch;
  static constexpr int kVt = D * kVPitch;
  static constexpr int kPs = kAttnWaves * 16 * kPPitch;
  static constexpr int kLdsBytes = (kKs + kVt + kPs) * 4;
  // Merge of the key halves: per lane, O (D/4 floats), m and l (4 each).
  static constexpr int kXfer = (D / 4 + 8) * kWave * 2;  // two row groups
  static_assert(kXfer <= kKs + kVt, "merge area");
  static constexpr int kLoads = kBKey * (D / 4) / kAttnThreads;  // float4 per thread per operand
  static_assert(kLoads * kAttnThreads * 4 == kBKey * D, "block load split");
};

struct attn_args {
  int Sq, Sk, binner;
  int vec;  // Q, K, V rows 16-byte aligned: float4 loads, else scalar loads
  float scale;
  const float *Q, *K, *V;
  float *O;
  int64_t ldq, ldk, ldv, ldo;
  int64_t sq_o, sq_i, sk_o, sk_i, sv_o, sv_i, so_o, so_i;
};

// Max and sum over the 16 lanes of a DPP row (the lanes that share a row of
// S): quad swaps, then the half-row and row mirrors.  Every lane ends with
// the same value (each step combines a pair of lanes symmetrically).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = fmaxf(v, dpp<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = fmaxf(v, dpp<0x141>(v));  // row_half_mirror
  return fmaxf(v, dpp<0x140>(v));  // row_mirror
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  return v + dpp<0x140>(v);
}

// e^x as 2^(x log2 e) on v_exp_f32: relative error about |x| 2^-24 from the
// product's rounding, far inside the tolerance of the fused path.
__device__ __forceinline__ float exp_fast(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

__device__ __forceinline__ float4 ld4u(const float *p, bool vec) {
  if (vec) return *reinterpret_cast<const float4 *>(p);
  return make_float4(p[0], p[1], p[2], p[3]);
}

__device__ __forceinline__ floatx4 mma4(floatx4 acc, float4 a, float4 b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, acc, 0, 0, 0);
  return acc;
}

template <int D>
__global__ __launch_bounds__(kAttnThreads) void attention_k(attn_args a) {
  using C = attn_cfg<D>;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float *Ks = lds, *Vt = lds + C::kKs, *Ps = lds + C::kKs + C::kVt;
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const int c = lane % 16, q = lane / 16;
  const int64_t zo = blockIdx.y / a.binner, zi = blockIdx.y % a.binner;
  const float *__restrict__ Q = a.Q + zo * a.sq_o + zi * a.sq_i;
  const float *__restrict__ K = a.K + zo * a.sk_o + zi * a.sk_i;
  const float *__restrict__ V = a.V + zo * a.sv_o + zi * a.sv_i;
  float *__restrict__ O = a.O + zo * a.so_o + zi * a.so_i;
  const int rg = wave % 2, kh = wave / 2;            // row group, key half
  const int row0 = blockIdx.x * kBQ + rg * 16;        // this wavefront's first query row
  const int Sq = a.Sq, Sk = a.Sk;

  // Q fragments: lane (c, q) holds Q[row0 + c][16 g + 4 q .. + 3] for each
  // group g (rows past Sq read row Sq - 1 and are never stored).
  float4 qf[C::kG];
  if (Sk > 0) {  // with no keys Q is not read (and may be null): O is 0
    const float *qr = Q + int64_t(min(row0 + c, Sq - 1)) * a.ldq + 4 * q;
#pragma unroll
    for (int g = 0; g < C::kG; ++g) qf[g] = ld4u(qr + 16 * g, a.vec);
  }

  // Staging registers of one key block: thread t loads float4 f = t + 256 u
  // of K as (key f / (D/4), d4 f % (D/4)) and of V as (key f % 64,
  // d4 f / 64), so the transposed LDS writes of V are conflict-free.
  float4 kst[C::kLoads], vst[C::kLoads];
  auto load_block = [&](int key0) {
#pragma unroll
    for (int u = 0; u < C::kLoads; ++u) {
      const int f = t + kAttnThreads * u;
      const int kk = f / (D / 4), kd = f % (D / 4);
      const int vk = f % kBKey, vd = f / kBKey;
      const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
      kst[u] = key0 + kk < Sk ? ld4u(K + int64_t(key0 + kk) * a.ldk + 4 * kd, a.vec) : z;
      vst[u] = key0 + vk < Sk ? ld4u(V + int64_t(key0 + vk) * a.ldv + 4 * vd, a.vec) : z;
    }
  };
  auto store_block = [&]() {
#pragma unroll
    for (int u = 0; u < C::kLoads; ++u) {
      const int f = t + kAttnThreads * u;
      const int kk = f / (D / 4), kd = f % (D / 4);
      const int vk = f % kBKey, vd = f / kBKey;
      *reinterpret_cast<float4 *>(Ks + kk * C::kKPitch + 4 * kd) = kst[u];
      Vt[(4 * vd + 0) * C::kVPitch + vk] = vst[u].x;
      Vt[(4 * vd + 1) * C::kVPitch + vk] = vst[u].y;
      Vt[(4 * vd + 2) * C::kVPitch + vk] = vst[u].z;
      Vt[(4 * vd + 3) * C::kVPitch + vk] = vst[u].w;
    }
  };

  floatx4 acc_o[C::kG];
#pragma unroll
  for (int j = 0; j < C::kG; ++j) acc_o[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m[4], l[4];  // running max and sum of rows 4 q + i
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.0f;
  }
  float *Pw = Ps + wave * 16 * C::kPPitch;  // this wavefront's 16 rows of P

  const int nblocks = (Sk + kBKey - 1) / kBKey;
  if (nblocks > 0) load_block(0);
  for (int kb = 0; kb < nblocks; ++kb) {
    const int key0 = kb * kBKey;
    __syncthreads();  // every wavefront is done reading the previous block
    store_block();
    __syncthreads();
    if (kb + 1 < nblocks) load_block(key0 + kBKey);  // lands while this block is multiplied

    // S = Q_w K^T over this wavefront's half: two 16-key blocks.
    const int kbase = kHalf * kh;  // first key of the half within the block
    floatx4 s[2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) s[jb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < C::kG; ++g)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const float4 kv = *reinterpret_cast<const float4 *>(
            Ks + (kbase + 16 * jb + c) * C::kKPitch + 16 * g + 4 * q);
        s[jb] = mma4(s[jb], qf[g], kv);
      }

    // Online softmax over the half.  Register i of block jb in lane (c, q)
    // is row 4 q + i, key key0 + kbase + 16 jb + c.
    float alpha[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float rm = -INFINITY;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        float v = s[jb][i] * a.scale;
        if (key0 + kbase + 16 * jb + c >= Sk) v = -INFINITY;
        s[jb][i] = v;
        rm = fmaxf(rm, v);
      }
      rm = row16_max(rm);
      const float mn = fmaxf(m[i], rm);
      const bool none = mn == -INFINITY;  // no finite score in this row yet
      alpha[i] = none ? 1.0f : exp_fast(m[i] - mn);
      float rs = 0.0f;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const float p = none ? 0.0f : exp_fast(s[jb][i] - mn);
        s[jb][i] = p;
        rs += p;
      }
      rs = row16_sum(rs);
      l[i] = l[i] * alpha[i] + rs;
      m[i] = mn;
    }
#pragma unroll
    for (int jd = 0; jd < C::kG; ++jd)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc_o[jd][i] *= alpha[i];

    // P to this wavefront's LDS rows, then back in the A-operand layout
    // (LDS accesses of one wavefront complete in order).
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int i = 0; i < 4; ++i) Pw[(4 * q + i) * C::kPPitch + 16 * jb + c] = s[jb][i];

    // O += P V over the half's two 16-key groups.
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const float4 pa = *reinterpret_cast<const float4 *>(Pw + c * C::kPPitch + 16 * g + 4 * q);
#pragma unroll
      for (int jd = 0; jd < C::kG; ++jd) {
        const float4 vb = *reinterpret_cast<const float4 *>(
            Vt + (16 * jd + c) * C::kVPitch + kbase + 16 * g + 4 * q);
        acc_o[jd] = mma4(acc_o[jd], pa, vb);
      }
    }
  }

  // Merge the key halves: the second half's wavefronts park (O, m, l) in
  // LDS (over the K/V stage), the first half's combine and store.  Lane
  // layouts of the two partners are identical.
  __syncthreads();  // every wavefront is done with the last K/V block
  float *X = lds + rg * (D / 4 + 8) * kWave;  // this row group's merge slots
  if (kh == 1) {
#pragma unroll
    for (int jd = 0; jd < C::kG; ++jd)
#pragma unroll
      for (int i = 0; i < 4; ++i) X[(4 * jd + i) * kWave + lane] = acc_o[jd][i];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      X[(D / 4 + i) * kWave + lane] = m[i];
      X[(D / 4 + 4 + i) * kWave + lane] = l[i];
    }
  }
  __syncthreads();
  if (kh == 1) return;
  // O / l, register i of block jd in lane (c, q) = O[row0 + 4 q + i][16 jd + c].
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float m1 = X[(D / 4 + i) * kWave + lane], l1 = X[(D / 4 + 4 + i) * kWave + lane];
    const float mm = fmaxf(m[i], m1);
    const float e0 = mm == -INFINITY ? 0.0f : expf(m[i] - mm);
    const float e1 = mm == -INFINITY ? 0.0f : expf(m1 - mm);
    const float lt = l[i] * e0 + l1 * e1;
    const int row = row0 + 4 * q + i;
    if (row >= Sq) continue;
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    float *orow = O + int64_t(row) * a.ldo;
#pragma unroll
    for (int jd = 0; jd < C::kG; ++jd)
      orow[16 * jd + c] = (acc_o[jd][i] * e0 + X[(4 * jd + i) * kWave + lane] * e1) * inv;
  }
}

template <int D>
int launch_attention(const attn_args &a, int64_t batch, hipStream_t s) {
  using C = attn_cfg<D>;
  static bool attr_done = false;
  if (!attr_done) {
    SILGPU_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(attention_k<D>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         C::kLdsBytes));
    attr_done = true;
  }
  dim3 grid(static_cast<unsigned>(cdiv(a.Sq, kBQ)), static_cast<unsigned>(batch));
  attention_k<D><<<grid, kAttnThreads, C::kLdsBytes, s>>>(a);
  SILGPU_LAUNCH_CHECK("attention_k");
  return SILGPU_OK;
}

bool rows16(const float *p, int64_t ld, int64_t so, int64_t si) {
  return aligned16(p) && ld % 4 == 0 && so % 4 == 0 && si % 4 == 0;
}

}  // namespace
}  // namespace silgpu

using namespace silgpu;

extern "C" {

int silgpu_attention_f32(const silgpu_attn_desc *d) {
  SILGPU_REQUIRE(d != nullptr, "silgpu_attention_f32: null descriptor");
  SILGPU_REQUIRE(d->Sq >= 0 && d->Sk >= 0 && d->batch_outer >= 0 && d->batch_inner >= 0,
                 "silgpu_attention_f32: negative extent");
  SILGPU_REQUIRE(d->D == 16 || d->D == 32 || d->D == 64 || d->D == 128,
                 "silgpu_attention_f32: head dim %lld not 16, 32, 64 or 128", (long long)d->D);
  SILGPU_REQUIRE(d->Sq <= INT32_MAX && d->Sk <= INT32_MAX,
                 "silgpu_attention_f32: sequence length exceeds int32");
  const int64_t batch = d->batch_outer * d->batch_inner;
  if (d->Sq == 0 || batch == 0) return SILGPU_OK;
  SILGPU_REQUIRE(batch <= 65535 && d->batch_inner <= INT32_MAX,
                 "silgpu_attention_f32: batch %lld exceeds the grid", (long long)batch);
  SILGPU_REQUIRE(d->O && (d->Sk == 0 || (d->Q && d->K && d->V)),
                 "silgpu_attention_f32: null pointer");
  SILGPU_REQUIRE(d->ldq >= d->D && d->ldk >= d->D && d->ldv >= d->D && d->ldo >= d->D,
                 "silgpu_attention_f32: a row stride is below the head dim");
  SILGPU_CTX(c);
  attn_args a{};
  a.Sq = static_cast<int>(d->Sq);
  a.Sk = static_cast<int>(d->Sk);
  a.binner = static_cast<int>(d->batch_inner);
  a.vec = rows16(d->Q, d->ldq, d->stride_q_outer, d->stride_q_inner) &&
          rows16(d->K, d->ldk, d->stride_k_outer, d->stride_k_inner) &&
          rows16(d->V, d->ldv, d->stride_v_outer, d->stride_v_inner);
  a.scale = d->scale;
  a.Q = d->Q;
  a.K = d->K;
  a.V = d->V;
  a.O = d->O;
  a.ldq = d->ldq;
  a.ldk = d->ldk;
  a.ldv = d->ldv;
  a.ldo = d->ldo;
  a.sq_o = d->stride_q_outer;
  a.sq_i = d->stride_q_inner;
  a.sk_o = d->stride_k_outer;
  a.sk_i = d->stride_k_inner;
  a.sv_o = d->stride_v_outer;
  a.sv_i = d->stride_v_inner;
  a.so_o = d->stride_o_outer;
  a.so_i = d->stride_o_inner;
  switch (d->D) {
    case 16: return launch_attention<16>(a, batch, c->stream);
    case 32: return launch_attention<32>(a, batch, c->stream);
    case 64: return launch_attention<64>(a, batch, c->stream);
    default: return launch_attention<128>(a, batch, c->stream);
  }
}

}  // extern "C"

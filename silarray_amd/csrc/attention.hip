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
// (row-major, pitch D + 8) and V (row-major, pitch D + 4) are staged in LDS
// with one 16-byte write per loaded float4; the next block's loads are
// issued before the current block is multiplied.  Both products are
// computed transposed on v_mfma_f32_16x16x4f32, so that each lane owns one
// query row:
//   S^T (32 keys x 16 rows) = K Q^T: the head dim in groups of 16 whose k
//     values go to the lane's k slot q as 16 g + 4 q + j at step j (any
//     assignment of k to slots adds the same products), so Q^T sits in
//     registers as a float4 per group and K is read with one ds_read_b128
//     per 16-key block and group; lane (c, q) then holds scores of row c at
//     keys 16 jb + 4 q + r;
//   online softmax per lane: row max and sum over its 8 registers and the
//     lanes c + 16, c + 32, c + 48, running max m and sum l, O rescaled by
//     one factor per lane;
//   O^T (D x 16 rows) += V^T P^T: the exponentiated scores are already the
//     B operand (key 16 jb + 4 q + j of row c at step j), so P never leaves
//     registers; lane (c, q) reads its V^T operands V[key 16 jb + 4 q + j]
//     [d 16 jd + c] for j < 4 as four ds_read_b32 (row-major V needs no
//     transposing writes: 38.8 against 40.9 us at the encoder shape, 51.5
//     against 56.1 at head dim 128).
// O is divided by l at the end and stored through the output strides (the
// head-merged [B*S, H*D] layout included) as a float4 per lane and block.
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
// LDS row pitches.  K is read with ds_read_b128 by lanes (c, q) at row c,
// float 4 q: with the pitch a multiple of 8 floats but not of 16 ((pitch /
// 4) % 4 == 2), the 16 lanes of each b128 pass hit distinct 16-byte bank
// groups.  V is read with ds_read_b32 by lanes (c, q) at row 4 q + j, float
// c: a pitch of 4 mod 8 floats puts the two q of each half-wave pass on
// disjoint halves of the 32 banks.
constexpr int kPadKV = 8;

template <int D>
struct attn_cfg {
  static_assert(D % 16 == 0 && D >= 16 && D <= 128, "head dim");
  static constexpr int kG = D / 16;                  // 16-deep groups of D = 16-column blocks of O
  static constexpr int kKPitch = D + kPadKV;         // Ks[key][d]
  static constexpr int kVPitch = D + 4;              // Vs[key][d]
  static constexpr int kKs = kBKey * kKPitch;
  static constexpr int kVs = kBKey * kVPitch;
  static constexpr int kLdsBytes = (kKs + kVs) * 4;
  // Merge of the key halves: per lane, O (D/4 floats), m and l.
  static constexpr int kXfer = (D / 4 + 2) * kWave * 2;  // two row groups
  static_assert(kXfer <= kKs + kVs, "merge area");
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
  float *Ks = lds, *Vs = lds + C::kKs;
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const int c = lane % 16, q = lane / 16;
  const int64_t zo = blockIdx.y / a.binner, zi = blockIdx.y % a.binner;
  const float *__restrict__ Q = a.Q + zo * a.sq_o + zi * a.sq_i;
  const float *__restrict__ K = a.K + zo * a.sk_o + zi * a.sk_i;
  const float *__restrict__ V = a.V + zo * a.sv_o + zi * a.sv_i;
  float *__restrict__ O = a.O + zo * a.so_o + zi * a.so_i;
  const int rg = wave % 2, kh = wave / 2;        // row group, key half
  const int row0 = blockIdx.x * kBQ + rg * 16;    // this wavefront's first query row
  const int row = row0 + c;                       // the query row of this lane
  const int Sq = a.Sq, Sk = a.Sk;
  const float scale2 = a.scale * 1.4426950408889634f;  // scale * log2(e)

  // Q fragments: lane (c, q) holds Q[row][16 g + 4 q .. + 3] for each group
  // g (rows past Sq read row Sq - 1 and are never stored).
  float4 qf[C::kG];
  if (Sk > 0) {  // with no keys Q is not read (and may be null): O is 0
    const float *qr = Q + int64_t(min(row, Sq - 1)) * a.ldq + 4 * q;
#pragma unroll
    for (int g = 0; g < C::kG; ++g) qf[g] = ld4u(qr + 16 * g, a.vec);
  }

  // Staging registers of one key block: thread t loads float4 f = t + 256 u
  // of K and of V as (key f / (D/4), d4 f % (D/4)): whole rows per group of
  // lanes, coalesced, and one ds_write_b128 each.
  // Per-thread source pointers at key 0, advanced by whole blocks.
  float4 kst[C::kLoads], vst[C::kLoads];
  const float *kp[C::kLoads], *vp[C::kLoads];
#pragma unroll
  for (int u = 0; u < C::kLoads; ++u) {
    const int f = t + kAttnThreads * u;
    kp[u] = K + int64_t(f / (D / 4)) * a.ldk + 4 * (f % (D / 4));
    vp[u] = V + int64_t(f / (D / 4)) * a.ldv + 4 * (f % (D / 4));
  }
  auto load_block = [&](int key0) {
    const int64_t ko = int64_t(key0) * a.ldk, vo = int64_t(key0) * a.ldv;
    if (key0 + kBKey <= Sk) {  // a full block: no masks
#pragma unroll
      for (int u = 0; u < C::kLoads; ++u) {
        kst[u] = ld4u(kp[u] + ko, a.vec);
        vst[u] = ld4u(vp[u] + vo, a.vec);
      }
    } else {
#pragma unroll
      for (int u = 0; u < C::kLoads; ++u) {
        const int f = t + kAttnThreads * u;
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
        kst[u] = key0 + f / (D / 4) < Sk ? ld4u(kp[u] + ko, a.vec) : z;
        vst[u] = key0 + f / (D / 4) < Sk ? ld4u(vp[u] + vo, a.vec) : z;
      }
    }
  };
  auto store_block = [&]() {
#pragma unroll
    for (int u = 0; u < C::kLoads; ++u) {
      const int f = t + kAttnThreads * u;
      const int kk = f / (D / 4), kd = f % (D / 4);
      *reinterpret_cast<float4 *>(Ks + kk * C::kKPitch + 4 * kd) = kst[u];
      *reinterpret_cast<float4 *>(Vs + kk * C::kVPitch + 4 * kd) = vst[u];
    }
  };

  // O^T accumulators: register r of block jd in lane (c, q) is
  // O[row][16 jd + 4 q + r].  Running max m and sum l of this lane's row.
  floatx4 acc_o[C::kG];
#pragma unroll
  for (int j = 0; j < C::kG; ++j) acc_o[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.0f;

  const int nblocks = (Sk + kBKey - 1) / kBKey;
  if (nblocks > 0) load_block(0);
  for (int kb = 0; kb < nblocks; ++kb) {
    const int key0 = kb * kBKey;
    const bool full = key0 + kBKey <= Sk;
    __syncthreads();  // every wavefront is done reading the previous block
    store_block();
    __syncthreads();
    if (kb + 1 < nblocks) load_block(key0 + kBKey);  // lands while this block is multiplied

    // S^T = K_half Q_w^T, two 16-key blocks: register r of block jb in lane
    // (c, q) is S[row][key0 + kbase + 16 jb + 4 q + r].  The A operand is K
    // (one ds_read_b128 per block and group), the B operand Q^T (qf).
    const int kbase = kHalf * kh;
    floatx4 st[2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) st[jb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < C::kG; ++g)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const float4 kv = *reinterpret_cast<const float4 *>(
            Ks + (kbase + 16 * jb + c) * C::kKPitch + 16 * g + 4 * q);
        st[jb] = mma4(st[jb], kv, qf[g]);
      }

    // Online softmax of this lane's row over the half: the row's 32 keys are
    // the 8 registers here and in lanes c + 16, c + 32, c + 48.  Scores are
    // kept in the base-2 domain, x = acc * (scale log2 e), so e^(s - m) is
    // one v_exp_f32 of x - m (relative error about |x - m| 2^-24); m is the
    // running maximum of x.
    float v[2][4];
    float rm = -INFINITY;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = st[jb][r] * scale2;
        if (!full && key0 + kbase + 16 * jb + 4 * q + r >= Sk) x = -INFINITY;
        v[jb][r] = x;
        rm = fmaxf(rm, x);
      }
    const auto fmax2 = [](float a, float b) { return fmaxf(a, b); };
    const auto add2 = [](float a, float b) { return a + b; };
    rm = pair_reduce<32>(pair_reduce<16>(rm, fmax2), fmax2);
    const float mn = fmaxf(m, rm);
    const bool none = mn == -INFINITY;  // no finite score in this row yet
    const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
    float4 p[2];
    float rs = 0.0f;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      float e[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        e[r] = none ? 0.0f : __builtin_amdgcn_exp2f(v[jb][r] - mn);
        rs += e[r];
      }
      p[jb] = make_float4(e[0], e[1], e[2], e[3]);
    }
    rs = pair_reduce<32>(pair_reduce<16>(rs, add2), add2);
    l = l * alpha + rs;
    m = mn;
#pragma unroll
    for (int jd = 0; jd < C::kG; ++jd) acc_o[jd] *= alpha;

    // O^T += V^T P^T: A operand V^T (four ds_read_b32 from Vs), B operand P^T,
    // which is p: register r of key block jb is key 16 jb + 4 q + r of this
    // lane's row, the operand layout the MFMA asks for.
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int jd = 0; jd < C::kG; ++jd) {
        const float *vr = Vs + (kbase + 16 * jb + 4 * q) * C::kVPitch + 16 * jd + c;
        const float4 vb = make_float4(vr[0], vr[C::kVPitch], vr[2 * C::kVPitch],
                                      vr[3 * C::kVPitch]);
        acc_o[jd] = mma4(acc_o[jd], vb, p[jb]);
      }
  }

  // Merge the key halves: the second half's wavefronts park (O, m, l) in
  // LDS (over the K/V stage), the first half's combine and store.  Lane
  // layouts of the two partners are identical.
  __syncthreads();  // every wavefront is done with the last K/V block
  float *X = lds + rg * (D / 4 + 2) * kWave;  // this row group's merge slots
  if (kh == 1) {
#pragma unroll
    for (int jd = 0; jd < C::kG; ++jd)
#pragma unroll
      for (int r = 0; r < 4; ++r) X[(4 * jd + r) * kWave + lane] = acc_o[jd][r];
    X[(D / 4) * kWave + lane] = m;
    X[(D / 4 + 1) * kWave + lane] = l;
  }
  __syncthreads();
  if (kh == 1 || row >= Sq) return;
  const float m1 = X[(D / 4) * kWave + lane], l1 = X[(D / 4 + 1) * kWave + lane];
  const float mm = fmaxf(m, m1);
  const float e0 = mm == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mm);
  const float e1 = mm == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - mm);
  const float lt = l * e0 + l1 * e1;
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  float *orow = O + int64_t(row) * a.ldo + 4 * q;
  const bool vst4 = (a.ldo & 3) == 0 && aligned16_dev(O);
#pragma unroll
  for (int jd = 0; jd < C::kG; ++jd) {
    float o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      o[r] = (acc_o[jd][r] * e0 + X[(4 * jd + r) * kWave + lane] * e1) * inv;
    if (vst4) {
      *reinterpret_cast<float4 *>(orow + 16 * jd) = make_float4(o[0], o[1], o[2], o[3]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) orow[16 * jd + r] = o[r];
    }
  }
}

template <int D>
int launch_attention(const attn_args &a, int64_t batch, hipStream_t s) {
  using C = attn_cfg<D>;
  // Once per process (a thread-safe static), before the first launch.
  static const hipError_t attr_rc =
      hipFuncSetAttribute(reinterpret_cast<const void *>(attention_k<D>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, C::kLdsBytes);
  SILGPU_HIP_CHECK(attr_rc);
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
  SILGPU_REQUIRE(d->O && (d->Sk == 0 || (d->Q && d->K && d->V)),
                 "silgpu_attention_f32: null pointer");
  SILGPU_REQUIRE(d->ldq >= d->D && d->ldk >= d->D && d->ldv >= d->D && d->ldo >= d->D,
                 "silgpu_attention_f32: a row stride is below the head dim");
  if (batch > kMaxGridBatch) {
    // More (batch, head) pairs than one launch's grid.y holds: launches of
    // at most kMaxGridBatch pairs, split as silgpu_gemm splits its batch.
    silgpu_attn_desc p = *d;
    auto shift = [&](int64_t o, int64_t i) {
      auto at = [](const float *x, int64_t off) { return x ? x + off : x; };
      p.Q = at(d->Q, o * d->stride_q_outer + i * d->stride_q_inner);
      p.K = at(d->K, o * d->stride_k_outer + i * d->stride_k_inner);
      p.V = at(d->V, o * d->stride_v_outer + i * d->stride_v_inner);
      p.O = d->O ? d->O + o * d->stride_o_outer + i * d->stride_o_inner : d->O;
    };
    if (d->batch_inner <= kMaxGridBatch) {
      const int64_t per = kMaxGridBatch / d->batch_inner;
      for (int64_t o0 = 0; o0 < d->batch_outer; o0 += per) {
        shift(o0, 0);
        p.batch_outer = d->batch_outer - o0 < per ? d->batch_outer - o0 : per;
        const int rc = silgpu_attention_f32(&p);
        if (rc != SILGPU_OK) return rc;
      }
    } else {
      for (int64_t o = 0; o < d->batch_outer; o++)
        for (int64_t i0 = 0; i0 < d->batch_inner; i0 += kMaxGridBatch) {
          shift(o, i0);
          p.batch_outer = 1;
          p.batch_inner =
              d->batch_inner - i0 < kMaxGridBatch ? d->batch_inner - i0 : kMaxGridBatch;
          const int rc = silgpu_attention_f32(&p);
          if (rc != SILGPU_OK) return rc;
        }
    }
    return SILGPU_OK;
  }
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

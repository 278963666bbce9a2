// Matrix products on gfx950: fp32 MFMA SGEMM and HBM-bound GEMV.
//
// SGEMM (the reference's STEEL / sgemm_32 / MPS paths, include/gpu.h:509-615,
// 1296-1328) runs on the fp32 matrix cores: v_mfma_f32_16x16x4_f32 (a 16x4
// A fragment times a 4x16 B fragment into a 16x16 accumulator of 4 registers
// per lane) or v_mfma_f32_32x32x2_f32 (32x2 by 2x32 into 32x32, 16
// registers).  Both keep a SIMD's matrix core busy for 256 flops per cycle
// per CU, so the kernel's job is to issue one back to back on every SIMD:
// operands are staged through LDS in k-major tiles, the next K tile is
// fetched into registers while the current one is multiplied (double-
// buffered LDS, one barrier per K tile), the fragments of k-step s+1 are read
// from LDS while the MFMAs of step s run (a scheduling barrier per step keeps
// the compiler from hoisting further and spilling), and the workgroup -> tile
// mapping keeps the workgroups of one XCD on neighbouring tiles so their A
// and B panels are shared in that XCD's L2.  Products too small to fill the
// 256 CUs split K: across workgroups (partial planes added by a second
// launch) or, for 64 x 64 tiles, also between two or four groups of waves
// inside a workgroup (added through LDS, no second launch).
//
// Epilogues (bias, sigmoid, relu) are applied to the accumulators before the
// single store, so linear / linear_sigmoid are one pass over C.
#include <hip/hip_runtime.h>

#include <cmath>

#include "internal.h"

namespace silgpu {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// fp32 MFMA shapes.  MI x MI output block, KI k values per instruction.
//   32x32x2: lane l supplies A[l%32][l/32] and B[l/32][l%32] and holds
//            C[8*(r/4) + 4*(l/32) + r%4][l%32] in register r < 16;
//   16x16x4: lane l supplies A[l%16][l/16] and B[l/16][l%16] and holds
//            C[4*(l/16) + r][l%16] in register r < 4.
template <int MI>
struct mfma;
template <>
struct mfma<32> {
  static constexpr int KI = 2, R = 16;
  typedef floatx16 acc_t;
  __device__ static acc_t run(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ static int row(int lane, int r) { return 8 * (r / 4) + 4 * (lane / 32) + (r % 4); }
};
template <>
struct mfma<16> {
  static constexpr int KI = 4, R = 4;
  typedef floatx4 acc_t;
  __device__ static acc_t run(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  __device__ static int row(int lane, int r) { return 4 * (lane / 16) + r; }
};

// ---- tile mapping -----------------------------------------------------------

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup id mod 8).
// Remap ids so each XCD gets a contiguous range of tiles, then raster that
// range in groups of kGroupM tile rows so concurrently running tiles share
// A row panels and B column panels.
constexpr int kXcds = 8;
constexpr int kGroupM = 8;

__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int &tm,
                                            int &tn) {
  const int nblocks = tiles_m * tiles_n;
  const int full = (nblocks / kXcds) * kXcds;
  if (bid < full) bid = (bid % kXcds) * (full / kXcds) + bid / kXcds;
  const int group_size = kGroupM * tiles_n;
  const int group = bid / group_size;
  const int first_m = group * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  const int in_group = bid % group_size;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

// ---- SGEMM kernel -----------------------------------------------------------

// Epilogue of one accumulator, in this order: scalar affine node folded in
// (fmaf, the node's own rounding), bias, activation, residual add.
struct epi_args {
  const float *bias;
  int64_t bias_len;
  const float *res;  // residual (batch 1 only), res[m * ldr + n]
  int64_t ldr;
  float scale, offset;
  int epi;
  int use_scale;
};

// apply_epi with the bias value of column n (bv) and the residual value of
// (m, n) (rv) already loaded; each is ignored where the epilogue has none.
__device__ __forceinline__ float apply_epi_vals(float v, float bv, float rv, const epi_args &e) {
  if (e.use_scale) v = fmaf(v, e.scale, e.offset);
  if (e.epi == SILGPU_EPI_BIAS || e.epi == SILGPU_EPI_BIAS_SIGMOID ||
      e.epi == SILGPU_EPI_BIAS_RELU)
    v += bv;
  if (e.epi == SILGPU_EPI_BIAS_SIGMOID) v = sigmoidf_dev(v);
  else if (e.epi == SILGPU_EPI_RELU || e.epi == SILGPU_EPI_BIAS_RELU) v = fmaxf(v, 0.0f);
  if (e.res) v = v + rv;
  return v;
}

__device__ __forceinline__ float apply_epi(float v, int64_t m, int64_t n, const epi_args &e) {
  if (e.use_scale) v = fmaf(v, e.scale, e.offset);
  if (e.epi == SILGPU_EPI_BIAS || e.epi == SILGPU_EPI_BIAS_SIGMOID ||
      e.epi == SILGPU_EPI_BIAS_RELU)
    v += e.bias[n % e.bias_len];
  if (e.epi == SILGPU_EPI_BIAS_SIGMOID) v = sigmoidf_dev(v);
  else if (e.epi == SILGPU_EPI_RELU || e.epi == SILGPU_EPI_BIAS_RELU) v = fmaxf(v, 0.0f);
  if (e.res) v = v + e.res[m * e.ldr + n];
  return v;
}

struct gemm_args {
  const float *A;
  const float *B;
  float *C;
  int64_t lda, ldb, ldc;
  // batch index z = zo * binner + zi: operand X at X + zo*sX2 + zi*sX
  int64_t sA, sB, sC;
  int64_t sA2, sB2, sC2;
  int binner;
  int M, N, K;
  int tiles_m, tiles_n;
  epi_args ep;
  // Split K: workgroup row blockIdx.y covers K range [y*klen, (y+1)*klen)
  // (klen a multiple of BK).  With gridDim.y > 1 raw accumulators go to
  // ws[y][M][N] and splitk_sum_k applies the epilogue.
  int klen;
  float *ws;
  // Implicit-GEMM convolution (sgemm_mfma_k<..., CONV>): A is the virtual
  // im2col matrix of an NHWC input [batch][H][W][C_in], row m = output
  // pixel (n, oh, ow), column k = (kh, kw, ci) with ci fastest, stride 1,
  // zero padding `pad` on every side (output H x W).  Row m of this launch
  // is output pixel cv_m0 + m (a launch may cover a range of the rows).
  int cv_h, cv_w, cv_cin, cv_k, cv_pad, cv_m0;
};

template <int BM, int BN, int BK, int WM, int WN, int MI>
struct cfg {
  static constexpr int kThreads = WM * WN * kWave;
  static constexpr int TM = BM / WM / MI;  // MFMA blocks per wave along M
  static constexpr int TN = BN / WN / MI;
  static constexpr int LA = BM + 4;        // LDS row pitch (floats), padded
  static constexpr int LB = BN + 4;
  static constexpr int kAStage = BK * LA;  // floats per stage
  static constexpr int kBStage = BK * LB;
  static constexpr int kLdsBytes = 2 * (kAStage + kBStage) * 4;
  static constexpr int NA = BM * BK / 4 / kThreads;  // 4-float groups per thread
  static constexpr int NB = BK * BN / 4 / kThreads;
  static_assert(TM >= 1 && TN >= 1 && TM * WM * MI == BM && TN * WN * MI == BN,
                "wave tile not a whole number of MFMA blocks");
  static_assert(NA >= 1 && NB >= 1 && NA * 4 * kThreads == BM * BK &&
                    NB * 4 * kThreads == BK * BN,
                "tile not divisible among threads");
  static_assert(BK % 4 == 0 && BK % mfma<MI>::KI == 0, "BK");
};

// Loads this thread's share of an R x Cc tile whose *contiguous* global axis
// has Cc elements (4 per group).  Group f = t + i*NT covers row f / (Cc/4),
// columns (f % (Cc/4))*4 .. +3.  Out-of-range elements read as 0.
template <int R, int Cc, int NT, int NG, bool VEC, bool EDGE>
__device__ __forceinline__ void load_groups(const float *__restrict__ base, int64_t ld,
                                            int row0, int col0, int rows, int cols, int t,
                                            float (&g)[NG][4]) {
  constexpr int GPR = Cc / 4;  // groups per row
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int f = t + i * NT;
    const int r = f / GPR;
    const int c = (f % GPR) * 4;
    const int gr = row0 + r, gc = col0 + c;
    const float *p = base + int64_t(gr) * ld + gc;
    if constexpr (VEC) {
      // VEC requires cols % 4 == 0, so a group is entirely in or out.
      if (!EDGE || (gr < rows && gc < cols)) {
        float4 v = *reinterpret_cast<const float4 *>(p);
        g[i][0] = v.x;
        g[i][1] = v.y;
        g[i][2] = v.z;
        g[i][3] = v.w;
      } else {
        g[i][0] = g[i][1] = g[i][2] = g[i][3] = 0.0f;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        g[i][j] = (!EDGE || (gr < rows && gc + j < cols)) ? p[j] : 0.0f;
    }
  }
}

// Stores groups into a k-major LDS tile S[k][x] (pitch L).
//  KMAJOR_GLOBAL = true : the global contiguous axis is x (groups run along
//                         x within one k row) -> one 16-byte LDS write.
//  KMAJOR_GLOBAL = false: the global contiguous axis is k (groups run along
//                         k within one x row) -> four 4-byte writes.
template <int R, int Cc, int NT, int NG, int L, bool KMAJOR_GLOBAL>
__device__ __forceinline__ void store_groups(float *__restrict__ S, int t,
                                             const float (&g)[NG][4]) {
  constexpr int GPR = Cc / 4;
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int f = t + i * NT;
    const int r = f / GPR;
    const int c = (f % GPR) * 4;
    if constexpr (KMAJOR_GLOBAL) {
      // row r is k, columns c.. are x
      *reinterpret_cast<float4 *>(S + r * L + c) = make_float4(g[i][0], g[i][1], g[i][2], g[i][3]);
    } else {
      // row r is x, columns c.. are k
#pragma unroll
      for (int j = 0; j < 4; ++j) S[(c + j) * L + r] = g[i][j];
    }
  }
}

// Implicit-GEMM gather of the A tile of a convolution: row m is output
// pixel (n, oh, ow), column k = (kh * K + kw) * C_in + ci is a tap and a
// channel, and A[m][k] = in[n][oh + kh - pad][ow + kw - pad][ci] (zero
// outside the image, past M and past K).  Each thread owns NG groups of 4
// consecutive k of the tile; a walk keeps every group's (kh, kw, ci) and
// steps it by the tile depth Cc per call, so the K loop divides nothing.
// NE: 1 when C_in % 4 == 0 (a group is ci .. ci + 3 of one tap, one
// float4 load), else 4 (one position per element).
template <int R, int Cc, int NT, int NG, bool VEC>
struct conv_walk {
  static constexpr int NE = VEC ? 1 : 4;
  int64_t base[NG];  // element offset of (n, oh - pad, ow - pad, 0)
  int oh[NG], ow[NG];  // oh = -1 past M
  int k[NG];           // reduction index of the group's first element
  int ci[NG][NE], kw[NG][NE], kh[NG][NE];

  __device__ __forceinline__ void init(const gemm_args &p, int row0, int k0, int t) {
    constexpr int GPR = Cc / 4;
    const int hw = p.cv_h * p.cv_w, cin = p.cv_cin;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int m = row0 + (t + i * NT) / GPR;
      oh[i] = -1;
      ow[i] = 0;
      base[i] = 0;
      if (m < p.M) {
        const int pm = p.cv_m0 + m, n = pm / hw, rem = pm - n * hw;
        oh[i] = rem / p.cv_w;
        ow[i] = rem - oh[i] * p.cv_w;
        base[i] = ((int64_t(n) * p.cv_h + oh[i] - p.cv_pad) * p.cv_w + ow[i] - p.cv_pad) * cin;
      }
      k[i] = k0 + ((t + i * NT) % GPR) * 4;
#pragma unroll
      for (int e = 0; e < NE; ++e) {
        const int ke = k[i] + e, khw = ke / cin;
        ci[i][e] = ke - khw * cin;
        kh[i][e] = khw / p.cv_k;
        kw[i][e] = khw - kh[i][e] * p.cv_k;
      }
    }
  }

  // The groups at the current k, then one step of Cc.
  __device__ __forceinline__ void gather(const gemm_args &p, const float *A, float (&g)[NG][4]) {
    const int cin = p.cv_cin, kk = p.cv_k, Kd = p.K;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      if constexpr (VEC) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        const int ih = oh[i] + kh[i][0] - p.cv_pad, iw = ow[i] + kw[i][0] - p.cv_pad;
        if (oh[i] >= 0 && k[i] < Kd && ih >= 0 && ih < p.cv_h && iw >= 0 && iw < p.cv_w)
          v = *reinterpret_cast<const float4 *>(
              A + base[i] + (kh[i][0] * p.cv_w + kw[i][0]) * cin + ci[i][0]);
        g[i][0] = v.x;
        g[i][1] = v.y;
        g[i][2] = v.z;
        g[i][3] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int ih = oh[i] + kh[i][e] - p.cv_pad, iw = ow[i] + kw[i][e] - p.cv_pad;
          g[i][e] = oh[i] >= 0 && k[i] + e < Kd && ih >= 0 && ih < p.cv_h && iw >= 0 &&
                            iw < p.cv_w
                        ? A[base[i] + (kh[i][e] * p.cv_w + kw[i][e]) * cin + ci[i][e]]
                        : 0.0f;
        }
      }
      k[i] += Cc;
#pragma unroll
      for (int e = 0; e < NE; ++e) {
        ci[i][e] += Cc;
        while (ci[i][e] >= cin) {
          ci[i][e] -= cin;
          if (++kw[i][e] == kk) {
            kw[i][e] = 0;
            ++kh[i][e];
          }
        }
      }
    }
  }
};

template <int BM, int BN, int BK, int WM, int WN, int MI, bool TA, bool TB, bool VEC, bool EDGE,
          bool CONV = false>
__global__ __launch_bounds__(WM *WN *kWave) void sgemm_mfma_k(gemm_args p) {
  using C = cfg<BM, BN, BK, WM, WN, MI>;
  using F = mfma<MI>;
  constexpr int NT = C::kThreads;
  extern __shared__ float lds[];
  float *As = lds;                    // [2][BK][LA]
  float *Bs = lds + 2 * C::kAStage;   // [2][BK][LB]

  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
  const int wm = wave / WN, wn = wave % WN;

  int tm, tn;
  tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int64_t zo = blockIdx.z / p.binner, zi = blockIdx.z % p.binner;
  const float *__restrict__ A = p.A + zo * p.sA2 + zi * p.sA;
  const float *__restrict__ B = p.B + zo * p.sB2 + zi * p.sB;
  float *__restrict__ Cp = p.C + zo * p.sC2 + zi * p.sC;
  const int M = p.M, N = p.N, K = p.K;

  typename F::acc_t acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int r = 0; r < F::R; ++r) acc[i][j][r] = 0.0f;

  float ga[C::NA][4], gb[C::NB][4];
  // Convolution: the pixels of this thread's A rows, fixed over the K loop.
  // Convolution: the walk of this thread's A groups through the taps.  The
  // loads below ask for k = kbeg, kbeg + BK, ... in order, one call each.
  conv_walk<BM, BK, NT, CONV ? C::NA : 1, VEC> cw;
  if constexpr (CONV) cw.init(p, m0, blockIdx.y * p.klen, t);
  // Global views: A non-trans is [M][K] (contiguous K), trans is [K][M].
  //               B non-trans is [K][N] (contiguous N), trans is [N][K].
  auto load_a = [&](int k0) {
    if constexpr (CONV)
      cw.gather(p, A, ga);
    else if constexpr (!TA)
      load_groups<BM, BK, NT, C::NA, VEC, EDGE>(A, p.lda, m0, k0, M, K, t, ga);
    else
      load_groups<BK, BM, NT, C::NA, VEC, EDGE>(A, p.lda, k0, m0, K, M, t, ga);
  };
  auto load_b = [&](int k0) {
    if constexpr (!TB)
      load_groups<BK, BN, NT, C::NB, VEC, EDGE>(B, p.ldb, k0, n0, K, N, t, gb);
    else
      load_groups<BN, BK, NT, C::NB, VEC, EDGE>(B, p.ldb, n0, k0, N, K, t, gb);
  };
  auto store_a = [&](int stage) {
    float *S = As + stage * C::kAStage;
    if constexpr (!TA)
      store_groups<BM, BK, NT, C::NA, C::LA, false>(S, t, ga);
    else
      store_groups<BK, BM, NT, C::NA, C::LA, true>(S, t, ga);
  };
  auto store_b = [&](int stage) {
    float *S = Bs + stage * C::kBStage;
    if constexpr (!TB)
      store_groups<BK, BN, NT, C::NB, C::LB, true>(S, t, gb);
    else
      store_groups<BN, BK, NT, C::NB, C::LB, false>(S, t, gb);
  };

  const int kbeg = blockIdx.y * p.klen;
  const int kend = min(K, kbeg + p.klen);
  const int KT = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
  const int kl = lane / MI;  // which k of the instruction this lane supplies
  const int lm = lane % MI;  // its row of A / column of B within a block
  const int a_col = wm * C::TM * MI + lm;
  const int b_col = wn * C::TN * MI + lm;

  if (KT > 0) {
    load_a(kbeg);
    load_b(kbeg);
    store_a(0);
    store_b(0);
    __syncthreads();
  }
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) {
      load_a(kbeg + (kt + 1) * BK);
      load_b(kbeg + (kt + 1) * BK);
    }
    const float *Sa = As + cur * C::kAStage + kl * C::LA + a_col;
    const float *Sb = Bs + cur * C::kBStage + kl * C::LB + b_col;
    // Fragments of k-step s+1 are read while the MFMAs of step s run.
    constexpr int S = BK / F::KI;
    float a[2][C::TM], b[2][C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; ++i) a[0][i] = Sa[i * MI];
#pragma unroll
    for (int j = 0; j < C::TN; ++j) b[0][j] = Sb[j * MI];
#pragma unroll
    for (int st = 0; st < S; ++st) {
      const int cf = st & 1, nf = cf ^ 1;
      if (st + 1 < S) {
#pragma unroll
        for (int i = 0; i < C::TM; ++i) a[nf][i] = Sa[(F::KI * (st + 1)) * C::LA + i * MI];
#pragma unroll
        for (int j = 0; j < C::TN; ++j) b[nf][j] = Sb[(F::KI * (st + 1)) * C::LB + j * MI];
      }
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) acc[i][j] = F::run(a[cf][i], b[cf][j], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (more) {
      store_a(cur ^ 1);
      store_b(cur ^ 1);
    }
    __syncthreads();
  }

  // Epilogue.  Accumulator register r of lane l in block (i, j) is
  // C[row][col] with col = MI*j + l%MI and row = MI*i + F::row(l, r)
  // (relative to the wave tile).
  if (gridDim.y > 1) {
    float *W = p.ws + int64_t(blockIdx.y) * M * N;
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      const int col = n0 + wn * C::TN * MI + j * MI + lm;
      if (EDGE && col >= N) continue;
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int r = 0; r < F::R; ++r) {
          const int row = m0 + wm * C::TM * MI + i * MI + F::row(lane, r);
          if (EDGE && row >= M) continue;
          W[int64_t(row) * N + col] = acc[i][j][r];
        }
    }
    return;
  }
  // One MFMA row block at a time (a scheduling barrier per block), so the
  // compiler does not precompute every store address at once and spill.  As
  // in the LDS-direct kernel, the epilogue's bias and residual values are
  // loaded ahead of the stores: the whole tile's where they fit 32
  // registers, else a chunk of row blocks (at most 16 values) ahead.
  constexpr int kVals = F::R * C::TN;
  constexpr int CH = C::TM * kVals <= 32 ? C::TM : (kVals >= 16 ? 1 : 16 / kVals);
  static_assert(C::TM % CH == 0, "epilogue chunks");
  const bool has_bias = p.ep.epi == SILGPU_EPI_BIAS || p.ep.epi == SILGPU_EPI_BIAS_SIGMOID ||
                        p.ep.epi == SILGPU_EPI_BIAS_RELU;
  const bool has_res = p.ep.res != nullptr;
  float bv[C::TN];
#pragma unroll
  for (int j = 0; j < C::TN; ++j) {
    const int col = n0 + wn * C::TN * MI + j * MI + lm;
    bv[j] = has_bias && (!EDGE || col < N) ? p.ep.bias[col % p.ep.bias_len] : 0.0f;
  }
  float rv[2][CH][F::R][C::TN];
  auto load_res = [&](int c, float (&dst)[CH][F::R][C::TN]) {
#pragma unroll
    for (int ii = 0; ii < CH; ++ii)
#pragma unroll
      for (int r = 0; r < F::R; ++r) {
        const int row = m0 + wm * C::TM * MI + (c * CH + ii) * MI + F::row(lane, r);
#pragma unroll
        for (int j = 0; j < C::TN; ++j) {
          const int col = n0 + wn * C::TN * MI + j * MI + lm;
          dst[ii][r][j] = has_res && (!EDGE || (row < M && col < N))
                              ? p.ep.res[int64_t(row) * p.ep.ldr + col]
                              : 0.0f;
        }
      }
  };
  load_res(0, rv[0]);
#pragma unroll
  for (int c = 0; c < C::TM / CH; ++c) {
    if (c + 1 < C::TM / CH) load_res(c + 1, rv[(c + 1) & 1]);
#pragma unroll
    for (int ii = 0; ii < CH; ++ii) {
      const int i = c * CH + ii;
#pragma unroll
      for (int r = 0; r < F::R; ++r) {
        const int row = m0 + wm * C::TM * MI + i * MI + F::row(lane, r);
        if (EDGE && row >= M) continue;
        float *__restrict__ crow = Cp + int64_t(row) * p.ldc;
#pragma unroll
        for (int j = 0; j < C::TN; ++j) {
          const int col = n0 + wn * C::TN * MI + j * MI + lm;
          if (EDGE && col >= N) continue;
          crow[col] = apply_epi_vals(acc[i][j][r], bv[j], rv[c & 1][ii][r][j], p.ep);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ---- small-M SGEMM (M <= 32) -----------------------------------------------
//
// C = A * B with at most 32 rows of A is bound by reading B once (2M flops per
// B element; at M = 32 about 15 flop/byte, below the fp32 ridge).  A
// wavefront computes a 32 x 32Q block of C as Q accumulator sets of the
// 32x32x2 MFMA: lane (c = lane % 32, s = lane / 32) supplies A row c and B
// columns n0 + Q c + q (q < Q) of set q, so B (row-major [K][N]) arrives as
// one Q-float vector load per k row straight into the MFMA operand registers
// -- no LDS staging -- and 32 lanes read 128Q contiguous bytes of a row.  The
// k values of a 16-deep chunk are assigned to the two k slots as
// k = k0 + 8 s + j at MFMA step j < 8 (any assignment of k to slots adds the
// same products), so lane s reads A[c][k0 + 8s .. k0 + 8s + 7], 32
// contiguous bytes.  The four wavefronts of a workgroup take interleaved
// chunks of the workgroup's K range and add their accumulators through LDS;
// workgroups along grid y take disjoint K ranges (split K) and write raw
// partial planes ws[y][M][N] that splitk_sum_k adds.  Rows >= M and columns
// >= N read clamped in-range addresses and are never stored; k >= K reads as
// zero in both operands.
// TB: B is [N][K] (k contiguous): lane column n reads 8 consecutive k.
// VA: A rows 16-byte aligned (lda % 4 == 0): two float4 loads per chunk.
// VB (TB only): B rows 16-byte aligned: two float4 loads per column.
constexpr int kSkWaves = 4;
constexpr int kSkChunk = 16;  // k values per chunk (8 MFMA steps x 2 slots)

template <int Q>
struct vecf;
template <>
struct vecf<1> {
  typedef float t;
  __device__ static float get(t v, int) { return v; }
};
template <>
struct vecf<2> {
  typedef float2 t;
  __device__ static float get(t v, int q) { return q == 0 ? v.x : v.y; }
};
template <>
struct vecf<4> {
  typedef float4 t;
  __device__ static float get(t v, int q) {
    return q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w;
  }
};

__device__ __forceinline__ const float *lane_at(const float *base, uint32_t lane_bytes) {
  return reinterpret_cast<const float *>(reinterpret_cast<const char *>(base) + lane_bytes);
}

template <int Q, bool TB, bool VA, bool VB>
struct skinny_chunk {
  float a[8];
  float b[Q][8];

  // Loads chunk k0 (k0 + 16 <= kend unless MASK).  arow: A row of this lane
  // (clamped); bcol: first B column of this lane (clamped so the Q columns
  // are in range).
  //
  // The unmasked loads address memory as (wave-uniform base) + (32-bit lane
  // byte offset): a_lane = (arow lda + 8 s) 4 and b_lane[q] =
  // ((bcol + q) ldb + 8 s) 4 (TB) or (8 s ldb + bcol) 4, so each load's base
  // is scalar arithmetic and the loads take the SGPR-base form, with no
  // 64-bit vector address math per load.
  template <bool MASK>
  __device__ __forceinline__ void load(const float *__restrict__ A, int64_t lda,
                                       const float *__restrict__ B, int64_t ldb, int arow,
                                       int bcol, int k0, int s, int kend, uint32_t a_lane,
                                       const uint32_t (&b_lane)[Q]) {
    if constexpr (!MASK) {
      const float *ap = lane_at(A + k0, a_lane);
      if constexpr (VA) {
        const float4 x0 = *reinterpret_cast<const float4 *>(ap);
        const float4 x1 = *reinterpret_cast<const float4 *>(ap + 4);
        a[0] = x0.x; a[1] = x0.y; a[2] = x0.z; a[3] = x0.w;
        a[4] = x1.x; a[5] = x1.y; a[6] = x1.z; a[7] = x1.w;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] = ap[j];
      }
      if constexpr (!TB) {
        typedef typename vecf<Q>::t V;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const V v = *reinterpret_cast<const V *>(lane_at(B + int64_t(k0 + j) * ldb, b_lane[0]));
#pragma unroll
          for (int q = 0; q < Q; ++q) b[q][j] = vecf<Q>::get(v, q);
        }
      } else {
#pragma unroll
        for (int q = 0; q < Q; ++q) {
          const float *bp = lane_at(B + k0, b_lane[q]);
          if constexpr (VB) {
            const float4 x0 = *reinterpret_cast<const float4 *>(bp);
            const float4 x1 = *reinterpret_cast<const float4 *>(bp + 4);
            b[q][0] = x0.x; b[q][1] = x0.y; b[q][2] = x0.z; b[q][3] = x0.w;
            b[q][4] = x1.x; b[q][5] = x1.y; b[q][6] = x1.z; b[q][7] = x1.w;
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) b[q][j] = bp[j];
          }
        }
      }
      return;
    }
    const int kb = k0 + 8 * s;
    const float *ap = A + int64_t(arow) * lda;
    if constexpr (VA && !MASK) {
      const float4 x0 = *reinterpret_cast<const float4 *>(ap + kb);
      const float4 x1 = *reinterpret_cast<const float4 *>(ap + kb + 4);
      a[0] = x0.x; a[1] = x0.y; a[2] = x0.z; a[3] = x0.w;
      a[4] = x1.x; a[5] = x1.y; a[6] = x1.z; a[7] = x1.w;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = kb + j;
        const float v = ap[MASK ? min(k, kend - 1) : k];
        a[j] = (!MASK || k < kend) ? v : 0.0f;
      }
    }
    if constexpr (!TB) {
      typedef typename vecf<Q>::t V;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = kb + j;
        const V v = *reinterpret_cast<const V *>(B + int64_t(MASK ? min(k, kend - 1) : k) * ldb +
                                                 bcol);
#pragma unroll
        for (int q = 0; q < Q; ++q) b[q][j] = (!MASK || k < kend) ? vecf<Q>::get(v, q) : 0.0f;
      }
    } else {
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const float *bp = B + int64_t(bcol + q) * ldb;
        if constexpr (VB && !MASK) {
          const float4 x0 = *reinterpret_cast<const float4 *>(bp + kb);
          const float4 x1 = *reinterpret_cast<const float4 *>(bp + kb + 4);
          b[q][0] = x0.x; b[q][1] = x0.y; b[q][2] = x0.z; b[q][3] = x0.w;
          b[q][4] = x1.x; b[q][5] = x1.y; b[q][6] = x1.z; b[q][7] = x1.w;
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int k = kb + j;
            const float v = bp[MASK ? min(k, kend - 1) : k];
            b[q][j] = (!MASK || k < kend) ? v : 0.0f;
          }
        }
      }
    }
  }

  __device__ __forceinline__ void mma(floatx16 (&acc)[Q]) const {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int q = 0; q < Q; ++q)
        acc[q] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], b[q][j], acc[q], 0, 0, 0);
  }
};

template <int Q, bool TB, bool VA, bool VB>
__global__ __launch_bounds__(kSkWaves *kWave) void sgemm_skinny_k(gemm_args p) {
  constexpr int U = Q == 4 ? 2 : 4;  // chunks in flight per wavefront
  constexpr int STRIDE = kSkChunk * kSkWaves;
  static_assert(16 % kSkWaves == 0 && kSkWaves * Q * 16 * kWave * 4 <= 65536, "LDS");
  __shared__ float red[kSkWaves][Q * 16][kWave];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int c = lane % 32, s = lane / 32;
  const int M = p.M, N = p.N, K = p.K;
  const int n0 = blockIdx.x * (32 * Q);
  const int arow = min(c, M - 1);
  int bcol = n0 + Q * c;
  if (bcol + Q > N) bcol = 0;  // whole vector out of range (N % Q == 0 when Q > 1)
  const int kbeg = blockIdx.y * p.klen;
  const int kend = min(K, kbeg + p.klen);
  const uint32_t a_lane = (uint32_t(arow) * uint32_t(p.lda) + 8u * uint32_t(s)) * 4u;
  uint32_t b_lane[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q)
    b_lane[q] = TB ? (uint32_t(bcol + q) * uint32_t(p.ldb) + 8u * uint32_t(s)) * 4u
                   : (8u * uint32_t(s) * uint32_t(p.ldb) + uint32_t(bcol)) * 4u;

  floatx16 acc[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[q][r] = 0.0f;

  // This wavefront's chunks start at k0 + i * STRIDE; the first nf are full.
  // Software pipeline: U chunks are in flight while the oldest is multiplied.
  const int k0 = kbeg + kSkChunk * wave;
  const int nf = kend - k0 >= kSkChunk ? (kend - k0 - kSkChunk) / STRIDE + 1 : 0;
  skinny_chunk<Q, TB, VA, VB> ch[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (u < nf)
      ch[u].template load<false>(p.A, p.lda, p.B, p.ldb, arow, bcol, k0 + u * STRIDE, s, kend,
                                 a_lane, b_lane);
  int i = 0;
  for (; i + U <= nf; i += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ch[u].mma(acc);
      if (i + u + U < nf)
        ch[u].template load<false>(p.A, p.lda, p.B, p.ldb, arow, bcol,
                                   k0 + (i + u + U) * STRIDE, s, kend, a_lane, b_lane);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (i + u < nf) ch[u].mma(acc);
  const int kt = k0 + nf * STRIDE;  // a partial last chunk, if any
  if (kt < kend) {
    skinny_chunk<Q, TB, VA, VB> t;
    t.template load<true>(p.A, p.lda, p.B, p.ldb, arow, bcol, kt, s, kend, a_lane, b_lane);
    t.mma(acc);
  }

  // Add the wavefronts' accumulators: every wavefront parks its sets in LDS,
  // then wavefront w finishes registers RPW w .. RPW w + RPW - 1 of every
  // set; register r of lane (c, s) is row 8 (r / 4) + 4 s + r % 4, column
  // n0 + Q c + q -- for Q = 4 one float4 of C per row.
#pragma unroll
  for (int q = 0; q < Q; ++q)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][q * 16 + r][lane] = acc[q][r];
  __syncthreads();
  const bool split = gridDim.y > 1;
  float *W = split ? p.ws + int64_t(blockIdx.y) * M * N : p.C;
  const int64_t ldw = split ? N : p.ldc;
  const int col = n0 + Q * c;
  if (col >= N) return;
  const bool vst = Q == 4 && (ldw & 3) == 0 && aligned16_dev(W);
  constexpr int RPW = 16 / kSkWaves;
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = RPW * wave + i;
    const int row = 8 * (r / 4) + 4 * s + r % 4;
    if (row >= M) continue;
    float v[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      v[q] = red[0][q * 16 + r][lane];
#pragma unroll
      for (int w = 1; w < kSkWaves; ++w) v[q] += red[w][q * 16 + r][lane];
      if (!split) v[q] = apply_epi(v[q], row, col + q, p.ep);
    }
    float *dst = W + int64_t(row) * ldw + col;
    if constexpr (Q == 4) {
      if (vst) {
        *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
        continue;
      }
    }
#pragma unroll
    for (int q = 0; q < Q; ++q) dst[q] = v[q];
  }
}

// ---- SGEMM with LDS-direct operand loads (BM x BN x BK tiles: 256 x 256,
// 128 x 128, 128 x 64)
//
// Full tiles only (M, N multiples of BM, BN, K range a multiple of BK,
// 16-byte aligned operands): every lane's 16-byte global_load_lds_dwordx4
// stays in bounds, so no lane needs masking.  The load engine writes each
// wave's 64 x 16 bytes to one contiguous 1 KB LDS window (lane L at 16 L),
// with no staging registers and no ds_write; the layout is chosen through
// which global chunk each lane fetches.  An operand tile of extent X (BM for
// A, BN for B) by BK takes X * BK / 256 windows either way:
//   - contiguous in K (A, or B transposed): a window holds 16 rows x 16 k,
//     window kh * X/16 + rg holding rows 16 rg.. and k 16 kh..; the 16-byte
//     chunk of (row rr, k quad kq) sits at position rr*4 + (kq ^ ((rr/2) & 3));
//   - contiguous in M or N (A transposed, or B): X = 256 one k row per
//     window, pitch 260 floats; X = 128 two k rows per window (lanes 0-31
//     the even row, 32-63 the odd one), pitch 264; X = 64 four k rows per
//     window (lanes 16p .. 16p+15 row p), pitch 272.
// MFMA step j of a 16-deep k block puts k = 4g + j in the k slot g = lane/16
// of both operands (any assignment of k to slots sums the same products), so
// a K-contiguous operand is read with one ds_read_b128 per 16-row block and
// k block -- lane (r, g) takes k = 4g .. 4g+3 of row r, one value for each of
// the four steps -- and an M/N-contiguous one with one ds_read_b32 per block
// and step.  LDS on gfx950 serves ds_read_b32 one half-wave per pass over 32
// banks and ds_read_b128 16 lanes per pass (equal lane bit 5 and equal
// parity of lane bits 2-4) over 64 banks, as measured with the bank-conflict
// counter; the swizzle and pitches make every read conflict-free under that
// model (tests/test_gemm_layout.py).  256 x 256: 8 waves (2 x 4) of 128 x 64;
// 128 x 128: 4 waves (2 x 2) of 64 x 64; 128 x 64: 4 waves of 64 x 32, or 8
// of 64 x 16 for launches of at most one workgroup per CU.  The
// next K tile's loads are issued before the current tile is multiplied, and
// one s_waitcnt + barrier ends each tile.  256 x 128 tiles run three 16-deep
// stages (75 KB of LDS, two workgroups per CU), so each barrier waits only
// for the stage consumed next while one more loads; 256 x 256 tiles (8
// waves) four stages (130 KB); the smaller tiles two stages, 32 deep where
// K allows (four 16-deep stages measured slower for them: 2048^3 123.9
// against 126.2 TFLOP/s with 128 x 64 tiles).
constexpr int kDtlBK = 16;  // K granularity of the path (BK = 16 or 32)
// Leading dimensions below 2^26 floats keep a window lane's 32-bit byte
// offset (at most 15 rows of the operand) in range.
constexpr int64_t kDtlMaxLd = int64_t(1) << 26;

// Pitch (floats) of an M/N-contiguous window for a tile extent X: one k row
// per window for 256, two for 128, four for 64 (the rows of one window at
// 0, X, 2X, ..; consecutive windows 16 banks apart, so a ds_read_b32 half-wave
// over k rows 4 apart is conflict-free).
template <int X>
constexpr int dtl_pitch() {
  return X == 256 ? 260 : X == 128 ? 264 : 272;
}

// BM x BN tiles, NW waves in a 2 x NW/2 grid: 256 x 128 with 4 waves of 128
// x 64 (two workgroups per CU, so two waves per SIMD), 256 x 256 with 8
// waves of 128 x 64 (one workgroup per CU); 128 x 128 with 4 waves of 64 x
// 64; 128 x 64 with 4 waves of 64 x 32 or (BK = 32) 8 waves of 64 x 16.
template <int BM, int BN, int BK, int NW = (BM == 256 ? 8 : 4), int NS = 2>
struct dtl_cfg {
  static constexpr int WM = 2, WN = NW / 2;
  static constexpr int kThreads = WM * WN * kWave;
  static constexpr int TM = BM / WM / 16, TN = BN / WN / 16;  // 16x16 blocks per wave
  static constexpr int kWinA = BM * BK / 256, kWinB = BN * BK / 256;  // windows per operand
  // floats per operand tile (>= the K-contiguous 256 per window)
  static constexpr int kOperandA = kWinA * dtl_pitch<BM>();
  static constexpr int kOperandB = kWinB * dtl_pitch<BN>();
  static constexpr int kStage = kOperandA + kOperandB;
  static constexpr int kLdsBytes = NS * kStage * 4;  // static, NS arrays of kStage floats
  // Waves per SIMD the register allocation aims at: one 8-wave workgroup per
  // CU (LDS allows no second) for 256 x 256, two 4-wave workgroups for 256 x
  // 128, three for the smaller tiles.  Without it the compiler squeezes the 256 tile toward
  // three waves and serialises the first fragment reads of every K tile.
  static constexpr int kWavesPerEU = (BM == 256 && BN == 256) ? NW / 4 : BM == 256 ? 2 : 3;
  static_assert(BK % kDtlBK == 0 && kWinA % (WM * WN) == 0 && kWinB % (WM * WN) == 0,
                "windows per wave");
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
};

// One 16-byte LDS-direct load per lane (global_load_lds_dwordx4): the
// data goes from memory straight into LDS at lds_dst + 16 * lane.
__device__ __forceinline__ void dtl16(const float *src, float *lds_dst) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                   (__attribute__((address_space(3))) void *)lds_dst, 16, 0, 0);
}

// The same load in its SGPR-base form: address = sbase (uniform, SGPRs) +
// voff (32-bit, per lane).  The compiler only emits the 64-bit VGPR-address
// form for the builtin, which costs one vector add per load and K tile; this
// form advances the K tile with scalar adds alone (8192^3: 144.1 -> 147.2
// TFLOP/s, MI355X).  M0 holds the LDS destination; one wait state separates
// its write from the load.  M0 is otherwise unused by this kernel (gfx9 LDS
// instructions do not read it), so clobbering it here is safe.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dtl16_s(const float *sbase, uint32_t voff, float *lds_dst) {
  const uint32_t m0v = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) float *)lds_dst));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(m0v),
               "v"(voff), "s"(sbase)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Source of lane `lane` for window w of an operand tile of extent X starting
// at x0 (rows x0.. of a [rows][K] operand when KCONTIG, else columns x0.. of
// a [K][cols] operand; k relative to the tile).
template <bool KCONTIG, int X>
__device__ __forceinline__ const float *dtl_src(const float *base, int64_t ld, int x0, int w,
                                                int lane) {
  if constexpr (KCONTIG) {
    const int rr = lane / 4, kq = (lane % 4) ^ ((rr / 2) & 3);
    const int rg = w % (X / 16), kh = w / (X / 16);
    return base + int64_t(x0 + 16 * rg + rr) * ld + 16 * kh + 4 * kq;
  } else if constexpr (X == 256) {
    return base + int64_t(w) * ld + x0 + 4 * lane;
  } else if constexpr (X == 128) {
    return base + int64_t(2 * w + lane / 32) * ld + x0 + 4 * (lane % 32);
  } else {
    return base + int64_t(4 * w + lane / 16) * ld + x0 + 4 * (lane % 16);
  }
}
// The same source split into a part uniform over the wave (`uni`, elements
// from the operand base: window w depends only on the wave) and a lane part
// (`lane_bytes`, 32-bit), for the SGPR-base form of the load (dtl16_s):
// advancing the K tile then costs scalar adds only, and no vector
// instruction competes with the MFMAs for issue.  The host keeps
// 16 * ld * 4 bytes below 2^32.
template <bool KCONTIG, int X>
__device__ __forceinline__ void dtl_src_split(int64_t ld, int x0, int w, int lane, int64_t &uni,
                                              uint32_t &lane_bytes) {
  if constexpr (KCONTIG) {
    const int rr = lane / 4, kq = (lane % 4) ^ ((rr / 2) & 3);
    const int rg = w % (X / 16), kh = w / (X / 16);
    uni = int64_t(x0 + 16 * rg) * ld + 16 * kh;
    lane_bytes = (uint32_t(rr) * uint32_t(ld) + 4u * uint32_t(kq)) * 4u;
  } else if constexpr (X == 256) {
    uni = int64_t(w) * ld + x0;
    lane_bytes = 16u * uint32_t(lane);
  } else if constexpr (X == 128) {
    uni = int64_t(2 * w) * ld + x0;
    lane_bytes = (uint32_t(lane / 32) * uint32_t(ld) + 4u * uint32_t(lane % 32)) * 4u;
  } else {
    uni = int64_t(4 * w) * ld + x0;
    lane_bytes = (uint32_t(lane / 16) * uint32_t(ld) + 4u * uint32_t(lane % 16)) * 4u;
  }
}
template <bool KCONTIG, int X>
__device__ __forceinline__ int dtl_window(int w) {
  return KCONTIG ? w * 256 : w * dtl_pitch<X>();
}
// LDS offset (floats) of element (x, k) of an operand tile of extent X.
template <bool KCONTIG, int X>
__device__ __forceinline__ int dtl_elem(int x, int k) {
  if constexpr (KCONTIG) {
    return ((k / 16) * (X / 16) + x / 16) * 256 +
           ((x % 16) * 4 + (((k % 16) / 4) ^ (((x % 16) / 2) & 3))) * 4 + (k % 4);
  } else if constexpr (X == 256) {
    return k * dtl_pitch<X>() + x;
  } else if constexpr (X == 128) {
    return (k / 2) * dtl_pitch<X>() + 128 * (k % 2) + x;
  } else {
    return (k / 4) * dtl_pitch<X>() + 64 * (k % 4) + x;
  }
}

// s_waitcnt vmcnt(N) lgkmcnt(0), expcnt not waited (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));
}

// Third word of a raw buffer resource descriptor: 32-bit data format, no
// swizzle.
constexpr int kRawRsrcWord3 = 0x00020000;

// Sixteen bytes of zeros in device memory: the source of the LDS-direct
// loads of convolution taps that fall into the padding.  Never written.
__device__ __attribute__((aligned(16))) float conv_zero_page[4];

// KG > 1: the workgroup is KG groups of NWV waves.  Group g runs the tile's
// K loop over the g-th of KG equal parts of the workgroup's K range, with
// its own LDS stages, and the groups' accumulators are added through LDS at
// the end (group 0 + group 1 + ...), so a product needs no second launch to
// add K splits where KG parts fill the CU.  Every group runs the same number
// of K tiles and so meets every barrier; the host keeps each K range a
// multiple of KG * BK.
template <int BM, int BN, int BK, int NWV, int NS, bool TA, bool TB, bool CONV = false, int KG = 1>
__global__ __launch_bounds__((dtl_cfg<BM, BN, BK, NWV, NS>::kThreads * KG))
__attribute__((amdgpu_waves_per_eu(dtl_cfg<BM, BN, BK, NWV, NS>::kWavesPerEU,
                                   dtl_cfg<BM, BN, BK, NWV, NS>::kWavesPerEU))) void sgemm_dtl_k(gemm_args p) {
  using D = dtl_cfg<BM, BN, BK, NWV, NS>;
  static_assert(NS >= 2 && NS <= 4, "stages");
  static_assert(KG >= 1 && (KG == 1 || !CONV), "K groups");
  static_assert(D::kLdsBytes * KG <= 160 * 1024, "LDS");
  using F = mfma<16>;
  constexpr int TM = D::TM, TN = D::TN, NW = D::WM * D::WN;
  constexpr int WPA = D::kWinA / NW, WPB = D::kWinB / NW;  // windows per wave
  constexpr bool AK = !TA, BKc = TB;  // operand contiguous in K
  // NS stages as NS LDS objects: alias analysis then sees that the loads
  // into one stage cannot touch the fragment reads from another, and the
  // compiler adds no wait for the prefetch before those reads.  Tile kt
  // reads stage kt % NS and issues the loads of tile kt + NS - 1.
  __shared__ __attribute__((aligned(16))) float lds0_[KG * D::kStage];
  __shared__ __attribute__((aligned(16))) float lds1_[KG * D::kStage];
  __shared__ __attribute__((aligned(16))) float lds2_[NS > 2 ? KG * D::kStage : 4];
  __shared__ __attribute__((aligned(16))) float lds3_[NS > 3 ? KG * D::kStage : 4];
  // The wave index through readfirstlane: the compiler then keeps it, and
  // every window and LDS address derived from it, in SGPRs.
  // (Not for the convolution: its gathers measured 1.5-2% slower so.)
  const int t = threadIdx.x, lane = t % kWave;
  const int wave_all = CONV ? t / kWave : __builtin_amdgcn_readfirstlane(t / kWave);
  const int grp = KG == 1 ? 0 : wave_all / NW;  // K group
  const int wave = KG == 1 ? wave_all : wave_all % NW;  // wave within the group
  float *const lds0 = lds0_ + (KG == 1 ? 0 : grp * D::kStage);
  float *const lds1 = lds1_ + (KG == 1 ? 0 : grp * D::kStage);
  float *const lds2 = lds2_ + (KG == 1 || NS <= 2 ? 0 : grp * D::kStage);
  float *const lds3 = lds3_ + (KG == 1 || NS <= 3 ? 0 : grp * D::kStage);
  const int wm = wave / D::WN, wn = wave % D::WN;
  int tm, tn;
  tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int64_t zo = blockIdx.z / p.binner, zi = blockIdx.z % p.binner;
  const float *__restrict__ A = p.A + zo * p.sA2 + zi * p.sA;
  const float *__restrict__ B = p.B + zo * p.sB2 + zi * p.sB;
  float *__restrict__ Cp = p.C + zo * p.sC2 + zi * p.sC;
  const int M = p.M, N = p.N;
  const int kbeg0 = blockIdx.y * p.klen;
  const int kend = min(p.K, kbeg0 + p.klen);
  // K % BK == 0 on this path; with KG groups each takes KT whole tiles.
  const int KT = kend > kbeg0 ? (kend - kbeg0) / BK / KG : 0;
  const int kbeg = kbeg0 + grp * KT * BK;
  // This wave loads windows wave + q*NW (q < WPA, WPB) of each operand.
  int64_t a_uni[WPA], b_uni[WPB];
  uint32_t a_lane[WPA], b_lane[WPB];
#pragma unroll
  for (int q = 0; q < WPA; ++q) {
    if constexpr (CONV) {
      a_uni[q] = 0;
      a_lane[q] = 0;
    } else {
      dtl_src_split<AK, BM>(p.lda, m0, wave + q * NW, lane, a_uni[q], a_lane[q]);
    }
  }
  const float *b_src[WPB];  // the convolution's B: per-lane pointers
#pragma unroll
  for (int q = 0; q < WPB; ++q) {
    dtl_src_split<BKc, BN>(p.ldb, n0, wave + q * NW, lane, b_uni[q], b_lane[q]);
    b_src[q] = CONV ? dtl_src<BKc, BN>(B, p.ldb, n0, wave + q * NW, lane) : nullptr;
  }
  // Advance of one K tile for each operand.
  const int64_t a_step = AK ? BK : int64_t(BK) * p.lda;
  const int64_t b_step = BKc ? BK : int64_t(BK) * p.ldb;
  constexpr int kBOff = D::kOperandA;
  // Convolution (CONV: A is the implicit im2col matrix of an NHWC input,
  // k = (kh * K + kw) * C_in + ci, C_in % BK == 0).  Every K tile then lies
  // in one tap (kh, kw), the same for the whole workgroup, and a lane's
  // channel offset within the tile is fixed: a window lane reads 4
  // channels of its pixel shifted by the tap, or the zero page where the
  // shifted pixel is padding.  issue() is called once per K tile, in order,
  // and steps the tap walk (tci, tkw, tkh) by BK.
  int64_t cv_base[CONV ? WPA : 1];
  int cv_oh[CONV ? WPA : 1], cv_ow[CONV ? WPA : 1], cv_off[CONV ? WPA : 1];
  int tci = 0, tkw = 0, tkh = 0;
  // The zero page's address, read once: as a global symbol it would be
  // reloaded through the GOT at every load, each reload a scalar load whose
  // wait (lgkmcnt 0) also waits for the fragment reads in flight (ResNet mid
  // and deep layers 90.5 -> 92.0 and 86.6 -> 87.9 TFLOP/s).  Measured and
  // not kept: a per-lane bit mask of the valid taps instead of the bounds
  // compares (fewer vector instructions, yet 87.4 and 84.4).
  const float *zero_src = conv_zero_page;
  if constexpr (CONV) asm volatile("" : "+s"(zero_src));
  if constexpr (CONV) {
    const int hw = p.cv_h * p.cv_w;
#pragma unroll
    for (int q = 0; q < WPA; ++q) {
      const int w = wave + q * NW, rr = lane / 4, kq = (lane % 4) ^ ((rr / 2) & 3);
      const int m = p.cv_m0 + m0 + 16 * (w % (BM / 16)) + rr;  // full tiles only
      const int n = m / hw, rem = m - n * hw;
      cv_oh[q] = rem / p.cv_w;
      cv_ow[q] = rem - cv_oh[q] * p.cv_w;
      cv_base[q] =
          ((int64_t(n) * p.cv_h + cv_oh[q] - p.cv_pad) * p.cv_w + cv_ow[q] - p.cv_pad) * p.cv_cin;
      cv_off[q] = 16 * (w / (BM / 16)) + 4 * kq;
    }
    const int khw = kbeg / p.cv_cin;
    tci = kbeg - khw * p.cv_cin;
    tkh = khw / p.cv_k;
    tkw = khw - tkh * p.cv_k;
  }
  auto issue = [&](int kt, float *S) {
    const int64_t k = int64_t(kbeg / BK + kt);
    if constexpr (CONV) {
      const int tap = (tkh * p.cv_w + tkw) * p.cv_cin + tci;
#pragma unroll
      for (int q = 0; q < WPA; ++q) {
        const int ih = cv_oh[q] + tkh - p.cv_pad, iw = cv_ow[q] + tkw - p.cv_pad;
        const bool in = unsigned(ih) < unsigned(p.cv_h) && unsigned(iw) < unsigned(p.cv_w);
        dtl16(in ? A + cv_base[q] + tap + cv_off[q] : zero_src,
              S + dtl_window<true, BM>(wave + q * NW));
      }
      tci += BK;
      if (tci == p.cv_cin) {
        tci = 0;
        if (++tkw == p.cv_k) {
          tkw = 0;
          ++tkh;
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < WPA; ++q)
        dtl16_s(A + a_uni[q] + k * a_step, a_lane[q], S + dtl_window<AK, BM>(wave + q * NW));
    }
#pragma unroll
    for (int q = 0; q < WPB; ++q) {
      if constexpr (CONV)
        dtl16(b_src[q] + k * b_step, S + kBOff + dtl_window<BKc, BN>(wave + q * NW));
      else
        dtl16_s(B + b_uni[q] + k * b_step, b_lane[q],
                S + kBOff + dtl_window<BKc, BN>(wave + q * NW));
    }
  };
  typename F::acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < F::R; ++r) acc[i][j][r] = 0.0f;
  const int lm = lane % 16, kg = lane / 16;
  const int xa = wm * TM * 16 + lm, xb = wn * TN * 16 + lm;
  // Fragments.  K-contiguous operand: four floats (steps 0-3) per 16-row
  // block, double-buffered over k blocks; M/N-contiguous: one float per block
  // for one step, double-buffered over steps.
  constexpr int kSteps = BK / 4, kBlocks = BK / 16;
  float a4[2][AK ? TM : 1][4], b4[2][BKc ? TN : 1][4];
  float a1[2][AK ? 1 : TM], b1[2][BKc ? 1 : TN];
  auto read4 = [](float (&dst)[4], const float *src) {
    const float4 v = *reinterpret_cast<const float4 *>(src);
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
    dst[3] = v.w;
  };
  // Reads for k block kh (K-contiguous operands) or step st (M/N-contiguous).
  auto read_block = [&](const float *Sa, const float *Sb, int kh) {
    if constexpr (AK) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
        read4(a4[kh & 1][i], Sa + dtl_elem<true, BM>(xa + 16 * i, 16 * kh + 4 * kg));
    }
    if constexpr (BKc) {
#pragma unroll
      for (int j = 0; j < TN; ++j)
        read4(b4[kh & 1][j], Sb + dtl_elem<true, BN>(xb + 16 * j, 16 * kh + 4 * kg));
    }
  };
  auto read_step = [&](const float *Sa, const float *Sb, int st) {
    const int k = 16 * (st / 4) + 4 * kg + st % 4;
    if constexpr (!AK) {
#pragma unroll
      for (int i = 0; i < TM; ++i) a1[st & 1][i] = Sa[dtl_elem<false, BM>(xa + 16 * i, k)];
    }
    if constexpr (!BKc) {
#pragma unroll
      for (int j = 0; j < TN; ++j) b1[st & 1][j] = Sb[dtl_elem<false, BN>(xb + 16 * j, k)];
    }
  };
  auto fa = [&](int st, int i) -> float {
    if constexpr (AK) return a4[(st / 4) & 1][i][st % 4];
    else return a1[st & 1][i];
  };
  auto fb = [&](int st, int j) -> float {
    if constexpr (BKc) return b4[(st / 4) & 1][j][st % 4];
    else return b1[st & 1][j];
  };
  // Waits until this wave's loads of tile `next` have landed, leaving the
  // loads of the tiles after it (at most NS - 2, kDma instructions each) in
  // flight, then the barrier makes every wave's loads visible.
  constexpr int kDma = WPA + WPB;
  auto land = [&](int next) {
    if constexpr (NS == 2) {
      wait_vm_lgkm0<0>();
    } else {
      const int after = min(KT - 1, next + NS - 2) - next;
      if (after >= 2)
        wait_vm_lgkm0<2 * kDma>();
      else if (after == 1)
        wait_vm_lgkm0<kDma>();
      else
        wait_vm_lgkm0<0>();
    }
    // The barrier as an opaque instruction: the compiler puts a full
    // s_waitcnt 0 before every s_barrier it sees on this target, and a
    // workgroup fence waits for the LDS-direct loads too (they write LDS), so
    // either would also wait for the prefetch of the tiles after `next`.  The
    // waits above have landed this wave's part of tile `next` in LDS and
    // completed its reads of the stage the next loads overwrite; the
    // "memory" clobber keeps the compiler from moving LDS accesses across.
    asm volatile("s_barrier" ::: "memory");
  };
  if (KT > 0) {
    issue(0, lds0);
    if constexpr (NS >= 3) {
      if (1 < KT) issue(1, lds1);
    }
    if constexpr (NS == 4) {
      if (2 < KT) issue(2, lds2);
    }
    land(0);
  }
  // One K tile: fragments from stage Sa while tile kt + NS - 1 loads into
  // Snext (the stage the previous tile read).  The loads are issued after the
  // first fragment reads: where the compiler cannot tell the stages apart
  // (at the loop head) it waits for all loads before reading, and then those
  // are loads issued one tile or more earlier, not the ones just issued.
  auto tile = [&](const float *Sa, float *Snext, int kt) {
    const float *Sb = Sa + kBOff;
    read_block(Sa, Sb, 0);
    read_step(Sa, Sb, 0);
    __builtin_amdgcn_sched_barrier(0);  // all first-step reads in flight together
    if (kt + NS - 1 < KT) issue(kt + NS - 1, Snext);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      // Row block 0 first: the wait for this step's fragments (the compiler
      // waits for all outstanding LDS reads) then comes before the next
      // reads are issued, and the remaining MFMAs of the step cover them.
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[0][j] = F::run(fa(st, 0), fb(st, j), acc[0][j]);
      __builtin_amdgcn_sched_barrier(0);
      if (st + 1 < kSteps) read_step(Sa, Sb, st + 1);
      if (st % 4 == 0 && st / 4 + 1 < kBlocks) read_block(Sa, Sb, st / 4 + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 1; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = F::run(fa(st, i), fb(st, j), acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
    land(kt + 1);
  };
  if constexpr (NS == 2) {
    for (int kt = 0; kt < KT; kt += 2) {
      tile(lds0, lds1, kt);
      if (kt + 1 < KT) tile(lds1, lds0, kt + 1);
    }
  } else if constexpr (NS == 3) {
    for (int kt = 0; kt < KT; kt += 3) {
      tile(lds0, lds2, kt);
      if (kt + 1 < KT) tile(lds1, lds0, kt + 1);
      if (kt + 2 < KT) tile(lds2, lds1, kt + 2);
    }
  } else {
    for (int kt = 0; kt < KT; kt += 4) {
      tile(lds0, lds3, kt);
      if (kt + 1 < KT) tile(lds1, lds0, kt + 1);
      if (kt + 2 < KT) tile(lds2, lds1, kt + 2);
      if (kt + 3 < KT) tile(lds3, lds2, kt + 3);
    }
  }
  if constexpr (KG > 1) {
    // Groups 1.. hand their accumulators to group 0 through LDS, in group
    // order, over the stage buffers (every wave's reads of them are done
    // at the first barrier): slot (i, j) of wave w, lane l at float4
    // ((i * TN + j) * NW + w) * 64 + l, so each store and load of a wave is
    // 1 KiB of consecutive LDS.
    static_assert(F::R == 4 && TM * TN * NW * kWave * 4 <= D::kStage * KG, "K-group exchange");
    float4 *const red = reinterpret_cast<float4 *>(lds0_);
    const int slot = wave * kWave + lane;
#pragma unroll
    for (int gs = 1; gs < KG; ++gs) {
      __syncthreads();
      if (grp == gs) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            red[(i * TN + j) * NW * kWave + slot] =
                make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      }
      __syncthreads();
      if (grp == 0) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const float4 v = red[(i * TN + j) * NW * kWave + slot];
            acc[i][j][0] += v.x;
            acc[i][j][1] += v.y;
            acc[i][j][2] += v.z;
            acc[i][j][3] += v.w;
          }
      }
    }
    if (grp != 0) return;
  }
  if (gridDim.y > 1) {
    // The raw accumulators to plane y through a buffer descriptor based at
    // this tile: one 32-bit lane offset, each store's row and column step in
    // the scalar offset (the host splits K here only where BM * N * 4 <
    // 2^30).  Against per-element 64-bit addresses this measured 1.3-3.6%
    // faster on products that do not split, from the block layout the
    // compiler then gives the K loop (2048^3 132.9 -> 128.4 us).
    const __amdgpu_buffer_rsrc_t w = __builtin_amdgcn_make_buffer_rsrc(
        p.ws + int64_t(blockIdx.y) * M * N + int64_t(m0) * N + n0, 0, 0x7fffffff, kRawRsrcWord3);
    const int lane_b = ((wm * TM * 16 + F::row(lane, 0)) * N + wn * TN * 16 + lm) * 4;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < F::R; ++r)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][r]), w, lane_b,
                                                ((i * 16 + r) * N + j * 16) * 4, 0);
    return;
  }
  // The epilogue's bias values (one per column block) and residual values
  // are loaded before the stores that use them: the whole tile's at once
  // where they take at most 32 registers per lane, else CH row blocks (at
  // most 16 values) at a time with the next chunk's loads issued before the
  // current chunk is stored.  A load-then-store per element would pay one
  // memory latency per row block (out-proj 2048x768x768 with bias and
  // residual on 192 workgroups: 50 us against 31 without an epilogue).
  constexpr int kVals = F::R * TN;
  constexpr int CH = TM * kVals <= 32 ? TM : (kVals >= 16 ? 1 : 16 / kVals);
  static_assert(TM % CH == 0, "epilogue chunks");
  const bool has_bias = p.ep.epi == SILGPU_EPI_BIAS || p.ep.epi == SILGPU_EPI_BIAS_SIGMOID ||
                        p.ep.epi == SILGPU_EPI_BIAS_RELU;
  const bool has_res = p.ep.res != nullptr;
  float bv[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j)
    bv[j] = has_bias ? p.ep.bias[(n0 + wn * TN * 16 + j * 16 + lm) % p.ep.bias_len] : 0.0f;
  float rv[2][CH][F::R][TN];
  auto load_res = [&](int c, float (&dst)[CH][F::R][TN]) {
#pragma unroll
    for (int ii = 0; ii < CH; ++ii)
#pragma unroll
      for (int r = 0; r < F::R; ++r) {
        const int row = m0 + wm * TM * 16 + (c * CH + ii) * 16 + F::row(lane, r);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          dst[ii][r][j] = has_res ? p.ep.res[int64_t(row) * p.ep.ldr + n0 + wn * TN * 16 +
                                             j * 16 + lm]
                                  : 0.0f;
      }
  };
  load_res(0, rv[0]);
#pragma unroll
  for (int c = 0; c < TM / CH; ++c) {
    if (c + 1 < TM / CH) load_res(c + 1, rv[(c + 1) & 1]);
#pragma unroll
    for (int ii = 0; ii < CH; ++ii) {
      const int i = c * CH + ii;
#pragma unroll
      for (int r = 0; r < F::R; ++r) {
        const int row = m0 + wm * TM * 16 + i * 16 + F::row(lane, r);
        float *__restrict__ crow = Cp + int64_t(row) * p.ldc;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int col = n0 + wn * TN * 16 + j * 16 + lm;
          crow[col] = apply_epi_vals(acc[i][j][r], bv[j], rv[c & 1][ii][r][j], p.ep);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ---- GEMV: y[1 x N] = x[1 x K] * B[K x N] -----------------------------------
//
// HBM-bound: B (K*N floats) is read once.  Pass 1: workgroup (ct, ks) covers
// 256 columns (one float4 per lane) and rows [ks*kc, (ks+1)*kc); its eight
// wavefronts take interleaved rows with eight 16-byte non-temporal loads in
// flight per lane, add their results in LDS and write one partial row
// partial[ks][ct*256 ..] to scratch.  The K split gives ~1024 workgroups to
// fill the GPU.  Pass 2 adds the partials per column.  Finishing inside
// pass 1 was measured on MI355X at 1x4096x4096 and lost every time: the
// last-workgroup pattern needs agent-scope fences (58 us per call), a packed
// (count, sum) compare-and-swap per column serialises at the memory-side
// atomic unit (50-300 us), and zero-fill + atomicAdd costs a launch as well
// (16.1 us); the second launch costs ~2 us.
constexpr int kGemvBlock = 256;  // finish kernels
constexpr int kGemvWaves = kGemvBlock / kWave;
constexpr int kGemvPartWaves = 8;  // partial kernel: 8 waves x 4 loads in flight
constexpr int kGemvPartBlock = kGemvPartWaves * kWave;
constexpr int kGemvCols = 256;  // columns per workgroup (64 lanes x float4)
constexpr int kGemvUnroll = 8;  // rows in flight per lane: every wave issues its 8 rows at once
constexpr int kGemvFinishLoads = 16;  // partial rows in flight per lane in pass 2

__device__ __forceinline__ float4 load_nt4(const float *p) {
  const float4 *q = reinterpret_cast<const float4 *>(p);
  float4 v;
  v.x = __builtin_nontemporal_load(&q->x);
  v.y = __builtin_nontemporal_load(&q->y);
  v.z = __builtin_nontemporal_load(&q->z);
  v.w = __builtin_nontemporal_load(&q->w);
  return v;
}

// VEC: N % 4 == 0, ldb % 4 == 0, B 16-byte aligned; lane owns 4 adjacent
// columns.  !VEC: lane owns columns c0 + lane + 64*q, q < 4.
template <bool VEC>
__global__ __launch_bounds__(kGemvPartBlock) void gemv_part_k(const float *__restrict__ x,
                                                              const float *__restrict__ Bm,
                                                              int64_t ldb, int64_t N, int64_t K,
                                                              int64_t kc,
                                                              float *__restrict__ partial) {
  __shared__ float4 red[kGemvPartWaves][kWave];
  // The wave index through readfirstlane: the row a wave reads is then
  // scalar, x[k] a scalar load, and each B load a uniform row base plus the
  // lane's 16-byte column offset.
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t c0 = int64_t(blockIdx.x) * kGemvCols;
  const int64_t k0 = int64_t(blockIdx.y) * kc;
  const int64_t k1 = k0 + kc < K ? k0 + kc : K;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if constexpr (VEC) {
    const int64_t col = c0 + lane * 4;
    if (col < N) {
      const float *bp = Bm + col;
      const float *bt = Bm + c0;  // the tile's first column, uniform
      const uint32_t lane_bytes = 16u * uint32_t(lane);
      int64_t k = k0 + wave;
      constexpr int U = kGemvUnroll, W = kGemvPartWaves;
      for (; k + (U - 1) * W < k1; k += U * W) {
        float4 v[U];
        float xv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          v[u] = load_nt4(lane_at(bt + (k + u * W) * ldb, lane_bytes));
          xv[u] = x[k + u * W];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          acc.x += xv[u] * v[u].x;
          acc.y += xv[u] * v[u].y;
          acc.z += xv[u] * v[u].z;
          acc.w += xv[u] * v[u].w;
        }
      }
      for (; k < k1; k += W) {
        float4 v = load_nt4(bp + k * ldb);
        float xv = x[k];
        acc.x += xv * v.x;
        acc.y += xv * v.y;
        acc.z += xv * v.z;
        acc.w += xv * v.w;
      }
    }
  } else {
    for (int64_t k = k0 + wave; k < k1; k += kGemvPartWaves) {
      const float xv = x[k];
      const float *row = Bm + k * ldb;
      const int64_t c = c0 + lane;
      if (c < N) acc.x += xv * row[c];
      if (c + 64 < N) acc.y += xv * row[c + 64];
      if (c + 128 < N) acc.z += xv * row[c + 128];
      if (c + 192 < N) acc.w += xv * row[c + 192];
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 1; w < kGemvPartWaves; ++w) {
    float4 o = red[w][lane];
    acc.x += o.x;
    acc.y += o.y;
    acc.z += o.z;
    acc.w += o.w;
  }
  // partial row ks holds N floats in the same per-lane order as the columns.
  float *prow = partial + int64_t(blockIdx.y) * (int64_t(gridDim.x) * kGemvCols) + c0;
  reinterpret_cast<float4 *>(prow)[lane] = acc;
}

// Pass 2 (used for !VEC): 64 columns per workgroup, the four wavefronts split
// the K splits.  Partial slot q of lane l in tile ct maps to column
// c0 + 4l + q (VEC) or c0 + l + 64q (!VEC).
template <bool VEC>
__global__ __launch_bounds__(kGemvBlock) void gemv_finish_k(const float *__restrict__ partial,
                                                            int64_t ks, int64_t pitch,
                                                            int64_t N, float *__restrict__ y) {
  __shared__ float red[kGemvWaves][kWave];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int64_t slot = int64_t(blockIdx.x) * kWave + lane;  // index into a partial row
  float s = 0.0f;
  if (slot < pitch) {
    int64_t j = wave;
    for (; j + 3 * kGemvWaves < ks; j += 4 * kGemvWaves) {
      float o0 = partial[j * pitch + slot];
      float o1 = partial[(j + kGemvWaves) * pitch + slot];
      float o2 = partial[(j + 2 * kGemvWaves) * pitch + slot];
      float o3 = partial[(j + 3 * kGemvWaves) * pitch + slot];
      s += o0;
      s += o1;
      s += o2;
      s += o3;
    }
    for (; j < ks; j += kGemvWaves) s += partial[j * pitch + slot];
  }
  red[wave][lane] = s;
  __syncthreads();
  if (wave != 0 || slot >= pitch) return;
  s = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
  const int64_t ct = slot / kGemvCols, within = slot % kGemvCols;
  const int64_t col = VEC ? slot : ct * kGemvCols + (within % 4) * 64 + within / 4;
  if (col < N) y[col] = s;
}

// Pass 2 for VEC: 256 columns per workgroup as float4 lanes; the four
// wavefronts take partial rows w, w+4, ... with kGemvFinishLoads loads in
// flight per lane, so the pass costs about one memory latency.
// EXACT: ks == kGemvFinishLoads * kGemvWaves (the usual 64 splits), so every
// lane issues its loads unguarded in one group.
template <bool EXACT>
__global__ __launch_bounds__(kGemvBlock) void gemv_finish_vec_k(const float *__restrict__ partial,
                                                                int64_t ks, int64_t pitch,
                                                                int64_t N, float *__restrict__ y) {
  __shared__ float4 red[kGemvWaves][kWave];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int64_t col = int64_t(blockIdx.x) * kGemvCols + lane * 4;  // < pitch
  constexpr int G = kGemvFinishLoads;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t j0 = wave; j0 < ks; j0 += int64_t(G) * kGemvWaves) {
    float4 v[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t j = j0 + int64_t(g) * kGemvWaves;
      v[g] = (EXACT || j < ks) ? *reinterpret_cast<const float4 *>(partial + j * pitch + col)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      s.x += v[g].x;
      s.y += v[g].y;
      s.z += v[g].z;
      s.w += v[g].w;
    }
  }
  red[wave][lane] = s;
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 1; w < kGemvWaves; ++w) {
    const float4 o = red[w][lane];
    s.x += o.x;
    s.y += o.y;
    s.z += o.z;
    s.w += o.w;
  }
  if (col < N) {  // N % 4 == 0: the four columns are in range together
    y[col] = s.x;
    y[col + 1] = s.y;
    y[col + 2] = s.z;
    y[col + 3] = s.w;
  }
}

// y[n] = sum_k x[k] * R[n*ldr + k]: one wavefront per output (rows of R
// contiguous).  Used for x * B^T (trans_b) and for A * v (N == 1).
template <bool VEC>
__global__ __launch_bounds__(256) void gemv_t_k(const float *__restrict__ x,
                                                int64_t incx,
                                                const float *__restrict__ R, int64_t ldr,
                                                float *__restrict__ y, int64_t incy,
                                                int64_t nrows, int64_t K) {
  const int64_t n = int64_t(blockIdx.x) * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (n >= nrows) return;
  const float *row = R + n * ldr;
  float acc = 0.0f;
  if (VEC && incx == 1) {
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    for (int64_t k = lane; k < K / 4; k += kWave) {
      float4 a = r4[k], b = x4[k];
      acc += a.x * b.x;
      acc += a.y * b.y;
      acc += a.z * b.z;
      acc += a.w * b.w;
    }
  } else {
    for (int64_t k = lane; k < K; k += kWave) acc += row[k] * x[k * incx];
  }
  acc = wave_sum(acc);
  if (lane == 0) y[n * incy] = acc;
}

// Applies an epilogue to a [M x N] block of C in place (GEMV paths).
__global__ __launch_bounds__(256) void epilogue_k(float *__restrict__ C, int64_t ldc,
                                                  int64_t M, int64_t N, epi_args ep) {
  const int64_t total = M * N;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * 256) {
    const int64_t m = i / N, n = i % N;
    C[m * ldc + n] = apply_epi(C[m * ldc + n], m, n, ep);
  }
}

// ---- host dispatch ----------------------------------------------------------

template <int BM, int BN, int BK, int WM, int WN, int MI, bool TA, bool TB, bool VEC, bool EDGE>
int launch_cfg(const gemm_args &a, int64_t batch, int splits, hipStream_t s) {
  using C = cfg<BM, BN, BK, WM, WN, MI>;
  auto kern = sgemm_mfma_k<BM, BN, BK, WM, WN, MI, TA, TB, VEC, EDGE>;
  // Once per process (a thread-safe static), before the first launch.
  static const hipError_t attr_rc =
      hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, C::kLdsBytes);
  SILGPU_HIP_CHECK(attr_rc);
  gemm_args g = a;
  g.tiles_m = static_cast<int>(cdiv(a.M, BM));
  g.tiles_n = static_cast<int>(cdiv(a.N, BN));
  g.klen = static_cast<int>(cdiv(cdiv(a.K, splits), BK) * BK);
  if (g.klen < BK) g.klen = BK;
  splits = static_cast<int>(a.K > 0 ? cdiv(a.K, g.klen) : 1);
  dim3 grid(static_cast<unsigned>(g.tiles_m * g.tiles_n), static_cast<unsigned>(splits),
            static_cast<unsigned>(batch));
  kern<<<grid, C::kThreads, C::kLdsBytes, s>>>(g);
  SILGPU_LAUNCH_CHECK("sgemm_mfma_k");
  return splits;  // >= 1: the number of K splits actually launched
}

// KG > 1 (K groups within the workgroup) needs K % (KG * BK) == 0: every
// workgroup's K range is then a whole number of KG * BK.
template <int BM, int BN, int BK, int NWV, int NS, bool TA, bool TB, int KG = 1>
int launch_dtl(const gemm_args &a, int64_t batch, int splits, hipStream_t s) {
  using D = dtl_cfg<BM, BN, BK, NWV, NS>;
  auto kern = sgemm_dtl_k<BM, BN, BK, NWV, NS, TA, TB, false, KG>;
  constexpr int kGran = BK * KG;
  SILGPU_REQUIRE(a.K % kGran == 0, "sgemm_dtl_k: K %d is not a multiple of %d", a.K, kGran);
  gemm_args g = a;
  g.tiles_m = static_cast<int>(a.M / BM);
  g.tiles_n = static_cast<int>(a.N / BN);
  // The split planes are stored with 32-bit offsets within a tile's rows.
  if (int64_t(BM) * a.N * 4 >= (int64_t(1) << 30)) splits = 1;
  g.klen = static_cast<int>(cdiv(cdiv(a.K, splits), kGran) * kGran);
  if (g.klen < kGran) g.klen = kGran;
  splits = static_cast<int>(a.K > 0 ? cdiv(a.K, g.klen) : 1);
  dim3 grid(static_cast<unsigned>(g.tiles_m * g.tiles_n), static_cast<unsigned>(splits),
            static_cast<unsigned>(batch));
  kern<<<grid, D::kThreads * KG, 0, s>>>(g);
  SILGPU_LAUNCH_CHECK("sgemm_dtl_k");
  return splits;
}

template <int BM, int BN, int BK, int WM, int WN, int MI, bool TA, bool TB>
int launch_tb(const gemm_args &a, int64_t batch, int splits, bool vec, hipStream_t s) {
  // Every split's K range is a multiple of BK except possibly the last, and
  // that one is too when K is.
  const bool edge = (a.M % BM) || (a.N % BN) || (a.K % BK);
  // Full tiles of 16-byte aligned operands: LDS-direct loads.
  if constexpr ((BM == 256 && BN == 256) || (BM == 128 && BN == 128) ||
                (BM == 128 && BN == 64)) {
    if (vec && a.M % BM == 0 && a.N % BN == 0 && a.K % kDtlBK == 0 && a.lda < kDtlMaxLd &&
        a.ldb < kDtlMaxLd) {
      if constexpr (BM == 256) {
        // The 256 x 256 plan runs as 256 x 128 tiles of 4 waves with three
        // 16-deep stages (75 KB of LDS), two workgroups per CU: each waits
        // at its own barriers while the other keeps the matrix cores busy
        // (8192^3: 142.5 TFLOP/s against 141.4 for one 256 x 256 workgroup
        // of 8 waves with four stages; 4096^3: 138.9 against 137.7, MI355X).
        return launch_dtl<BM, BN / 2, kDtlBK, 4, 3, TA, TB>(a, batch, splits, s);
      } else if constexpr (BN == 128) {
        return launch_dtl<BM, BN, kDtlBK, 4, 2, TA, TB>(a, batch, splits, s);
      } else {
        if (a.K % 32 == 0) {
          // A launch of at most one workgroup per CU runs the tile on 8
          // waves of 64 x 16 (two per SIMD, so each hides the other's
          // fragment and barrier waits); with more workgroups per CU the
          // 4 waves of 64 x 32 read fewer fragments per MFMA and win.
          // MI355X, µs, 4 waves against 8: 1024^3 (2 K splits, 256
          // workgroups) 24.9 / 24.1, 640x2560x640 27.5 / 24.6,
          // 256x1024x4096 24.7 / 23.9; 2048x768x768 (4 splits, 768
          // workgroups) 30.4 / 33.4, 2048x3072x768 76.5 / 81.4.
          const int64_t klen = cdiv(cdiv(a.K, splits), 32) * 32;
          const int64_t wgs = int64_t(a.M / BM) * (a.N / BN) * batch * cdiv(a.K, klen);
          const context *c = ctx();
          if (c && wgs <= c->cu_count)
            return launch_dtl<BM, BN, 32, 8, 2, TA, TB>(a, batch, splits, s);
          return launch_dtl<BM, BN, 32, 4, 2, TA, TB>(a, batch, splits, s);
        }
        return launch_dtl<BM, BN, kDtlBK, 4, 2, TA, TB>(a, batch, splits, s);
      }
    }
  }
  if (vec) {
    return edge ? launch_cfg<BM, BN, BK, WM, WN, MI, TA, TB, true, true>(a, batch, splits, s)
                : launch_cfg<BM, BN, BK, WM, WN, MI, TA, TB, true, false>(a, batch, splits, s);
  }
  return launch_cfg<BM, BN, BK, WM, WN, MI, TA, TB, false, true>(a, batch, splits, s);
}

template <int BM, int BN, int BK, int WM, int WN, int MI>
int launch_tiles(const gemm_args &a, int64_t batch, int splits, bool ta, bool tb, bool vec,
                 hipStream_t s) {
  if (!ta && !tb) return launch_tb<BM, BN, BK, WM, WN, MI, false, false>(a, batch, splits, vec, s);
  if (!ta && tb) return launch_tb<BM, BN, BK, WM, WN, MI, false, true>(a, batch, splits, vec, s);
  if (ta && !tb) return launch_tb<BM, BN, BK, WM, WN, MI, true, false>(a, batch, splits, vec, s);
  return launch_tb<BM, BN, BK, WM, WN, MI, true, true>(a, batch, splits, vec, s);
}

// 64 x 64 tiles on the LDS-direct kernel as two K groups of 4 waves (32 x 32
// each, 8 waves per workgroup): where 64 x 64 tiles fill the CUs once, the
// product runs in one launch with the K range halved inside each workgroup
// instead of split across workgroups and added by a second launch.
// Operands the LDS-direct loads cannot take run the register-staged 64 x 64
// tile (`k2` false).
// The same tile as four K groups of 4 waves (16 waves, 136 KB of LDS: one
// workgroup per CU, four waves per SIMD), for long K.
int launch_k4(const gemm_args &a, int64_t batch, int splits, bool ta, bool tb, bool vec,
              hipStream_t s, bool &k2) {
  k2 = vec && a.M % 64 == 0 && a.N % 64 == 0 && a.K % 128 == 0 && a.lda < kDtlMaxLd &&
       a.ldb < kDtlMaxLd;
  if (!k2) return launch_tiles<64, 64, 16, 2, 2, 16>(a, batch, splits, ta, tb, vec, s);
  if (!ta && !tb) return launch_dtl<64, 64, 32, 4, 2, false, false, 4>(a, batch, splits, s);
  if (!ta && tb) return launch_dtl<64, 64, 32, 4, 2, false, true, 4>(a, batch, splits, s);
  if (ta && !tb) return launch_dtl<64, 64, 32, 4, 2, true, false, 4>(a, batch, splits, s);
  return launch_dtl<64, 64, 32, 4, 2, true, true, 4>(a, batch, splits, s);
}
int launch_k2(const gemm_args &a, int64_t batch, int splits, bool ta, bool tb, bool vec,
              hipStream_t s, bool &k2) {
  k2 = vec && a.M % 64 == 0 && a.N % 64 == 0 && a.K % 64 == 0 && a.lda < kDtlMaxLd &&
       a.ldb < kDtlMaxLd;
  if (!k2) return launch_tiles<64, 64, 16, 2, 2, 16>(a, batch, splits, ta, tb, vec, s);
  if (!ta && !tb) return launch_dtl<64, 64, 32, 4, 2, false, false, 2>(a, batch, splits, s);
  if (!ta && tb) return launch_dtl<64, 64, 32, 4, 2, false, true, 2>(a, batch, splits, s);
  if (ta && !tb) return launch_dtl<64, 64, 32, 4, 2, true, false, 2>(a, batch, splits, s);
  return launch_dtl<64, 64, 32, 4, 2, true, true, 2>(a, batch, splits, s);
}

// Adds the K-split partial planes ws[s][M][N] (s < splits) and applies the
// epilogue: C[m*ldc + n] = epi(sum_s ws[s][m][n]).  A thread owns one output
// group (4 floats when VEC: N % 4 == 0, else 1) and keeps 8 plane loads in
// flight.  DEEP (many splits, few outputs): the four wavefronts of a
// workgroup share 64 groups and take planes w, w + 4, ..., then add their
// sums through LDS; otherwise each thread walks every plane of its group.
constexpr int kSumWaves = 4;  // 256 threads

template <bool VEC, bool DEEP>
__global__ __launch_bounds__(256) void splitk_sum_k(const float *__restrict__ ws, int splits,
                                                    int64_t M, int64_t N,
                                                    float *__restrict__ C, int64_t ldc,
                                                    epi_args ep) {
  constexpr int P = VEC ? 4 : 1;
  constexpr int G = 8;
  typedef typename vecf<P>::t V;
  const int64_t plane = M * N;
  const int64_t groups = plane / P;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int64_t gi = DEEP ? int64_t(blockIdx.x) * kWave + lane
                          : int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int ds = DEEP ? kSumWaves : 1;
  float v[P];
#pragma unroll
  for (int q = 0; q < P; ++q) v[q] = 0.0f;
  // The epilogue's bias and residual values are loaded with the planes, not
  // after their sum, so their latency overlaps the plane loads'.
  const int64_t e = gi * P, m = e / N, n = e % N;
  const bool has_bias = ep.epi == SILGPU_EPI_BIAS || ep.epi == SILGPU_EPI_BIAS_SIGMOID ||
                        ep.epi == SILGPU_EPI_BIAS_RELU;
  float bv[P], rv[P];
#pragma unroll
  for (int q = 0; q < P; ++q) {
    const bool mine = gi < groups && (!DEEP || wave == 0);
    bv[q] = mine && has_bias ? ep.bias[(n + q) % ep.bias_len] : 0.0f;
    rv[q] = mine && ep.res ? ep.res[m * ep.ldr + n + q] : 0.0f;
  }
  if (gi < groups) {
    const float *src = ws + gi * P;
    // Groups of G planes, all loads of a group in flight together (the last
    // group predicated, so two or three planes also cost one latency).
    for (int sp = DEEP ? wave : 0; sp < splits; sp += G * ds) {
      V x[G];
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (sp + g * ds < splits)
          x[g] = *reinterpret_cast<const V *>(src + int64_t(sp + g * ds) * plane);
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (sp + g * ds < splits)
#pragma unroll
          for (int q = 0; q < P; ++q) v[q] += vecf<P>::get(x[g], q);
    }
  }
  if constexpr (DEEP) {
    __shared__ float red[kSumWaves - 1][P][kWave];
    if (wave > 0)
#pragma unroll
      for (int q = 0; q < P; ++q) red[wave - 1][q][lane] = v[q];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < kSumWaves - 1; ++w)
#pragma unroll
      for (int q = 0; q < P; ++q) v[q] += red[w][q][lane];
  }
  if (gi >= groups) return;
#pragma unroll
  for (int q = 0; q < P; ++q) v[q] = apply_epi_vals(v[q], bv[q], rv[q], ep);
  float *dst = C + m * ldc + n;
  if constexpr (VEC)
    *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
  else
    dst[0] = v[0];
}

// Tile configurations (BM x BN, waves WM x WN; BK = 16, 32 for 32x128).
enum tile_cfg {
  TILE_AUTO = 0,
  TILE_128x128 = 1,
  TILE_64x64 = 2,
  TILE_32x128 = 3,
  TILE_128x64 = 4,
  TILE_256x256 = 5,
  // M <= 32 (batch 1, A not transposed): sgemm_skinny_k with 32Q columns per
  // workgroup; the automatic choice is TILE_SKINNY (Q = 1) or, for wide and
  // deep products, TILE_SKINNY_Q2.
  TILE_SKINNY = 6,
  TILE_SKINNY_Q2 = 7,
  TILE_SKINNY_Q4 = 8,
  // 64 x 64 tiles with the K range halved between two wave groups of each
  // workgroup (launch_k2), or quartered between four (launch_k4).
  TILE_64x64_K2 = 9,
  TILE_64x64_K4 = 10
};

struct plan {
  int tile;
  int splits;
  // Batch 1: the last tail_rows rows of C run as a second product with
  // tail_splits K splits (the main product then fills whole rounds of CUs).
  int tail_rows = 0;
  int tail_splits = 1;
};

// Shape heuristic (choose_plan): a cost model of each candidate tile and K
// split -- workgroup rounds per CU, the tile's sustained MFMA efficiency,
// occupancy, a K-loop ramp, a per-K-step latency floor and the split-K
// partial pass -- calibrated on MI355X tile x split sweeps (squares up to
// 4096^3, linear_sigmoid 256x4096x4096, transformer projections, small and
// ragged products).  M <= 32 with batch 1 goes to the small-M kernel.
// The 32x128 tile for M <= 32, K split for about 256 workgroups.
plan small_m_tiles(int64_t M, int64_t N, int64_t K, int64_t batch) {
  plan p{TILE_32x128, 1};
  if (batch == 1) {
    int64_t sp = cdiv(256, cdiv(M, 32) * cdiv(N, 128));
    if (sp > K / 256) sp = K / 256;
    if (sp > 64) sp = 64;
    if (sp > 1) p.splits = static_cast<int>(sp);
  }
  return p;
}

int skinny_splits(int64_t M, int64_t N, int64_t K, int Q);

plan choose_plan(int64_t M, int64_t N, int64_t K, int64_t batch, bool dtl_ok) {
  auto tiles = [&](int bm, int bn) { return cdiv(M, bm) * cdiv(N, bn) * batch; };
  // M <= 32: the small-M kernel (splits chosen at launch), or where it does
  // not apply (batched, A transposed) the 32x128 tile.  Where 32-column
  // groups would each walk 2048 or more rows of B in 128-byte pieces (wide N
  // and deep K), 64-column groups with twice the K splits read 256-byte
  // pieces: 19.8 -> 17.9 us at 8 x 4096 x 4096 on MI355X; at N 768..3072
  // the 32-column groups measured ahead, so the wider groups need N > 3072.
  if (M <= 32 && batch == 1)
    return plan{N > 3072 && K / skinny_splits(M, N, K, 1) >= 2048 ? TILE_SKINNY_Q2 : TILE_SKINNY,
                0};
  if (M <= 32) return small_m_tiles(M, N, K, batch);
  // Batched products with a short K loop (attention's Q K^T at head dim 64)
  // are bound by storing C, which the many small tiles overlap with other
  // tiles' K loops: 64x64 measured 25% faster than 128x128 at
  // 48 x 512x512x64 on MI355X.
  if (batch > 1 && K <= 128 && M >= 64 && N >= 64) return plan{TILE_64x64, 1};
  // Predicted time of each (tile, K split): every CU runs ceil(WG / 256)
  // workgroups, min(that, occupancy) of them at once; a SIMD holding a
  // single wavefront reaches kSingleWave of the rate it reaches with two or
  // more.  eff is the fraction of fp32 MFMA peak each tile reaches at large
  // K -- for the LDS-direct kernel where the operands allow it, else for the
  // register-staged one -- and the K loop reaches half its rate at klen =
  // kK0.  A workgroup also takes at least lat per 16-deep K step (one global
  // -> LDS round trip that nothing else hides when a CU holds few
  // workgroups: the floor of small products).  Split-K adds the partial-sum
  // pass: a launch, (splits + 1) M x N fp32 passes and a per-plane latency.
  // A 128x64 launch of at most one workgroup per CU runs 8 waves (two per
  // SIMD, launch_tb), at kEff8 of the 4-wave tile's rate.  Fitted on MI355X
  // to full tile x split sweeps (splits 1, 2, 3, 4, 6, 8, 16) of 46 shapes
  // from 64 x 768 x 2048 to 2048 x 2304 x 768, aligned and ragged, with the
  // picks of the large squares (2048^3 .. 8192^3) held: the plan costs 1.5%
  // more than the best fixed plan (geometric mean; before the 3- and 6-way
  // splits and the 8-wave tile were modelled, 2.1%).  Against the previous
  // plans, 51 shapes: 0.57% faster in the geometric mean, 2048x768x768
  // 30.0 -> 28.3 us, 768^3 20.0 -> 17.6, 512x1024x4096 41.2 -> 39.6, and
  // one shape slower, 100x5000x5000 70.3 -> 74.7.
  struct cand {
    int tile, bm, bn, bk, waves, occupancy;
    double eff, lat;
  };
  // The 128x64 tile runs the LDS-direct kernel when the operands allow it
  // (fitted 0.82 of peak at three workgroups per CU on the 2048-row
  // transformer and square shapes), the register-staged one otherwise.
  const bool dtl128 = dtl_ok && M % 128 == 0 && N % 128 == 0;
  const bool dtl64 = dtl_ok && M % 128 == 0 && N % 64 == 0;
  const cand cands[] = {{TILE_256x256, 256, 256, 16, 8, 1, 0.87, 1.15e-6},
                        {TILE_128x128, 128, 128, 16, 4, 3, dtl128 ? 0.81 : 0.70, 1.25e-6},
                        {TILE_128x64, 128, 64, 16, 4, dtl64 ? 3 : 5, dtl64 ? 0.86 : 0.71, 0.57e-6},
                        {TILE_64x64, 64, 64, 16, 4, 8, 0.64, 0.442e-6}};
  constexpr double kK0 = 48.0, kSingleWave = 0.8755, kLaunch = 4.0e-6, kEff8 = 0.909;
  const double rate_cu = 157.3e12 / 256.0;
  auto round_time = [&](const cand &cd, int64_t nwg, double klen) {
    const int64_t per_cu = cdiv(nwg, 256);
    const int64_t conc = per_cu < cd.occupancy ? per_cu : cd.occupancy;
    const bool w8 = cd.tile == TILE_128x64 && dtl64 && K % 32 == 0 && nwg <= 256;
    const double per_simd = double(conc) * (w8 ? 8 : cd.waves) / 4.0;
    const double f = per_simd >= 2.0 ? 1.0 : per_simd >= 1.0 ? kSingleWave
                                                              : kSingleWave * per_simd;
    const double t = double(per_cu) * 2.0 * cd.bm * cd.bn * klen /
                     (rate_cu * cd.eff * (w8 ? kEff8 : 1.0) * f * (klen / (klen + kK0)));
    const double floor_t = double(cdiv(per_cu, conc)) * (klen / 16.0) * cd.lat;
    return t > floor_t ? t : floor_t;
  };
  auto sum_time = [](int sp, int64_t rows, int64_t cols) {
    return 0.8e-6 + double(sp + 1) * double(rows) * double(cols) * 4.0 / 5.0e12 + 0.05e-6 * sp;
  };
  plan best{TILE_128x128, 1};
  double best_t = 1e30;
  for (const cand &cd : cands) {
    for (int sp : {1, 2, 3, 4, 6, 8, 16}) {
      if (sp > 1 && (batch != 1 || K / sp < 64)) continue;
      // 3- and 6-way splits only for the two smaller tiles: for the larger
      // ones they won nowhere in the sweeps and moved 3000^3 to a plan 7%
      // slower.
      if ((sp == 3 || sp == 6) && (cd.tile == TILE_256x256 || cd.tile == TILE_128x128)) continue;
      const int64_t wg = tiles(cd.bm, cd.bn) * sp;
      const double klen = double(cdiv(cdiv(K, sp), cd.bk) * cd.bk);
      double t = round_time(cd, wg, klen);
      if (sp > 1) t += sum_time(sp, M, N);
      if (t < best_t * 0.999) {
        best_t = t;
        best = plan{cd.tile, sp};
      }
    }
  }
  // Peeling a thin last round: when the tiles of an unsplit product fill
  // whole rounds of the 256 CUs plus part of another, the tile rows past
  // the last whole round can run as a second product split along K, so
  // the first launch has no partly filled round.  Same per-round model,
  // plus one launch for the second product.
  if (batch == 1) {
    for (const cand &cd : cands) {
      const int64_t tm = cdiv(M, cd.bm), tn = cdiv(N, cd.bn), wg = tm * tn;
      if (wg <= 256 || wg % 256 == 0) continue;
      const int64_t rows_main = (wg / 256) * 256 / tn;
      if (rows_main < 1 || rows_main >= tm) continue;
      const double t_main = round_time(cd, rows_main * tn, double(cdiv(K, cd.bk) * cd.bk));
      const int64_t mt = M - rows_main * cd.bm;
      for (int sp : {1, 2, 3, 4, 6, 8}) {
        if (sp > 1 && K / sp < 128) continue;
        const double klen = double(cdiv(cdiv(K, sp), cd.bk) * cd.bk);
        double t = t_main + round_time(cd, cdiv(mt, cd.bm) * tn * sp, klen) + kLaunch;
        if (sp > 1) t += sum_time(sp, mt, N);
        if (t < best_t * 0.97) {
          best_t = t;
          best = plan{cd.tile, 1, static_cast<int>(mt), sp};
        }
      }
    }
  }
  // Where the pick adds K splits in a second launch and 64 x 64 tiles times
  // at most 8 K splits fill 7/8 or more of the CUs in one round, the 64 x 64
  // tile with the K range halved inside each workgroup (TILE_64x64_K2)
  // needs fewer splits, or none, for the same fill.  A rule rather than a
  // candidate of the model: the model's times of the split plans miss by
  // -5..+5 us on these shapes, while this tile's time is a steady ~4 us
  // launch and ramp plus its MFMA time.  MI355X, us, previous pick ->
  // TILE_64x64_K2: 1024^3 24.1 -> 20.7 (2 splits -> none), 256x4096x4096
  // 70.1 -> 67.2, 512x1024x1024 18.3 -> 16.0, 256x2048x512 14.3 -> 12.2,
  // 256x1024x4096 23.9 -> 22.7, 128x2048x768 12.6 -> 11.0, 512^3 10.8 ->
  // 10.0; with 192 tiles (1024x768x2048) it lost, 34.2 -> 36.0.
  if (batch == 1 && dtl_ok && best.splits > 1 && best.tail_rows == 0 && M % 64 == 0 &&
      N % 64 == 0 && K % 64 == 0) {
    const int64_t t64 = (M / 64) * (N / 64);
    int64_t sp = t64 > 0 ? 256 / t64 : 0;
    if (sp > 8) sp = 8;
    while (sp > 1 && K / sp < 128) --sp;
    // Unsplit with K >= 3072: four wave groups (four waves per SIMD) of at
    // least 768 each beat two (256x4096x4096 67.4 -> 65.2 us, 1024x1024x3072
    // 51.7 -> 50.8); with shorter groups the two-group tile wins (1024^3
    // 20.9 against 21.5).
    if (sp == 1 && t64 >= 224 && K >= 3072 && K % 128 == 0) return plan{TILE_64x64_K4, 1};
    if (sp >= 1 && t64 * sp >= 224) return plan{TILE_64x64_K2, static_cast<int>(sp)};
  }
  // Batched products never split K across workgroups; where their 64 x 64
  // tiles fill at most one round of the CUs, the K groups are the only K
  // parallelism there is.  MI355X, us, previous pick -> K groups: 8 x
  // 256x256x4096 120.8 -> 65.7 (four groups), 4 x 512x512x2048 63.3 -> 36.5,
  // 16 x 128x128x1024 33.0 -> 20.4, 48 x 64x64x512 18.5 -> 12.4, 64 x
  // 64x64x256 11.2 -> 8.9; with 512 tiles (8 x 512x512x512) two groups lost,
  // 21.4 -> 23.0.
  if (batch > 1 && dtl_ok && M % 64 == 0 && N % 64 == 0 && K % 64 == 0 &&
      (M / 64) * (N / 64) * batch <= 256)
    return plan{K >= 3072 && K % 128 == 0 ? TILE_64x64_K4 : TILE_64x64_K2, 1};
  // A batched pick of unsplit 128 x 64 tiles that leaves its last round at
  // most half full (batched products cannot peel it into a split second
  // launch) runs faster as twice as many 64 x 64 tiles on two K groups:
  // MI355X, us, 288 to 640 tiles of 128 x 64: 3 x 1024^3 66.8 -> 55.6,
  // 12 x 512x512x1024 67.3 -> 56.9, 5 x 512x1024x2048 126.6 -> 101.1,
  // 9 x 512x512x2048 126.5 -> 101.2, 10 x 512x1024x1024 96.0 -> 90.1 (11 of
  // 11 shapes); with a fuller last round (448 tiles) 67.1 against 72.2, and
  // with whole rounds or one partial one it lost 2-8%.
  if (batch > 1 && dtl_ok && best.tile == TILE_128x64 && best.splits == 1 && M % 128 == 0 &&
      N % 64 == 0 && K % 64 == 0) {
    const int64_t t = (M / 128) * (N / 64) * batch;
    if (t > 256 && t < 768 && t % 256 != 0 && t % 256 <= 128) return plan{TILE_64x64_K2, 1};
  }
  return best;
}

template <int Q, bool TB, bool VA, bool VB>
void launch_skinny_k(const gemm_args &g, dim3 grid, hipStream_t s) {
  sgemm_skinny_k<Q, TB, VA, VB><<<grid, kSkWaves * kWave, 0, s>>>(g);
}

template <int Q, bool TB>
int launch_skinny_q(const gemm_args &a, int splits, bool va, bool vb, hipStream_t s) {
  gemm_args g = a;
  constexpr int64_t kStep = int64_t(kSkChunk) * kSkWaves;
  g.klen = static_cast<int>(cdiv(cdiv(a.K, splits), kStep) * kStep);
  if (g.klen < kStep) g.klen = static_cast<int>(kStep);
  splits = static_cast<int>(a.K > 0 ? cdiv(a.K, g.klen) : 1);
  dim3 grid(static_cast<unsigned>(cdiv(a.N, 32 * Q)), static_cast<unsigned>(splits));
  if (!TB || !vb) {
    if (va) launch_skinny_k<Q, TB, true, false>(g, grid, s);
    else launch_skinny_k<Q, TB, false, false>(g, grid, s);
  } else {
    if (va) launch_skinny_k<Q, TB, true, true>(g, grid, s);
    else launch_skinny_k<Q, TB, false, true>(g, grid, s);
  }
  SILGPU_LAUNCH_CHECK("sgemm_skinny_k");
  return splits;
}

// K splits for the small-M kernel: about one workgroup per CU (measured best
// on MI355X for M <= 32 at N, K in 768..4096), each K range at least 128
// deep.
int skinny_splits(int64_t M, int64_t N, int64_t K, int Q) {
  (void)M;
  int64_t sp = 256 / cdiv(N, 32 * Q);
  if (sp > K / 128) sp = K / 128;
  if (sp > 65535) sp = 65535;
  return sp < 1 ? 1 : static_cast<int>(sp);
}

// Column-group width of the small-M kernel for `tile`: Q > 1 needs N % Q == 0
// and, without trans_b, 16-byte-aligned B rows.
int skinny_q(const gemm_args &a, int tile, bool tb) {
  int Q = tile == TILE_SKINNY_Q2 ? 2 : tile == TILE_SKINNY_Q4 ? 4 : 1;
  while (Q > 1 && (a.N % Q != 0 || (!tb && !(a.ldb % Q == 0 && aligned16(a.B))))) Q /= 2;
  return Q;
}

// Launches the small-M kernel with column-group width Q; returns the number
// of K splits launched.
int launch_skinny(const gemm_args &a, int Q, int splits, bool tb, hipStream_t s) {
  const bool va = a.lda % 4 == 0 && aligned16(a.A);
  const bool bvec = a.ldb % 4 == 0 && aligned16(a.B);
  if (Q == 4)
    return tb ? launch_skinny_q<4, true>(a, splits, va, bvec, s)
              : launch_skinny_q<4, false>(a, splits, va, bvec, s);
  if (Q == 2)
    return tb ? launch_skinny_q<2, true>(a, splits, va, bvec, s)
              : launch_skinny_q<2, false>(a, splits, va, bvec, s);
  return tb ? launch_skinny_q<1, true>(a, splits, va, bvec, s)
            : launch_skinny_q<1, false>(a, splits, va, bvec, s);
}

int launch_split_sum(const gemm_args &a, int launched, context *c);

// Where a product's scratch comes from.  silgpu_gemm: the split-K workspace
// (grown with hipMalloc on demand) and the partials area reserved at init.
// silgpu_gemm_noalloc: one fixed device array for both, never allocated
// per call; a K split whose partial planes would not fit it is narrowed to
// the widest that fits (down to none).
struct scratch_src {
  float *fixed = nullptr;
  size_t fixed_bytes = 0;
};

// The products the last GEMM entry-point call on this thread launched, for
// silgpu_gemm_last_plan: up to two (the main product and a peeled last
// round of rows), each with its tile configuration, K splits and rows of C.
struct launch_record {
  int n = 0;
  int tile[2] = {0, 0};
  int splits[2] = {0, 0};
  int rows[2] = {0, 0};
};
thread_local launch_record g_last_launch;

int run_sgemm(const gemm_args &a0, int64_t batch, plan pl, bool ta, bool tb, bool vec,
              context *c, const scratch_src &ss) {
  if (pl.tail_rows > 0 && pl.tail_rows < a0.M && batch == 1) {
    // Rows [0, M - tail) as one product, the last tail rows as another.
    const int head = a0.M - pl.tail_rows;
    gemm_args h = a0, t = a0;
    h.M = head;
    t.M = pl.tail_rows;
    t.A = a0.A + (ta ? int64_t(head) : int64_t(head) * a0.lda);
    t.C = a0.C + int64_t(head) * a0.ldc;
    if (t.ep.res) t.ep.res += int64_t(head) * t.ep.ldr;
    const bool tvec = vec && aligned16(t.A);
    int rc = run_sgemm(h, 1, plan{pl.tile, 1}, ta, tb, vec, c, ss);
    if (rc != SILGPU_OK) return rc;
    return run_sgemm(t, 1, plan{pl.tile, pl.tail_splits}, ta, tb, tvec, c, ss);
  }
  gemm_args a = a0;
  // The small-M kernel's per-lane byte offsets are 32-bit.
  const int64_t kLane = int64_t(1) << 30;
  const bool lane32 = int64_t(a.M) * a.lda + 8 < kLane &&
                      (tb ? (int64_t(a.N) + 4) * a.ldb + 8 : 8 * a.ldb + a.N) < kLane;
  const bool skinny_tile = pl.tile >= TILE_SKINNY && pl.tile <= TILE_SKINNY_Q4;
  const bool skinny = skinny_tile && a.M <= 32 && batch == 1 && !ta && lane32;
  if (skinny_tile && !skinny)
    pl = pl.splits >= 1 ? plan{TILE_32x128, pl.splits} : small_m_tiles(a.M, a.N, a.K, batch);
  int splits = pl.splits;
  int q = 1;
  if (skinny) {
    q = skinny_q(a, pl.tile, tb);
    if (splits < 1) splits = skinny_splits(a.M, a.N, a.K, q);
  }
  if (splits < 1) splits = 1;
  if (batch != 1 || a.K == 0) splits = 1;
  if (splits > 1) {
    const size_t plane = size_t(a.M) * size_t(a.N) * sizeof(float);
    if (ss.fixed) {
      const size_t fit = ss.fixed_bytes / plane;
      if (size_t(splits) > fit) splits = fit >= 2 ? static_cast<int>(fit) : 1;
      a.ws = ss.fixed;
    } else {
      int rc = ensure_workspace(c, size_t(splits) * plane);
      if (rc != SILGPU_OK) return rc;
      a.ws = static_cast<float *>(c->workspace);
    }
  }
  int launched;
  bool k2 = false;
  if (skinny) {
    launched = launch_skinny(a, q, splits, tb, c->stream);
  } else {
    switch (pl.tile) {
      case TILE_64x64_K2:
        launched = launch_k2(a, batch, splits, ta, tb, vec, c->stream, k2);
        break;
      case TILE_64x64_K4:
        launched = launch_k4(a, batch, splits, ta, tb, vec, c->stream, k2);
        break;
      case TILE_64x64:
        launched = launch_tiles<64, 64, 16, 2, 2, 16>(a, batch, splits, ta, tb, vec, c->stream);
        break;
      case TILE_32x128:
        launched = launch_tiles<32, 128, 32, 1, 4, 16>(a, batch, splits, ta, tb, vec, c->stream);
        break;
      case TILE_128x64:
        launched = launch_tiles<128, 64, 16, 2, 2, 16>(a, batch, splits, ta, tb, vec, c->stream);
        break;
      case TILE_256x256:
        launched = launch_tiles<256, 256, 16, 2, 4, 16>(a, batch, splits, ta, tb, vec, c->stream);
        break;
      default:
        launched = launch_tiles<128, 128, 16, 2, 2, 16>(a, batch, splits, ta, tb, vec, c->stream);
        break;
    }
  }
  if (launched < 0) return launched;
  launch_record &rec = g_last_launch;
  if (rec.n < 2) {
    const bool known = pl.tile == TILE_64x64 || pl.tile == TILE_32x128 ||
                       pl.tile == TILE_128x64 || pl.tile == TILE_256x256;
    rec.tile[rec.n] = skinny ? (q == 4 ? TILE_SKINNY_Q4 : q == 2 ? TILE_SKINNY_Q2 : TILE_SKINNY)
                      : pl.tile == TILE_64x64_K2 ? (k2 ? TILE_64x64_K2 : TILE_64x64)
                      : pl.tile == TILE_64x64_K4 ? (k2 ? TILE_64x64_K4 : TILE_64x64)
                      : known ? pl.tile : TILE_128x128;
    rec.splits[rec.n] = launched;
    rec.rows[rec.n] = a.M;
    ++rec.n;
  }
  return launched > 1 ? launch_split_sum(a, launched, c) : SILGPU_OK;
}

// Adds the `splits` partial planes a.ws[s][M][N] into C with the epilogue.
int launch_split_sum(const gemm_args &a, int launched, context *c) {
  {
    const bool v4 = a.N % 4 == 0 && a.ldc % 4 == 0 && aligned16(a.C);
    const int64_t groups = a.M * int64_t(a.N) / (v4 ? 4 : 1);
    const bool deep = launched >= 8 && groups < 65536;
    const unsigned g = static_cast<unsigned>(cdiv(groups, deep ? kWave : 256));
    if (v4 && deep)
      splitk_sum_k<true, true><<<g, 256, 0, c->stream>>>(a.ws, launched, a.M, a.N, a.C, a.ldc,
                                                         a.ep);
    else if (v4)
      splitk_sum_k<true, false><<<g, 256, 0, c->stream>>>(a.ws, launched, a.M, a.N, a.C,
                                                          a.ldc, a.ep);
    else if (deep)
      splitk_sum_k<false, true><<<g, 256, 0, c->stream>>>(a.ws, launched, a.M, a.N, a.C,
                                                          a.ldc, a.ep);
    else
      splitk_sum_k<false, false><<<g, 256, 0, c->stream>>>(a.ws, launched, a.M, a.N, a.C,
                                                           a.ldc, a.ep);
    SILGPU_LAUNCH_CHECK("splitk_sum_k");
  }
  return SILGPU_OK;
}

// Implicit-GEMM convolution on the LDS-direct kernel: full 128 x 64 tiles
// (M % 128 == 0, C_out % 64 == 0) and C_in % 16 == 0, so every K tile of
// BK = 32 (C_in % 32 == 0) or 16 lies in one tap.
// splits > 1 (dividing K / BK): partial planes to a.ws, added by
// launch_split_sum.
template <int BK>
int launch_conv_dtl(const gemm_args &a, int splits, hipStream_t s) {
  using D = dtl_cfg<128, 64, BK, 4, 2>;
  auto kern = sgemm_dtl_k<128, 64, BK, 4, 2, false, true, true>;
  gemm_args g = a;
  g.tiles_m = a.M / 128;
  g.tiles_n = a.N / 64;
  g.klen = a.K / splits;
  SILGPU_REQUIRE(splits == 1 || int64_t(128) * a.N * 4 < (int64_t(1) << 30),
                 "conv2d: %lld output channels are too many for a K split",
                 static_cast<long long>(a.N));
  dim3 grid(static_cast<unsigned>(int64_t(g.tiles_m) * g.tiles_n), static_cast<unsigned>(splits),
            1u);
  kern<<<grid, D::kThreads, 0, s>>>(g);
  SILGPU_LAUNCH_CHECK("sgemm_dtl_k (conv2d)");
  return SILGPU_OK;
}

// Implicit-GEMM convolution on the register-staged MFMA kernel (CONV): the A
// tile is gathered from the NHWC input, B is the OHWI weight read as a
// [C_out][K*K*C_in] matrix (transposed B), C is the NHWC output.
template <int BM, int BN, int WM, int WN, bool VEC>
int launch_conv_cfg(const gemm_args &a, hipStream_t s) {
  using C = cfg<BM, BN, 16, WM, WN, 16>;
  auto kern = sgemm_mfma_k<BM, BN, 16, WM, WN, 16, false, true, VEC, true, true>;
  // Once per process (a thread-safe static), before the first launch.
  static const hipError_t attr_rc =
      hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, C::kLdsBytes);
  SILGPU_HIP_CHECK(attr_rc);
  gemm_args g = a;
  g.tiles_m = static_cast<int>(cdiv(a.M, BM));
  g.tiles_n = static_cast<int>(cdiv(a.N, BN));
  g.klen = static_cast<int>(cdiv(a.K, 16) * 16);
  if (g.klen < 16) g.klen = 16;
  dim3 grid(static_cast<unsigned>(int64_t(g.tiles_m) * g.tiles_n), 1u, 1u);
  kern<<<grid, C::kThreads, C::kLdsBytes, s>>>(g);
  SILGPU_LAUNCH_CHECK("sgemm_mfma_k (conv2d)");
  return SILGPU_OK;
}

int launch_gemv_n(const float *x, const float *Bm, int64_t ldb, float *y, int64_t N,
                  int64_t K, context *c, const scratch_src &ss) {
  float *partial = ss.fixed ? ss.fixed : static_cast<float *>(c->partials);
  const int64_t partial_bytes = ss.fixed ? int64_t(ss.fixed_bytes) : int64_t(kPartialBytes);
  // Wider than one partial row of the scratch area holds: column pieces of
  // whole 256-column tiles, each its own pass 1 and finish.
  const int64_t max_cols = partial_bytes / int64_t(sizeof(float)) / kGemvCols * kGemvCols;
  if (N > max_cols) {
    for (int64_t c0 = 0; c0 < N; c0 += max_cols) {
      const int rc = launch_gemv_n(x, Bm + c0, ldb, y + c0, N - c0 < max_cols ? N - c0 : max_cols,
                                   K, c, ss);
      if (rc != SILGPU_OK) return rc;
    }
    return SILGPU_OK;
  }
  const bool vec = N % 4 == 0 && ldb % 4 == 0 && aligned16(Bm);
  const int64_t ct = cdiv(N, kGemvCols);
  const int64_t pitch = ct * kGemvCols;
  // K splits: ~1024 workgroups, >= 32 rows per split, partials fit scratch.
  int64_t ks = 1024 / ct;
  if (ks > K / 32) ks = K / 32;
  if (ks < 1) ks = 1;
  if (ks > 65535) ks = 65535;
  while (ks > 1 && ks * pitch * int64_t(sizeof(float)) > partial_bytes) ks /= 2;
  SILGPU_REQUIRE(pitch * int64_t(sizeof(float)) <= partial_bytes,
                 "silgpu_sgemv: N %lld exceeds the %lld-byte scratch area", (long long)N,
                 (long long)partial_bytes);
  const int64_t kc = cdiv(K, ks);
  ks = cdiv(K, kc);
  dim3 grid(static_cast<unsigned>(ct), static_cast<unsigned>(ks));
  if (vec)
    gemv_part_k<true><<<grid, kGemvPartBlock, 0, c->stream>>>(x, Bm, ldb, N, K, kc, partial);
  else
    gemv_part_k<false><<<grid, kGemvPartBlock, 0, c->stream>>>(x, Bm, ldb, N, K, kc, partial);
  SILGPU_LAUNCH_CHECK("gemv_part_k");
  if (vec && ks == int64_t(kGemvFinishLoads) * kGemvWaves) {
    gemv_finish_vec_k<true><<<static_cast<unsigned>(ct), kGemvBlock, 0, c->stream>>>(
        partial, ks, pitch, N, y);
  } else if (vec) {
    gemv_finish_vec_k<false><<<static_cast<unsigned>(ct), kGemvBlock, 0, c->stream>>>(
        partial, ks, pitch, N, y);
  } else {
    const unsigned fgrid = static_cast<unsigned>(cdiv(pitch, kWave));
    gemv_finish_k<false><<<fgrid, kGemvBlock, 0, c->stream>>>(partial, ks, pitch, N, y);
  }
  SILGPU_LAUNCH_CHECK("gemv_finish_k");
  return SILGPU_OK;
}

int launch_gemv_t(const float *x, int64_t incx, const float *R, int64_t ldr, float *y,
                  int64_t incy, int64_t nrows, int64_t K, context *c) {
  const bool vec = K % 4 == 0 && ldr % 4 == 0 && aligned16(R) && aligned16(x);
  unsigned grid = static_cast<unsigned>(cdiv(nrows, 4));
  if (vec)
    gemv_t_k<true><<<grid, 256, 0, c->stream>>>(x, incx, R, ldr, y, incy, nrows, K);
  else
    gemv_t_k<false><<<grid, 256, 0, c->stream>>>(x, incx, R, ldr, y, incy, nrows, K);
  SILGPU_LAUNCH_CHECK("gemv_t_k");
  return SILGPU_OK;
}

int apply_epilogue(float *C, int64_t ldc, int64_t M, int64_t N, const epi_args &ep,
                   context *c) {
  if (ep.epi == SILGPU_EPI_NONE && !ep.use_scale && !ep.res) return SILGPU_OK;
  int64_t g = cdiv(M * N, 256);
  if (g > 4096) g = 4096;
  epilogue_k<<<static_cast<unsigned>(g), 256, 0, c->stream>>>(C, ldc, M, N, ep);
  SILGPU_LAUNCH_CHECK("epilogue_k");
  return SILGPU_OK;
}


}  // namespace
}  // namespace silgpu

using namespace silgpu;

extern "C" {

int silgpu_sgemv(const float *d_x, const float *d_B, int64_t ldb, float *d_y, int64_t N,
                 int64_t K) {
  SILGPU_REQUIRE(N >= 0 && K >= 0, "silgpu_sgemv: negative extent");
  if (N == 0) return SILGPU_OK;
  SILGPU_REQUIRE(ldb >= N, "silgpu_sgemv: ldb %lld < N %lld", (long long)ldb, (long long)N);
  SILGPU_REQUIRE(d_y != nullptr, "silgpu_sgemv: null y");
  SILGPU_CTX(c);
  if (K == 0) return silgpu_fill_u32(d_y, 0u, N);
  SILGPU_REQUIRE(d_x && d_B, "silgpu_sgemv: null pointer");
  return launch_gemv_n(d_x, d_B, ldb, d_y, N, K, c, scratch_src{});
}

}  // extern "C"

namespace {

// Shared body of silgpu_sgemm / silgpu_sgemm_tuned / silgpu_gemm_noalloc.
// `forced` (tuning only) skips the vector-product routing and the shape
// heuristic.  `noalloc`: the library must already be initialised, and all
// scratch comes from the fixed array found at init.
int gemm_impl(const silgpu_gemm_desc &d, const plan *forced, bool noalloc = false) {
  g_last_launch = launch_record{};
  const int64_t M = d.M, N = d.N, K = d.K;
  SILGPU_REQUIRE(M >= 0 && N >= 0 && K >= 0 && d.batch_outer >= 0 && d.batch_inner >= 0,
                 "silgpu_gemm: negative extent");
  SILGPU_REQUIRE(M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
                 "silgpu_gemm: extent exceeds int32");
  SILGPU_REQUIRE(d.epilogue >= SILGPU_EPI_NONE && d.epilogue <= SILGPU_EPI_BIAS_RELU,
                 "silgpu_gemm: unknown epilogue %d", d.epilogue);
  const int64_t batch = d.batch_outer * d.batch_inner;
  if (M == 0 || N == 0 || batch == 0) return SILGPU_OK;
  const bool ta = d.trans_a != 0, tb = d.trans_b != 0;
  SILGPU_REQUIRE(d.lda >= (ta ? M : K) && d.lda >= 1, "silgpu_gemm: lda %lld too small",
                 (long long)d.lda);
  SILGPU_REQUIRE(d.ldb >= (tb ? K : N) && d.ldb >= 1, "silgpu_gemm: ldb %lld too small",
                 (long long)d.ldb);
  SILGPU_REQUIRE(d.ldc >= N, "silgpu_gemm: ldc %lld < N %lld", (long long)d.ldc, (long long)N);
  const bool uses_bias = d.epilogue == SILGPU_EPI_BIAS || d.epilogue == SILGPU_EPI_BIAS_SIGMOID ||
                         d.epilogue == SILGPU_EPI_BIAS_RELU;
  SILGPU_REQUIRE(!uses_bias || (d.bias && d.bias_len > 0),
                 "silgpu_gemm: bias epilogue without bias");
  SILGPU_REQUIRE(!d.residual || (batch == 1 && d.ldr >= N),
                 "silgpu_gemm: a residual needs batch 1 and ldr >= N");
  SILGPU_REQUIRE(d.C != nullptr && (K == 0 || (d.A && d.B)), "silgpu_gemm: null pointer");
  if (batch > kMaxGridBatch) {
    // More products than one launch's grid.z holds: launches of at most
    // kMaxGridBatch products, whole outer indices where the inner batch
    // fits in one, else pieces of each outer index's inner batch.
    silgpu_gemm_desc p = d;
    auto shift = [&](int64_t o, int64_t i) {
      auto at = [](const float *x, int64_t off) { return x ? x + off : x; };
      p.A = at(d.A, o * d.stride_a_outer + i * d.stride_a_inner);
      p.B = at(d.B, o * d.stride_b_outer + i * d.stride_b_inner);
      p.C = d.C + o * d.stride_c_outer + i * d.stride_c_inner;
    };
    if (d.batch_inner <= kMaxGridBatch) {
      const int64_t per = kMaxGridBatch / d.batch_inner;
      for (int64_t o0 = 0; o0 < d.batch_outer; o0 += per) {
        shift(o0, 0);
        p.batch_outer = d.batch_outer - o0 < per ? d.batch_outer - o0 : per;
        const int rc = gemm_impl(p, forced, noalloc);
        if (rc != SILGPU_OK) return rc;
      }
    } else {
      for (int64_t o = 0; o < d.batch_outer; o++)
        for (int64_t i0 = 0; i0 < d.batch_inner; i0 += kMaxGridBatch) {
          shift(o, i0);
          p.batch_outer = 1;
          p.batch_inner =
              d.batch_inner - i0 < kMaxGridBatch ? d.batch_inner - i0 : kMaxGridBatch;
          const int rc = gemm_impl(p, forced, noalloc);
          if (rc != SILGPU_OK) return rc;
        }
    }
    return SILGPU_OK;
  }
  context *c = noalloc ? ctx_if_ready() : ctx();
  if (!c) return noalloc ? SILGPU_ERR_INVALID : SILGPU_ERR_NODEVICE;
  scratch_src ss{};
  if (noalloc) {
    ss.fixed = c->noalloc_scratch;
    ss.fixed_bytes = kNoAllocScratchBytes;
  }

  epi_args ep{};
  ep.bias = d.bias;
  ep.bias_len = d.bias_len > 0 ? d.bias_len : 1;
  ep.res = d.residual;
  ep.ldr = d.ldr;
  ep.scale = d.scale;
  ep.offset = d.scale_offset;
  ep.epi = d.epilogue;
  ep.use_scale = d.use_scale != 0;

  // Vector products (the reference routes M == 1 to sgemv, include/array.h:2675-2676).
  if (!forced && batch == 1 && K > 0 && (M == 1 || N == 1)) {
    int rc;
    if (M == 1 && !tb && !ta) {
      // y = x * B with x = A[0..K) contiguous and B [K][N].
      rc = launch_gemv_n(d.A, d.B, d.ldb, d.C, N, K, c, ss);
      if (rc != SILGPU_OK) return rc;
      return apply_epilogue(d.C, d.ldc, 1, N, ep, c);
    } else if (M == 1 && tb) {
      // y[n] = sum_k x[k] * B[n*ldb + k]
      rc = launch_gemv_t(d.A, ta ? d.lda : 1, d.B, d.ldb, d.C, 1, N, K, c);
      if (rc != SILGPU_OK) return rc;
      return apply_epilogue(d.C, d.ldc, 1, N, ep, c);
    } else if (N == 1 && !ta) {
      // y[m] = sum_k A[m*lda + k] * b[k], b[k] = B[k*ldb] (non-trans) or B[k] (trans)
      rc = launch_gemv_t(d.B, tb ? 1 : d.ldb, d.A, d.lda, d.C, d.ldc, M, K, c);
      if (rc != SILGPU_OK) return rc;
      return apply_epilogue(d.C, d.ldc, M, 1, ep, c);
    }
  }

  gemm_args a{};
  a.A = d.A;
  a.B = d.B;
  a.C = d.C;
  a.lda = d.lda;
  a.ldb = d.ldb;
  a.ldc = d.ldc;
  a.sA = d.stride_a_inner;
  a.sB = d.stride_b_inner;
  a.sC = d.stride_c_inner;
  a.sA2 = d.stride_a_outer;
  a.sB2 = d.stride_b_outer;
  a.sC2 = d.stride_c_outer;
  a.binner = static_cast<int>(d.batch_inner);
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  a.ep = ep;
  const bool vec = aligned16(d.A) && aligned16(d.B) && d.lda % 4 == 0 && d.ldb % 4 == 0 &&
                   (ta ? M % 4 == 0 : K % 4 == 0) && (tb ? K % 4 == 0 : N % 4 == 0) &&
                   (batch == 1 || (d.stride_a_inner % 4 == 0 && d.stride_b_inner % 4 == 0 &&
                                   d.stride_a_outer % 4 == 0 && d.stride_b_outer % 4 == 0));
  const bool dtl_ok = vec && K % 16 == 0 && d.lda < kDtlMaxLd && d.ldb < kDtlMaxLd;
  return run_sgemm(a, batch, forced ? *forced : choose_plan(M, N, K, batch, dtl_ok),
                   ta, tb, vec, c, ss);
}

silgpu_gemm_desc plain_desc(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                            const float *d_A, int64_t lda, int64_t stride_a, const float *d_B,
                            int64_t ldb, int64_t stride_b, float *d_C, int64_t ldc,
                            int64_t stride_c, int64_t batch, const float *d_bias,
                            int64_t bias_len, int epilogue) {
  silgpu_gemm_desc d{};
  d.trans_a = trans_a;
  d.trans_b = trans_b;
  d.M = M;
  d.N = N;
  d.K = K;
  d.A = d_A;
  d.lda = lda;
  d.B = d_B;
  d.ldb = ldb;
  d.C = d_C;
  d.ldc = ldc;
  d.batch_outer = batch > 0 ? 1 : 0;
  d.batch_inner = batch;
  d.stride_a_inner = stride_a;
  d.stride_b_inner = stride_b;
  d.stride_c_inner = stride_c;
  d.epilogue = epilogue;
  d.bias = d_bias;
  d.bias_len = bias_len;
  return d;
}

}  // namespace

extern "C" {

int silgpu_sgemm(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, const float *d_A,
                 int64_t lda, int64_t stride_a, const float *d_B, int64_t ldb,
                 int64_t stride_b, float *d_C, int64_t ldc, int64_t stride_c, int64_t batch,
                 const float *d_bias, int64_t bias_len, int epilogue) {
  SILGPU_REQUIRE(batch >= 0, "silgpu_sgemm: negative batch");
  return gemm_impl(plain_desc(trans_a, trans_b, M, N, K, d_A, lda, stride_a, d_B, ldb, stride_b,
                              d_C, ldc, stride_c, batch, d_bias, bias_len, epilogue),
                   nullptr);
}

int silgpu_sgemm_tuned(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                       const float *d_A, int64_t lda, int64_t stride_a, const float *d_B,
                       int64_t ldb, int64_t stride_b, float *d_C, int64_t ldc, int64_t stride_c,
                       int64_t batch, const float *d_bias, int64_t bias_len, int epilogue,
                       int tile, int splits) {
  SILGPU_REQUIRE(tile >= TILE_128x128 && tile <= TILE_64x64_K4,
                 "silgpu_sgemm_tuned: unknown tile configuration %d", tile);
  SILGPU_REQUIRE(splits >= 1 && splits <= 256, "silgpu_sgemm_tuned: splits %d not in [1, 256]",
                 splits);
  SILGPU_REQUIRE(batch >= 0, "silgpu_sgemm_tuned: negative batch");
  plan pl{tile, splits};
  return gemm_impl(plain_desc(trans_a, trans_b, M, N, K, d_A, lda, stride_a, d_B, ldb, stride_b,
                              d_C, ldc, stride_c, batch, d_bias, bias_len, epilogue),
                   &pl);
}

int silgpu_gemm(const silgpu_gemm_desc *desc) {
  SILGPU_REQUIRE(desc != nullptr, "silgpu_gemm: null descriptor");
  return gemm_impl(*desc, nullptr);
}

int silgpu_gemm_noalloc(const silgpu_gemm_desc *desc) {
  SILGPU_REQUIRE(desc != nullptr, "silgpu_gemm_noalloc: null descriptor");
  return gemm_impl(*desc, nullptr, true);
}

int silgpu_gemm_last_plan(int *n, int *tiles, int *splits, int *rows) {
  SILGPU_REQUIRE(n && tiles && splits && rows, "silgpu_gemm_last_plan: null argument");
  const launch_record &rec = g_last_launch;
  *n = rec.n;
  for (int i = 0; i < rec.n; ++i) {
    tiles[i] = rec.tile[i];
    splits[i] = rec.splits[i];
    rows[i] = rec.rows[i];
  }
  return SILGPU_OK;
}

int silgpu_conv2d_f32(const float *d_in, const float *d_w, float *d_out, int64_t N, int64_t H,
                      int64_t W, int64_t C_in, int64_t K, int64_t C_out) {
  SILGPU_REQUIRE(N >= 0 && H >= 0 && W >= 0 && C_in >= 0 && C_out >= 0 && K >= 1,
                 "silgpu_conv2d_f32: negative extent or kernel size < 1");
  int64_t M = 0, Kd = 0;
  SILGPU_REQUIRE(!__builtin_mul_overflow(N, H, &M) && !__builtin_mul_overflow(M, W, &M) &&
                     !__builtin_mul_overflow(K, K, &Kd) &&
                     !__builtin_mul_overflow(Kd, C_in, &Kd),
                 "silgpu_conv2d_f32: extent product overflows int64");
  if (M == 0 || C_out == 0) return SILGPU_OK;
  SILGPU_REQUIRE(M <= INT32_MAX && Kd <= INT32_MAX && C_out <= INT32_MAX &&
                     M * C_in <= INT64_MAX / 4 && K * W * C_in <= INT32_MAX,
                 "silgpu_conv2d_f32: extent exceeds int32");
  SILGPU_REQUIRE(d_out != nullptr, "silgpu_conv2d_f32: null output");
  SILGPU_CTX(c);
  if (Kd == 0) return silgpu_fill_u32(d_out, 0u, M * C_out);
  SILGPU_REQUIRE(d_in && d_w, "silgpu_conv2d_f32: null pointer");
  gemm_args a{};
  a.A = d_in;
  a.B = d_w;
  a.C = d_out;
  a.ldb = Kd;
  a.ldc = C_out;
  a.binner = 1;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(C_out);
  a.K = static_cast<int>(Kd);
  a.ep.bias_len = 1;
  a.ep.epi = SILGPU_EPI_NONE;
  a.cv_h = static_cast<int>(H);
  a.cv_w = static_cast<int>(W);
  a.cv_cin = static_cast<int>(C_in);
  a.cv_k = static_cast<int>(K);
  a.cv_pad = static_cast<int>(K / 2);
  if (Kd <= kConvDirectMaxK && C_out <= kConvDirectMaxCo)
    return conv2d_direct(d_in, d_w, d_out, static_cast<int>(M), static_cast<int>(H),
                         static_cast<int>(W), static_cast<int>(C_in), static_cast<int>(K),
                         static_cast<int>(C_out), c->stream);
  const bool vec = C_in % 4 == 0 && aligned16(d_in) && aligned16(d_w);
  if (vec && C_in % 16 == 0 && M % 128 == 0 && C_out % 64 == 0) {
    // Three 128 x 64 workgroups fit a CU.  Between one and two tiles per CU
    // (two on some CUs, one on others) the K range is split in two, so the
    // pieces fill three rounds.  When the pieces fill whole rounds of all
    // CUs plus a thin last round, the tile rows of that last round run as a
    // second launch split further along K (one piece per CU at most) with
    // its own split sum, instead of a round of a few workgroups at full
    // depth.
    const int BK = C_in % 32 == 0 ? 32 : 16;
    const int64_t tiles_n = C_out / 64, tiles_m = M / 128, tiles = tiles_m * tiles_n;
    const int64_t cus = c->cu_count, slots = cus * 3, kt = Kd / BK;
    // (Measured: 88.5 -> 85.2 us at 16x28x28x128 -> 256, K = 1152; with K
    // = 576 the halves are too short and the split sum costs more than the
    // balance gains, 48.7 -> 56.6 us at 8x56x56x64 -> 128.)
    const int gs = tiles > cus && 2 * tiles > slots && 4 * (2 * tiles) <= 5 * slots &&
                           kt % 2 == 0 && Kd >= 1024
                       ? 2 : 1;
    const int64_t pieces = tiles * gs, rem = pieces % slots;
    int64_t rows_main = tiles_m;
    int splits = 1;
    if (pieces > slots && rem > 0 && rem * 4 <= slots) {
      const int64_t rem_rows = cdiv(rem, tiles_n * gs);
      rows_main = tiles_m - rem_rows;
      for (int64_t sp = 2; sp <= kt; ++sp)
        if (kt % sp == 0 && rem_rows * tiles_n * sp <= cus) splits = int(sp);
    }
    auto conv = [&](gemm_args g, int sp) {
      if (sp > 1) {
        int rc = ensure_workspace(c, size_t(sp) * size_t(g.M) * size_t(C_out) * sizeof(float));
        if (rc != SILGPU_OK) return rc;
        g.ws = static_cast<float *>(c->workspace);
      }
      int rc = BK == 32 ? launch_conv_dtl<32>(g, sp, c->stream)
                        : launch_conv_dtl<16>(g, sp, c->stream);
      if (rc != SILGPU_OK || sp == 1) return rc;
      return launch_split_sum(g, sp, c);
    };
    gemm_args main = a;
    main.M = static_cast<int>(rows_main * 128);
    int rc = conv(main, gs);
    if (rc != SILGPU_OK || rows_main == tiles_m) return rc;
    gemm_args tail = a;
    tail.cv_m0 = main.M;
    tail.M = static_cast<int>(M) - main.M;
    tail.C = d_out + int64_t(main.M) * C_out;
    return conv(tail, splits);
  }
  if (C_out <= 32)
    return vec ? launch_conv_cfg<64, 64, 2, 2, true>(a, c->stream)
               : launch_conv_cfg<64, 64, 2, 2, false>(a, c->stream);
  return vec ? launch_conv_cfg<128, 64, 2, 2, true>(a, c->stream)
             : launch_conv_cfg<128, 64, 2, 2, false>(a, c->stream);
}

}  // extern "C"

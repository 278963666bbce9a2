// Direct 2-D convolution for short reductions (K*K*C_in <= kConvDirectMaxK,
// e.g. the 3-channel first layer of an image network), where a tiled
// implicit GEMM would spend its time filling and draining its tiles.
//
// Layouts as silgpu_conv2d_f32: NHWC input [N][H][W][C_in], OHWI weight
// [C_out][K][K][C_in], NHWC output; stride 1, zero padding K/2 (tap (kh, kw)
// of output pixel (oh, ow) reads input (oh + kh - K/2, ow + kw - K/2), zero
// outside the image).  Each output is the float32 sum over k = (kh*K + kw)*
// C_in + ci, as matrix-core products of four terms at a time.

#include "internal.h"

namespace silgpu {
namespace {

// Matrix-core direct convolution for reductions K*K*C_in <= kConvDirectMaxK:
// no LDS and no barrier.  A wave computes 16 output pixels x 16*NB output
// channels per tile as C^T = W * X^T on v_mfma_f32_16x16x4f32 over k = (kh*K +
// kw)*C_in + ci, four k per instruction in KS steps (4*KS >= K*K*C_in; k past
// the reduction multiplies zeros).  Lane (l16, g) = (lane % 16, lane / 16)
// supplies, at step s, weight w[co0 + 16b + l16][k] with k = 4s + g (held in
// registers for all of the wave's tiles) and the input of pixel px0 + l16 at
// that k (a cached gather, zero in the padding), and ends holding channels
// co0 + 16b + 4g .. + 3 of pixel px0 + l16: one float4 store.  The (kh, kw,
// ci) of a lane's k at each step are decoded once per wave.  Past K*K*C_in
// the shifts are -2^30: H*W < 2^31 leaves H or W below 2^16, so one of the
// shifted coordinates is negative and nothing is read.  Waves walk the
// 16-pixel tiles grid-stride with the next tile's gathers issued before the
// current tile's products.
typedef float cvx4 __attribute__((ext_vector_type(4)));
constexpr int kMcWaves = 4;           // waves per workgroup
constexpr int kMcMaxWaves = 256 * 8;  // 8 waves per CU of the 256

template <int KS, int NB, bool VEC>
__global__ __launch_bounds__(kMcWaves * 64) void conv_mfma_direct_k(
    const float *__restrict__ in, const float *__restrict__ w, float *__restrict__ out, int M,
    int H, int W, int cin, int K, int Co) {
  const int lane = threadIdx.x % 64, l16 = lane % 16, g = lane / 16;
  const int wave = blockIdx.x * kMcWaves + threadIdx.x / 64;
  const int nwaves = gridDim.x * kMcWaves, tiles = (M >> 4) + ((M & 15) != 0);
  const int co0 = blockIdx.y * 16 * NB, KD = K * K * cin, pad = K / 2;
  float wt[KS][NB];
  int dh[KS], dw[KS], off[KS];
  const float *wrow[NB];  // this lane's weight row in each channel block
#pragma unroll
  for (int b = 0; b < NB; ++b) wrow[b] = w + int64_t(co0 + 16 * b + l16) * KD;
  // (kh, kw, ci) of k = 4s + g without division: k grows by 4 per step, so
  // ci passes cin, and kw passes K, at most 4 times per step.
  int ci = g, kh = 0, kw = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (ci >= cin) ci -= cin, ++kw;
#pragma unroll
  for (int s = 0; s < KS; ++s) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (kw >= K) kw -= K, ++kh;
    const int k = 4 * s + g;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int co = co0 + 16 * b + l16;
      wt[s][b] = k < KD && co < Co ? wrow[b][k] : 0.0f;
    }
    dh[s] = k < KD ? kh - pad : -(1 << 30);  // past K*K*C_in: never inside
    dw[s] = k < KD ? kw - pad : -(1 << 30);
    off[s] = k < KD ? (dh[s] * W + dw[s]) * cin + ci : 0;
    ci += 4;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (ci >= cin) ci -= cin, ++kw;
  }
  // Pixel indices as unsigned: 16 * tile + 15 may pass INT32_MAX.
  const unsigned hw = unsigned(H) * unsigned(W), uw = unsigned(W);
  auto gather = [&](int t, float (&x)[KS]) {
    const unsigned m = 16u * unsigned(t) + unsigned(l16), n = m / hw, rem = m - n * hw;
    const int oh = int(rem / uw), ow = int(rem - unsigned(oh) * uw);
    const bool valid = m < unsigned(M);
    const float *px = in + int64_t(m) * cin;  // once per tile, not per step
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const bool inside = valid && unsigned(oh + dh[s]) < unsigned(H) &&
                          unsigned(ow + dw[s]) < unsigned(W);
      x[s] = inside ? px[off[s]] : 0.0f;
    }
  };
  int t = wave;
  float x[KS];
  if (t < tiles) gather(t, x);
  while (t < tiles) {
    const int tn = t + nwaves;
    float xn[KS];
    if (tn < tiles) gather(tn, xn);
    cvx4 acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = cvx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int b = 0; b < NB; ++b)
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(wt[s][b], x[s], acc[b], 0, 0, 0);
    const unsigned m = 16u * unsigned(t) + unsigned(l16);
    if (m < unsigned(M)) {
      float *o = out + int64_t(m) * Co;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int c = co0 + 16 * b + 4 * g;
        if (VEC && c + 4 <= Co) {
          *reinterpret_cast<float4 *>(o + c) =
              make_float4(acc[b][0], acc[b][1], acc[b][2], acc[b][3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (c + r < Co) o[c + r] = acc[b][r];
        }
      }
    }
    t = tn;
#pragma unroll
    for (int s = 0; s < KS; ++s) x[s] = xn[s];
  }
}

template <int KS, int NB, bool VEC>
void launch_mcd(const float *in, const float *w, float *out, int M, int H, int W, int cin, int K,
                int Co, int waves, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((waves + kMcWaves - 1) / kMcWaves),
                  static_cast<unsigned>((Co + 16 * NB - 1) / (16 * NB)), 1u);
  conv_mfma_direct_k<KS, NB, VEC><<<grid, kMcWaves * 64, 0, s>>>(in, w, out, M, H, W, cin, K,
                                                                 Co);
}

template <int KS, bool VEC>
void launch_mcd_nb(const float *in, const float *w, float *out, int M, int H, int W, int cin,
                   int K, int Co, int waves, hipStream_t s) {
  if (Co <= 16) launch_mcd<KS, 1, VEC>(in, w, out, M, H, W, cin, K, Co, waves, s);
  else if (Co <= 32) launch_mcd<KS, 2, VEC>(in, w, out, M, H, W, cin, K, Co, waves, s);
  else launch_mcd<KS, 4, VEC>(in, w, out, M, H, W, cin, K, Co, waves, s);
}

template <bool VEC>
int launch_direct(const float *in, const float *w, float *out, int M, int H, int W, int cin,
                  int K, int Co, hipStream_t s) {
  // Waves: one per 16-pixel tile up to kMcMaxWaves, then grid-stride.
  const int tiles = (M >> 4) + ((M & 15) != 0);
  const int waves = tiles < kMcMaxWaves ? tiles : kMcMaxWaves;
  const int steps = (K * K * cin + 3) / 4;
  if (steps <= 1) launch_mcd_nb<1, VEC>(in, w, out, M, H, W, cin, K, Co, waves, s);
  else if (steps <= 2) launch_mcd_nb<2, VEC>(in, w, out, M, H, W, cin, K, Co, waves, s);
  else if (steps <= 4) launch_mcd_nb<4, VEC>(in, w, out, M, H, W, cin, K, Co, waves, s);
  else if (steps <= 7) launch_mcd_nb<7, VEC>(in, w, out, M, H, W, cin, K, Co, waves, s);
  else if (steps <= 10) launch_mcd_nb<10, VEC>(in, w, out, M, H, W, cin, K, Co, waves, s);
  else launch_mcd_nb<16, VEC>(in, w, out, M, H, W, cin, K, Co, waves, s);
  SILGPU_LAUNCH_CHECK("conv_mfma_direct_k");
  return SILGPU_OK;
}

}  // namespace

int conv2d_direct(const float *in, const float *w, float *out, int M, int H, int W, int cin,
                  int K, int Co, hipStream_t s) {
  return Co % 4 == 0 && aligned16(out) ? launch_direct<true>(in, w, out, M, H, W, cin, K, Co, s)
                                       : launch_direct<false>(in, w, out, M, H, W, cin, K, Co, s);
}

}  // namespace silgpu

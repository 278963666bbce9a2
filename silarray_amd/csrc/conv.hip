// Direct 2-D convolution for short reductions (K*K*C_in <= kConvDirectMaxK,
// e.g. the 3-channel first layer of an image network), where an MFMA tile
// would spend its time filling and draining: one output pixel and 16
// output channels per thread, the weights of those channels in LDS.
//
// Layouts as silgpu_conv2d_f32: NHWC input [N][H][W][C_in], OHWI weight
// [C_out][K][K][C_in], NHWC output; stride 1, zero padding K/2.  Each output
// is the float32 sum over k = (kh*K + kw)*C_in + ci in increasing k, one
// fused multiply-add per term (padding taps contribute 0 * w, as in the
// implicit GEMM).

#include "internal.h"

namespace silgpu {
namespace {

constexpr int kDirCo = 16;        // output channels per thread
constexpr int kDirThreads = 256;  // output pixels per workgroup
constexpr size_t kDirStagedLds = size_t(64) << 10;

// STAGED: the input pixels the workgroup's 256 outputs can touch -- pixel
// indices m0 - halo .. m0 + 255 + halo with halo = pad * (W + 1), one
// contiguous NHWC range -- are copied to LDS first (coalesced, all loads in
// flight together); a tap inside the image reads pixel m + (kh - pad) * W +
// (kw - pad) of that range.  Otherwise every tap is a global (cached) load.
template <bool VEC, bool STAGED>
__global__ __launch_bounds__(kDirThreads) void conv_direct_k(
    const float *__restrict__ in, const float *__restrict__ w, float *__restrict__ out, int M,
    int H, int W, int cin, int K, int pad, int Co, int Kd, int halo) {
  extern __shared__ float4 lds4[];
  float *ws = reinterpret_cast<float *>(lds4);  // [Kd][kDirCo], 0 past C_out
  float *xs = ws + Kd * kDirCo;                 // staged pixels [p0, p1) x C_in
  const int co0 = blockIdx.y * kDirCo, m0 = blockIdx.x * kDirThreads;
  for (int i = threadIdx.x; i < Kd * kDirCo; i += kDirThreads) {
    const int k = i / kDirCo, c = i % kDirCo;
    ws[i] = co0 + c < Co ? w[int64_t(co0 + c) * Kd + k] : 0.0f;
  }
  int p0 = 0;
  if constexpr (STAGED) {
    p0 = max(0, m0 - halo);
    const int p1 = min(M, m0 + kDirThreads + halo);
    const float *src = in + int64_t(p0) * cin;
    const int nf = (p1 - p0) * cin;
    for (int i = threadIdx.x; i < nf; i += kDirThreads) xs[i] = src[i];
  }
  __syncthreads();
  const int m = m0 + threadIdx.x;
  if (m >= M) return;
  const int hw = H * W, n = m / hw, rem = m - n * hw, oh = rem / W, ow = rem - oh * W;
  const float *img = in + int64_t(n) * hw * cin;
  float acc[kDirCo];
#pragma unroll
  for (int c = 0; c < kDirCo; ++c) acc[c] = 0.0f;
  const float4 *wk = lds4;
  for (int kh = 0; kh < K; ++kh) {
    const int ih = oh + kh - pad;
    for (int kw = 0; kw < K; ++kw) {
      const int iw = ow + kw - pad;
      const bool inside = unsigned(ih) < unsigned(H) && unsigned(iw) < unsigned(W);
      const float *px = STAGED ? xs + (m + (kh - pad) * W + (kw - pad) - p0) * cin
                               : img + (int64_t(ih) * W + iw) * cin;
      for (int ci = 0; ci < cin; ++ci, wk += kDirCo / 4) {
        const float x = inside ? px[ci] : 0.0f;
#pragma unroll
        for (int c4 = 0; c4 < kDirCo / 4; ++c4) {
          const float4 v = wk[c4];
          acc[4 * c4 + 0] = fmaf(x, v.x, acc[4 * c4 + 0]);
          acc[4 * c4 + 1] = fmaf(x, v.y, acc[4 * c4 + 1]);
          acc[4 * c4 + 2] = fmaf(x, v.z, acc[4 * c4 + 2]);
          acc[4 * c4 + 3] = fmaf(x, v.w, acc[4 * c4 + 3]);
        }
      }
    }
  }
  float *o = out + int64_t(m) * Co + co0;
  const int nc = min(kDirCo, Co - co0);
  if constexpr (VEC) {  // C_out % 4 == 0, 16-byte aligned output
#pragma unroll
    for (int c4 = 0; c4 < kDirCo / 4; ++c4)
      if (4 * c4 < nc)
        *reinterpret_cast<float4 *>(o + 4 * c4) =
            make_float4(acc[4 * c4], acc[4 * c4 + 1], acc[4 * c4 + 2], acc[4 * c4 + 3]);
  } else {
#pragma unroll
    for (int c = 0; c < kDirCo; ++c)
      if (c < nc) o[c] = acc[c];
  }
}

template <bool VEC>
int launch_direct(const float *in, const float *w, float *out, int M, int H, int W, int cin,
                  int K, int Co, hipStream_t s) {
  const int Kd = K * K * cin, pad = K / 2;
  const dim3 grid(static_cast<unsigned>((M + kDirThreads - 1) / kDirThreads),
                  static_cast<unsigned>((Co + kDirCo - 1) / kDirCo), 1u);
  const size_t wbytes = size_t(Kd) * kDirCo * sizeof(float);
  const int64_t halo = int64_t(pad) * (int64_t(W) + 1);
  const size_t staged = wbytes + size_t(kDirThreads + 2 * halo) * cin * sizeof(float);
  if (staged <= kDirStagedLds) {
    // Once per process (a thread-safe static), before the first launch.
    static const hipError_t attr_rc =
        hipFuncSetAttribute(reinterpret_cast<const void *>(conv_direct_k<VEC, true>),
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(kDirStagedLds));
    SILGPU_HIP_CHECK(attr_rc);
    conv_direct_k<VEC, true><<<grid, kDirThreads, staged, s>>>(in, w, out, M, H, W, cin, K, pad,
                                                               Co, Kd, static_cast<int>(halo));
  } else {
    conv_direct_k<VEC, false><<<grid, kDirThreads, wbytes, s>>>(in, w, out, M, H, W, cin, K, pad,
                                                                Co, Kd, 0);
  }
  SILGPU_LAUNCH_CHECK("conv_direct_k");
  return SILGPU_OK;
}

}  // namespace

int conv2d_direct(const float *in, const float *w, float *out, int M, int H, int W, int cin,
                  int K, int Co, hipStream_t s) {
  return Co % 4 == 0 && aligned16(out) ? launch_direct<true>(in, w, out, M, H, W, cin, K, Co, s)
                                       : launch_direct<false>(in, w, out, M, H, W, cin, K, Co, s);
}

}  // namespace silgpu

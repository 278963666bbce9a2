// Elementwise kernels: binary ops with the reference's i % len broadcast,
// stride-based broadcast, unary ops, affine, bias+sigmoid, sigmoid backward,
// fills and the fused elementwise program that sil::eval() lowers chains to.
//
// All of these are HBM-bound: 8 (unary) or 12 (binary) bytes per element.
// Each thread moves 16-byte vectors (global_load_dwordx4) in a grid-stride
// loop so a launch keeps enough bytes in flight to approach HBM bandwidth.
#include <hip/hip_runtime.h>

#include <cmath>

#include "internal.h"


namespace silgpu {
namespace {

constexpr int kBlock = 256;

// Grid size for a grid-stride loop over `work` items.  Streaming kernels on
// MI355X run fastest with one 16-byte vector per thread and a grid as large
// as the work (measured: 6.1 TB/s for a copy against 4.3-5.2 TB/s for a
// grid-stride loop over a grid of a few thousand workgroups), so the cap only
// bounds pathological sizes.
inline unsigned grid_for(int64_t work, int64_t per_block = kBlock) {
  int64_t g = cdiv(work, per_block);
  if (g < 1) g = 1;
  if (g > (int64_t(1) << 24)) g = int64_t(1) << 24;
  return static_cast<unsigned>(g);
}

template <int OP>
__device__ __forceinline__ float apply_f(float a, float b) {
  if constexpr (OP == SILGPU_ADD) return a + b;
  else if constexpr (OP == SILGPU_SUB) return a - b;
  else if constexpr (OP == SILGPU_MUL) return a * b;
  else if constexpr (OP == SILGPU_DIV) return a / b;
  else return powf(a, b);
}

template <int OP>
__device__ __forceinline__ int32_t apply_i(int32_t a, int32_t b) {
  if constexpr (OP == SILGPU_ADD) return a + b;
  else if constexpr (OP == SILGPU_SUB) return a - b;
  else if constexpr (OP == SILGPU_MUL) return a * b;
  else if constexpr (OP == SILGPU_DIV) return b == 0 ? 0 : a / b;
  // gpu_kernels.metal:860-862: round(pow(float(a), float(b)))
  else return static_cast<int32_t>(rintf(powf(static_cast<float>(a), static_cast<float>(b))));
}

template <int OP>
__device__ __forceinline__ float4 apply4(float4 a, float4 b) {
  return make_float4(apply_f<OP>(a.x, b.x), apply_f<OP>(a.y, b.y), apply_f<OP>(a.z, b.z),
                     apply_f<OP>(a.w, b.w));
}

// Both operands full length, 16-byte aligned: pure streaming.
template <int OP, bool NT>
__global__ __launch_bounds__(kBlock) void binary_full_vec(const float4 *__restrict__ a,
                                                          const float4 *__restrict__ b,
                                                          float4 *__restrict__ out,
                                                          int64_t n4) {
  int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n4; i += stride)
    st4<NT>(out + i, apply4<OP>(ld4<NT>(a + i), ld4<NT>(b + i)));
}

// One side is a single value (scalar operand, the reference's B_length == 1
// fast path, gpu_kernels.metal:891-893).  SCALAR_ON_B selects the side.
template <int OP, bool SCALAR_ON_B, bool NT>
__global__ __launch_bounds__(kBlock) void binary_scalar_vec(const float4 *__restrict__ v,
                                                            const float *__restrict__ s,
                                                            float4 *__restrict__ out,
                                                            int64_t n4) {
  float sv = s[0];
  float4 s4 = make_float4(sv, sv, sv, sv);
  int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n4; i += stride) {
    const float4 x = ld4<NT>(v + i);
    st4<NT>(out + i, SCALAR_ON_B ? apply4<OP>(x, s4) : apply4<OP>(s4, x));
  }
}

// Full-length operand against a repeating operand whose length is a multiple
// of 4 (row-vector bias add and the like).  ROW_ON_B selects the side.
template <int OP, bool ROW_ON_B>
__global__ __launch_bounds__(kBlock) void binary_row_vec(const float4 *__restrict__ v,
                                                         const float4 *__restrict__ row,
                                                         float4 *__restrict__ out,
                                                         int64_t n4, int64_t row4) {
  int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n4; i += stride) {
    float4 r = row[i % row4];
    out[i] = ROW_ON_B ? apply4<OP>(v[i], r) : apply4<OP>(r, v[i]);
  }
}

// General rule of the reference kernel: out[i] = a[i % a_len] op b[i % b_len]
// (gpu_kernels.metal:826-842), one element per thread iteration.
template <int OP, typename T>
__global__ __launch_bounds__(kBlock) void binary_mod(const T *__restrict__ a, int64_t a_len,
                                                     const T *__restrict__ b, int64_t b_len,
                                                     T *__restrict__ out, int64_t n) {
  int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    T x = a[a_len == n ? i : i % a_len];
    T y = b[b_len == n ? i : i % b_len];
    if constexpr (sizeof(T) == 4 && std::is_same<T, float>::value)
      out[i] = apply_f<OP>(x, y);
    else
      out[i] = apply_i<OP>(x, y);
  }
}

struct strided_args {
  int ndim;
  int64_t shape[8];
  int64_t sa[8];
  int64_t sb[8];
};

template <int OP>
__global__ __launch_bounds__(kBlock) void binary_strided(const float *__restrict__ a,
                                                         const float *__restrict__ b,
                                                         float *__restrict__ out, int64_t n,
                                                         strided_args g) {
  int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    int64_t rem = i, oa = 0, ob = 0;
    for (int d = g.ndim - 1; d >= 0; --d) {
      int64_t idx = rem % g.shape[d];
      rem /= g.shape[d];
      oa += idx * g.sa[d];
      ob += idx * g.sb[d];
    }
    out[i] = apply_f<OP>(a[oa], b[ob]);
  }
}

template <int OP>
int launch_binary_f32(const float *a, int64_t a_len, const float *b, int64_t b_len,
                      float *out, int64_t n, hipStream_t s) {
  bool al = aligned16(a) && aligned16(b) && aligned16(out);
  if (al && n % 4 == 0) {
    int64_t n4 = n / 4;
    const bool nt = n * 4 >= kStreamBytes;
    const float4 *a4 = reinterpret_cast<const float4 *>(a);
    const float4 *b4 = reinterpret_cast<const float4 *>(b);
    float4 *o4 = reinterpret_cast<float4 *>(out);
    if (a_len == n && b_len == n) {
      if (nt) binary_full_vec<OP, true><<<grid_for(n4), kBlock, 0, s>>>(a4, b4, o4, n4);
      else binary_full_vec<OP, false><<<grid_for(n4), kBlock, 0, s>>>(a4, b4, o4, n4);
      SILGPU_LAUNCH_CHECK("binary_full_vec");
      return SILGPU_OK;
    }
    if (a_len == n && b_len == 1) {
      if (nt) binary_scalar_vec<OP, true, true><<<grid_for(n4), kBlock, 0, s>>>(a4, b, o4, n4);
      else binary_scalar_vec<OP, true, false><<<grid_for(n4), kBlock, 0, s>>>(a4, b, o4, n4);
      SILGPU_LAUNCH_CHECK("binary_scalar_vec");
      return SILGPU_OK;
    }
    if (b_len == n && a_len == 1) {
      if (nt) binary_scalar_vec<OP, false, true><<<grid_for(n4), kBlock, 0, s>>>(b4, a, o4, n4);
      else binary_scalar_vec<OP, false, false><<<grid_for(n4), kBlock, 0, s>>>(b4, a, o4, n4);
      SILGPU_LAUNCH_CHECK("binary_scalar_vec");
      return SILGPU_OK;
    }
    if (a_len == n && b_len % 4 == 0 && n % b_len == 0) {
      binary_row_vec<OP, true><<<grid_for(n4), kBlock, 0, s>>>(
          reinterpret_cast<const float4 *>(a), reinterpret_cast<const float4 *>(b),
          reinterpret_cast<float4 *>(out), n4, b_len / 4);
      SILGPU_LAUNCH_CHECK("binary_row_vec");
      return SILGPU_OK;
    }
    if (b_len == n && a_len % 4 == 0 && n % a_len == 0) {
      binary_row_vec<OP, false><<<grid_for(n4), kBlock, 0, s>>>(
          reinterpret_cast<const float4 *>(b), reinterpret_cast<const float4 *>(a),
          reinterpret_cast<float4 *>(out), n4, a_len / 4);
      SILGPU_LAUNCH_CHECK("binary_row_vec");
      return SILGPU_OK;
    }
  }
  binary_mod<OP, float><<<grid_for(n), kBlock, 0, s>>>(a, a_len, b, b_len, out, n);
  SILGPU_LAUNCH_CHECK("binary_mod<f32>");
  return SILGPU_OK;
}

// ---- unary ------------------------------------------------------------------

template <int OP>
__device__ __forceinline__ float unary_f(float x) {
  if constexpr (OP == SILGPU_SIGMOID) return sigmoidf_dev(x);
  else return fmaxf(x, 0.0f);
}

template <int OP, bool NT>
__global__ __launch_bounds__(kBlock) void unary_vec(const float4 *__restrict__ in,
                                                    float4 *__restrict__ out, int64_t n4) {
  int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n4; i += stride) {
    float4 v = ld4<NT>(in + i);
    st4<NT>(out + i, make_float4(unary_f<OP>(v.x), unary_f<OP>(v.y), unary_f<OP>(v.z),
                                 unary_f<OP>(v.w)));
  }
}

template <int OP>
__global__ __launch_bounds__(kBlock) void unary_scalar(const float *__restrict__ in,
                                                       float *__restrict__ out, int64_t n) {
  int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
    out[i] = unary_f<OP>(in[i]);
}

template <int OP>
int launch_unary(const float *in, float *out, int64_t n, hipStream_t s) {
  if (aligned16(in) && aligned16(out) && n % 4 == 0) {
    if (n * 4 >= kStreamBytes)
      unary_vec<OP, true><<<grid_for(n / 4), kBlock, 0, s>>>(
          reinterpret_cast<const float4 *>(in), reinterpret_cast<float4 *>(out), n / 4);
    else
      unary_vec<OP, false><<<grid_for(n / 4), kBlock, 0, s>>>(
          reinterpret_cast<const float4 *>(in), reinterpret_cast<float4 *>(out), n / 4);
    SILGPU_LAUNCH_CHECK("unary_vec");
  } else {
    unary_scalar<OP><<<grid_for(n), kBlock, 0, s>>>(in, out, n);
    SILGPU_LAUNCH_CHECK("unary_scalar");
  }
  return SILGPU_OK;
}

__global__ __launch_bounds__(kBlock) void sigmoid_backward_k(const float *__restrict__ dout,
                                                             const float *__restrict__ x,
                                                             float *__restrict__ out,
                                                             int64_t n) {
  int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    float s = sigmoidf_dev(x[i]);
    out[i] = dout[i] * s * (1.0f - s);
  }
}

__global__ __launch_bounds__(kBlock) void bias_sigmoid_k(float *__restrict__ data,
                                                         const float *__restrict__ bias,
                                                         int64_t n, int64_t cols) {
  int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
    data[i] = sigmoidf_dev(data[i] + bias[i % cols]);
}

template <bool NT>
__global__ __launch_bounds__(kBlock) void affine_vec(const float4 *__restrict__ in,
                                                     float4 *__restrict__ out, int64_t n4,
                                                     float scale, float offset) {
  int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n4; i += stride) {
    float4 v = ld4<NT>(in + i);
    st4<NT>(out + i, make_float4(fmaf(v.x, scale, offset), fmaf(v.y, scale, offset),
                                 fmaf(v.z, scale, offset), fmaf(v.w, scale, offset)));
  }
}

__global__ __launch_bounds__(kBlock) void affine_scalar(const float *__restrict__ in,
                                                        float *__restrict__ out, int64_t n,
                                                        float scale, float offset) {
  int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
    out[i] = fmaf(in[i], scale, offset);
}

__global__ __launch_bounds__(kBlock) void fill_u32_k(uint32_t *__restrict__ d, uint32_t v,
                                                     int64_t n) {
  int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) d[i] = v;
}

// ---- fused elementwise program ------------------------------------------------
//
// Each thread evaluates the program for kVec = 4 consecutive output elements
// per grid-stride step: thread t of workgroup b holds elements
// (b * kBlock + t) * 4 + c, so every load and store instruction of a wave
// covers 1 KiB of contiguous memory (16-byte accesses where the operand is
// 16-byte aligned).  Register indices are uniform across the workgroup, so
// the switch statements below become scalar branches.  Every operation
// rounds to fp32 (the file is compiled with -ffp-contract=off), which makes
// the fused result bit-identical to evaluating the graph node by node.
// Measured on MI355X (c = a + b over 10M floats): 25.3 us = 4.7 TB/s, against
// 46.5 us with 8 strided scalar loads per lane and the register file in
// scratch memory, and 27.3 us with two groups of four per thread (112 VGPRs).

constexpr int kVec = 4;

struct vreg {
  float v[kVec];
};

// The program's eight registers of four floats as one 32-float vector value:
// the register index is uniform, so a dynamic element access compiles to an
// indexed VGPR move (M0-relative), and the file never leaves VGPRs.  (An
// array or struct accessed through a switch is merged by the compiler into
// one indexed memory access, which puts it in scratch.)
typedef float regvec __attribute__((ext_vector_type(SILGPU_PROG_MAX_REGS * 4)));

struct regfile {
  regvec g0;
  __device__ __forceinline__ vreg get(int i) const {
    vreg v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v.v[e] = g0[i * 4 + e];
    return v;
  }
  __device__ __forceinline__ void set(int i, const vreg &v) {
#pragma unroll
    for (int e = 0; e < 4; ++e) g0[i * 4 + e] = v.v[e];
  }
};
static_assert(SILGPU_PROG_MAX_REGS * 4 == 32 && kVec == 4, "one 32-float register vector");

// How an input is read at output element i.
enum prog_in_mode : int32_t {
  kInContig = 0,   // src[i]
  kInScalar = 1,   // src[0]
  kInStrided = 2,  // src[sum_d idx_d * stride_d]
  kInPeriod = 3,   // src[i % period]: a contiguous block repeated along the
                   // leading axes (a row or matrix broadcast)
};

struct prog_launch {
  silgpu_program p;
  int32_t mode[SILGPU_PROG_MAX_INPUTS];
  int32_t vec[SILGPU_PROG_MAX_INPUTS];  // 16-byte loads (aligned; period % 4 == 0)
  int64_t period[SILGPU_PROG_MAX_INPUTS];
  int32_t out_vec;                      // 16-byte stores
  int32_t small;                        // n < 2^32: 32-bit index arithmetic
};

__device__ __forceinline__ int64_t strided_offset(const silgpu_program &p, int in,
                                                  int64_t i) {
  int64_t rem = i, off = 0;
  for (int d = p.ndim - 1; d >= 0; --d) {
    int64_t idx = rem % p.shape[d];
    rem /= p.shape[d];
    off += idx * p.inputs[in].strides[d];
  }
  return off;
}

__device__ __forceinline__ int64_t period_offset(int64_t i, int64_t period, bool small) {
  return small ? int64_t(uint32_t(i) % uint32_t(period)) : i % period;
}

// The four elements i .. i + 3 of input k (zeros past n).
__device__ __forceinline__ float4 load_group(const prog_launch &L, int k, int64_t i, int64_t n,
                                             bool small) {
  const silgpu_program &p = L.p;
  const float *src = p.inputs[k].ptr;
  const int mode = L.mode[k];
  if (mode == kInScalar) {
    const float sv = src[0];
    return make_float4(sv, sv, sv, sv);
  }
  const int64_t period = L.period[k];
  if (L.vec[k] && i + 3 < n) {
    const int64_t o = mode == kInContig ? i : period_offset(i, period, small);
    return *reinterpret_cast<const float4 *>(src + o);
  }
  float x[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int64_t ic = i + c;
    x[c] = 0.0f;
    if (ic < n) {
      const int64_t o = mode == kInContig  ? ic
                        : mode == kInPeriod ? period_offset(ic, period, small)
                                            : strided_offset(p, k, ic);
      x[c] = src[o];
    }
  }
  return make_float4(x[0], x[1], x[2], x[3]);
}

__global__ __launch_bounds__(kBlock) void program_k(prog_launch L, float *__restrict__ out,
                                                    int64_t n) {
  const silgpu_program &p = L.p;
  const bool small = L.small != 0;
  const int64_t step = int64_t(gridDim.x) * kBlock * kVec;
  for (int64_t b0 = int64_t(blockIdx.x) * kBlock * kVec; b0 < n; b0 += step) {
    const int64_t i0 = b0 + int64_t(threadIdx.x) * 4;
    regfile r{};
    for (int pc = 0; pc < p.n_instrs; ++pc) {
      const silgpu_prog_instr ins = p.instrs[pc];
      vreg d;
      switch (ins.op) {
        case SILGPU_PI_LOAD: {
          const float4 x0 = load_group(L, ins.a, i0, n, small);
          d.v[0] = x0.x;
          d.v[1] = x0.y;
          d.v[2] = x0.z;
          d.v[3] = x0.w;
          break;
        }
        case SILGPU_PI_CONST:
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = ins.imm;
          break;
        case SILGPU_PI_ADD: {
          vreg a = r.get(ins.a), b = r.get(ins.b);
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = a.v[e] + b.v[e];
          break;
        }
        case SILGPU_PI_SUB: {
          vreg a = r.get(ins.a), b = r.get(ins.b);
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = a.v[e] - b.v[e];
          break;
        }
        case SILGPU_PI_MUL: {
          vreg a = r.get(ins.a), b = r.get(ins.b);
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = a.v[e] * b.v[e];
          break;
        }
        case SILGPU_PI_DIV: {
          vreg a = r.get(ins.a), b = r.get(ins.b);
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = a.v[e] / b.v[e];
          break;
        }
        case SILGPU_PI_POW: {
          vreg a = r.get(ins.a), b = r.get(ins.b);
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = powf(a.v[e], b.v[e]);
          break;
        }
        case SILGPU_PI_ADDI: {
          vreg a = r.get(ins.a);
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = a.v[e] + ins.imm;
          break;
        }
        case SILGPU_PI_MULI: {
          vreg a = r.get(ins.a);
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = a.v[e] * ins.imm;
          break;
        }
        case SILGPU_PI_RSUBI: {
          vreg a = r.get(ins.a);
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = ins.imm - a.v[e];
          break;
        }
        case SILGPU_PI_RDIVI: {
          vreg a = r.get(ins.a);
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = ins.imm / a.v[e];
          break;
        }
        case SILGPU_PI_SIGMOID: {
          vreg a = r.get(ins.a);
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = sigmoidf_dev(a.v[e]);
          break;
        }
        case SILGPU_PI_RELU: {
          vreg a = r.get(ins.a);
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = fmaxf(a.v[e], 0.0f);
          break;
        }
        case SILGPU_PI_FMAI: {
          vreg a = r.get(ins.a);
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = fmaf(a.v[e], ins.imm, ins.imm2);
          break;
        }
        case SILGPU_PI_SIGBWD: {
          vreg a = r.get(ins.a), b = r.get(ins.b);
#pragma unroll
          for (int e = 0; e < kVec; ++e) {
            float s = sigmoidf_dev(a.v[e]);
            d.v[e] = b.v[e] * s * (1.0f - s);
          }
          break;
        }
        default:
#pragma unroll
          for (int e = 0; e < kVec; ++e) d.v[e] = 0.0f;
          break;
      }
      r.set(ins.dst, d);
    }
    const vreg res = r.get(p.out_reg);
    if (L.out_vec && i0 + 3 < n) {
      *reinterpret_cast<float4 *>(out + i0) = make_float4(res.v[0], res.v[1], res.v[2], res.v[3]);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (i0 + c < n) out[i0 + c] = res.v[c];
    }
  }
}

// Program that is one input followed only by FMAI on the same register: the
// lowering of a chain of scalar affine nodes (x*a+b repeated).  No register
// file, so the loop body is one fma per element per step.
struct chain_launch {
  const float *in;
  int32_t n_steps;
  float scale[SILGPU_PROG_MAX_INSTRS];
  float offset[SILGPU_PROG_MAX_INSTRS];
};

// float4s per thread per grid-stride step: on 64M floats (20 steps) 4 moved
// 6.00 TB/s, 1 (one grid-stride vector) 5.93, 8 5.73.
constexpr int kChainVec = 4;

// Applies the chain to four floats.
__device__ __forceinline__ float4 chain4(const chain_launch &L, float4 v) {
  for (int s = 0; s < L.n_steps; ++s) {
    const float a = L.scale[s], b = L.offset[s];
    v.x = fmaf(v.x, a, b);
    v.y = fmaf(v.y, a, b);
    v.z = fmaf(v.z, a, b);
    v.w = fmaf(v.w, a, b);
  }
  return v;
}

// A workgroup moves one contiguous block of kBlock * kChainVec float4s per
// step, each thread kChainVec of them strided by the workgroup width, all
// loads issued before the first store.  Whole blocks carry no per-slot
// checks (with them the compiler makes the first store wait for every load).
template <bool NT>
__global__ __launch_bounds__(kBlock) void affine_chain_k(chain_launch L,
                                                         float4 *__restrict__ out,
                                                         int64_t n4) {
  const float4 *in = reinterpret_cast<const float4 *>(L.in);
  constexpr int64_t kSpan = int64_t(kBlock) * kChainVec;
  const int64_t stride = int64_t(gridDim.x) * kSpan;
  for (int64_t b0 = int64_t(blockIdx.x) * kSpan; b0 < n4; b0 += stride) {
    const int64_t base = b0 + threadIdx.x;
    float4 v[kChainVec];
    if (b0 + kSpan <= n4) {
#pragma unroll
      for (int u = 0; u < kChainVec; ++u) v[u] = ld4<NT>(in + base + u * kBlock);
#pragma unroll
      for (int u = 0; u < kChainVec; ++u) st4<NT>(out + base + u * kBlock, chain4(L, v[u]));
    } else {
#pragma unroll
      for (int u = 0; u < kChainVec; ++u) {
        const int64_t i = base + int64_t(u) * kBlock;
        v[u] = i < n4 ? ld4<NT>(in + i) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int u = 0; u < kChainVec; ++u) {
        const int64_t i = base + int64_t(u) * kBlock;
        if (i < n4) st4<NT>(out + i, chain4(L, v[u]));
      }
    }
  }
}

}  // namespace
}  // namespace silgpu

using namespace silgpu;

#define SILGPU_DISPATCH_OP(op, FN, ...)                                           \
  switch (op) {                                                                   \
    case SILGPU_ADD: return FN<SILGPU_ADD>(__VA_ARGS__);                          \
    case SILGPU_SUB: return FN<SILGPU_SUB>(__VA_ARGS__);                          \
    case SILGPU_MUL: return FN<SILGPU_MUL>(__VA_ARGS__);                          \
    case SILGPU_DIV: return FN<SILGPU_DIV>(__VA_ARGS__);                          \
    case SILGPU_POW: return FN<SILGPU_POW>(__VA_ARGS__);                          \
    default: return set_error(SILGPU_ERR_INVALID, "unknown binary op %d", op);    \
  }

namespace {

template <int OP>
int launch_binary_i32(const int32_t *a, int64_t a_len, const int32_t *b, int64_t b_len,
                      int32_t *out, int64_t n, hipStream_t s) {
  binary_mod<OP, int32_t><<<grid_for(n), kBlock, 0, s>>>(a, a_len, b, b_len, out, n);
  SILGPU_LAUNCH_CHECK("binary_mod<i32>");
  return SILGPU_OK;
}

template <int OP>
int launch_strided(const float *a, const float *b, float *out, int64_t n,
                   const strided_args &g, hipStream_t s) {
  binary_strided<OP><<<grid_for(n), kBlock, 0, s>>>(a, b, out, n, g);
  SILGPU_LAUNCH_CHECK("binary_strided");
  return SILGPU_OK;
}

int check_binary_lens(int64_t a_len, int64_t b_len, int64_t n) {
  SILGPU_REQUIRE(n >= 0, "binary: n = %lld is negative", (long long)n);
  if (n == 0) return SILGPU_OK;
  SILGPU_REQUIRE(a_len > 0 && b_len > 0, "binary: operand length 0 with n = %lld",
                 (long long)n);
  return SILGPU_OK;
}

}  // namespace

extern "C" {

int silgpu_binary_f32(int op, const float *d_a, int64_t a_len, const float *d_b,
                      int64_t b_len, float *d_out, int64_t n) {
  int rc = check_binary_lens(a_len, b_len, n);
  if (rc != SILGPU_OK || n == 0) return rc;
  SILGPU_REQUIRE(d_a && d_b && d_out, "silgpu_binary_f32: null pointer");
  SILGPU_CTX(c);
  SILGPU_DISPATCH_OP(op, launch_binary_f32, d_a, a_len, d_b, b_len, d_out, n, c->stream);
}

int silgpu_binary_i32(int op, const int32_t *d_a, int64_t a_len, const int32_t *d_b,
                      int64_t b_len, int32_t *d_out, int64_t n) {
  int rc = check_binary_lens(a_len, b_len, n);
  if (rc != SILGPU_OK || n == 0) return rc;
  SILGPU_REQUIRE(d_a && d_b && d_out, "silgpu_binary_i32: null pointer");
  SILGPU_CTX(c);
  SILGPU_DISPATCH_OP(op, launch_binary_i32, d_a, a_len, d_b, b_len, d_out, n, c->stream);
}

int silgpu_binary_strided_f32(int op, int ndim, const int64_t *shape, const float *d_a,
                              const int64_t *a_strides, const float *d_b,
                              const int64_t *b_strides, float *d_out) {
  SILGPU_REQUIRE(ndim >= 0 && ndim <= 8, "silgpu_binary_strided_f32: ndim %d not in [0, 8]",
                 ndim);
  SILGPU_REQUIRE(ndim == 0 || (shape && a_strides && b_strides),
                 "silgpu_binary_strided_f32: null shape/strides");
  strided_args g{};
  g.ndim = ndim;
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) {
    SILGPU_REQUIRE(shape[d] >= 0, "silgpu_binary_strided_f32: negative extent");
    g.shape[d] = shape[d];
    g.sa[d] = a_strides[d];
    g.sb[d] = b_strides[d];
    n *= shape[d];
  }
  if (n == 0) return SILGPU_OK;
  SILGPU_REQUIRE(d_a && d_b && d_out, "silgpu_binary_strided_f32: null pointer");
  SILGPU_CTX(c);
  SILGPU_DISPATCH_OP(op, launch_strided, d_a, d_b, d_out, n, g, c->stream);
}

int silgpu_unary_f32(int op, const float *d_in, float *d_out, int64_t n) {
  SILGPU_REQUIRE(n >= 0, "silgpu_unary_f32: negative n");
  if (n == 0) return SILGPU_OK;
  SILGPU_REQUIRE(d_in && d_out, "silgpu_unary_f32: null pointer");
  SILGPU_CTX(c);
  switch (op) {
    case SILGPU_SIGMOID: return launch_unary<SILGPU_SIGMOID>(d_in, d_out, n, c->stream);
    case SILGPU_RELU: return launch_unary<SILGPU_RELU>(d_in, d_out, n, c->stream);
    default: return set_error(SILGPU_ERR_INVALID, "unknown unary op %d", op);
  }
}

int silgpu_sigmoid_backward_f32(const float *d_dout, const float *d_x, float *d_out,
                                int64_t n) {
  SILGPU_REQUIRE(n >= 0, "silgpu_sigmoid_backward_f32: negative n");
  if (n == 0) return SILGPU_OK;
  SILGPU_REQUIRE(d_dout && d_x && d_out, "silgpu_sigmoid_backward_f32: null pointer");
  SILGPU_CTX(c);
  sigmoid_backward_k<<<grid_for(n), kBlock, 0, c->stream>>>(d_dout, d_x, d_out, n);
  SILGPU_LAUNCH_CHECK("sigmoid_backward_k");
  return SILGPU_OK;
}

int silgpu_bias_sigmoid_f32(float *d_data, const float *d_bias, int64_t n, int64_t cols) {
  SILGPU_REQUIRE(n >= 0 && cols > 0, "silgpu_bias_sigmoid_f32: bad n/cols");
  if (n == 0) return SILGPU_OK;
  SILGPU_REQUIRE(d_data && d_bias, "silgpu_bias_sigmoid_f32: null pointer");
  SILGPU_CTX(c);
  bias_sigmoid_k<<<grid_for(n), kBlock, 0, c->stream>>>(d_data, d_bias, n, cols);
  SILGPU_LAUNCH_CHECK("bias_sigmoid_k");
  return SILGPU_OK;
}

int silgpu_affine_f32(const float *d_in, float *d_out, int64_t n, float scale,
                      float offset) {
  SILGPU_REQUIRE(n >= 0, "silgpu_affine_f32: negative n");
  if (n == 0) return SILGPU_OK;
  SILGPU_REQUIRE(d_in && d_out, "silgpu_affine_f32: null pointer");
  SILGPU_CTX(c);
  if (aligned16(d_in) && aligned16(d_out) && n % 4 == 0) {
    const float4 *i4 = reinterpret_cast<const float4 *>(d_in);
    float4 *o4 = reinterpret_cast<float4 *>(d_out);
    if (n * 4 >= kStreamBytes)
      affine_vec<true><<<grid_for(n / 4), kBlock, 0, c->stream>>>(i4, o4, n / 4, scale, offset);
    else
      affine_vec<false><<<grid_for(n / 4), kBlock, 0, c->stream>>>(i4, o4, n / 4, scale, offset);
    SILGPU_LAUNCH_CHECK("affine_vec");
  } else {
    affine_scalar<<<grid_for(n), kBlock, 0, c->stream>>>(d_in, d_out, n, scale, offset);
    SILGPU_LAUNCH_CHECK("affine_scalar");
  }
  return SILGPU_OK;
}

int silgpu_fill_u32(void *d_dst, uint32_t value, int64_t n) {
  SILGPU_REQUIRE(n >= 0, "silgpu_fill_u32: negative n");
  if (n == 0) return SILGPU_OK;
  SILGPU_REQUIRE(d_dst != nullptr, "silgpu_fill_u32: null pointer");
  SILGPU_CTX(c);
  fill_u32_k<<<grid_for(n), kBlock, 0, c->stream>>>(static_cast<uint32_t *>(d_dst), value,
                                                     n);
  SILGPU_LAUNCH_CHECK("fill_u32_k");
  return SILGPU_OK;
}

int silgpu_program_f32(const silgpu_program *prog, float *d_out) {
  SILGPU_REQUIRE(prog != nullptr, "silgpu_program_f32: prog is null");
  const silgpu_program &p = *prog;
  SILGPU_REQUIRE(p.n_inputs >= 0 && p.n_inputs <= SILGPU_PROG_MAX_INPUTS,
                 "silgpu_program_f32: n_inputs %d out of range", p.n_inputs);
  SILGPU_REQUIRE(p.n_instrs >= 1 && p.n_instrs <= SILGPU_PROG_MAX_INSTRS,
                 "silgpu_program_f32: n_instrs %d out of range", p.n_instrs);
  SILGPU_REQUIRE(p.ndim >= 0 && p.ndim <= SILGPU_PROG_MAX_DIMS,
                 "silgpu_program_f32: ndim %d out of range", p.ndim);
  SILGPU_REQUIRE(p.out_reg >= 0 && p.out_reg < SILGPU_PROG_MAX_REGS,
                 "silgpu_program_f32: out_reg %d out of range", p.out_reg);
  int64_t n = 1;
  for (int d = 0; d < p.ndim; ++d) {
    SILGPU_REQUIRE(p.shape[d] >= 0, "silgpu_program_f32: negative extent");
    n *= p.shape[d];
  }
  if (n == 0) return SILGPU_OK;
  SILGPU_REQUIRE(d_out != nullptr, "silgpu_program_f32: d_out is null");
  prog_launch L{};
  L.p = p;
  for (int i = 0; i < p.n_inputs; ++i) {
    SILGPU_REQUIRE(p.inputs[i].ptr != nullptr, "silgpu_program_f32: input %d is null", i);
    bool all_zero = true, contiguous = true;
    int64_t expect = 1;
    for (int d = p.ndim - 1; d >= 0; --d) {
      if (p.inputs[i].strides[d] != 0) all_zero = false;
      if (p.shape[d] != 1 && p.inputs[i].strides[d] != expect) contiguous = false;
      expect *= p.shape[d];
    }
    // A contiguous block over the trailing axes [k, ndim) repeated along
    // axes [0, k) (zero strides there): offset = i % period.
    int k = p.ndim;
    int64_t period = 1;
    while (k > 0 && (p.shape[k - 1] == 1 || p.inputs[i].strides[k - 1] == period)) {
      period *= p.shape[k - 1];
      --k;
    }
    bool repeated = true;
    for (int d = 0; d < k; ++d)
      if (p.shape[d] != 1 && p.inputs[i].strides[d] != 0) repeated = false;
    const bool aligned = aligned16(p.inputs[i].ptr);
    if (all_zero) {
      L.mode[i] = kInScalar;
    } else if (contiguous) {
      L.mode[i] = kInContig;
      L.vec[i] = aligned;
    } else if (repeated) {
      L.mode[i] = kInPeriod;
      L.period[i] = period;
      L.vec[i] = aligned && period % 4 == 0;
    } else {
      L.mode[i] = kInStrided;
    }
  }
  L.out_vec = aligned16(d_out);
  L.small = n <= int64_t(UINT32_MAX);
  bool chain = p.n_inputs == 1 && L.mode[0] == 0 && p.instrs[0].op == SILGPU_PI_LOAD &&
               p.instrs[0].a == 0 && p.out_reg == p.instrs[0].dst && n % 4 == 0 &&
               aligned16(p.inputs[0].ptr) && aligned16(d_out);
  for (int pc = 0; pc < p.n_instrs; ++pc) {
    const silgpu_prog_instr &ins = p.instrs[pc];
    SILGPU_REQUIRE(ins.dst >= 0 && ins.dst < SILGPU_PROG_MAX_REGS && ins.a >= 0 &&
                       ins.b >= 0 && ins.b < SILGPU_PROG_MAX_REGS,
                   "silgpu_program_f32: register index out of range at %d", pc);
    if (ins.op == SILGPU_PI_LOAD)
      SILGPU_REQUIRE(ins.a < p.n_inputs, "silgpu_program_f32: load of input %d of %d", ins.a,
                     p.n_inputs);
    else
      SILGPU_REQUIRE(ins.a < SILGPU_PROG_MAX_REGS,
                     "silgpu_program_f32: register index out of range at %d", pc);
    SILGPU_REQUIRE(ins.op >= SILGPU_PI_LOAD && ins.op <= SILGPU_PI_SIGBWD,
                   "silgpu_program_f32: unknown opcode %d at %d", ins.op, pc);
    if (pc > 0 && !(ins.op == SILGPU_PI_FMAI && ins.dst == p.instrs[0].dst &&
                    ins.a == p.instrs[0].dst))
      chain = false;
  }
  SILGPU_CTX(c);
  // One binary operation on two loaded inputs, each contiguous, a scalar or
  // a repeated block: the reference's a[i % a_len] op b[i % b_len] rule, run
  // by the dedicated binary kernels (16-byte non-temporal streams).
  if (p.n_instrs == 3 && p.instrs[2].dst == p.out_reg && p.instrs[2].op >= SILGPU_PI_ADD &&
      p.instrs[2].op <= SILGPU_PI_POW && p.instrs[0].op == SILGPU_PI_LOAD &&
      p.instrs[1].op == SILGPU_PI_LOAD && p.instrs[0].dst != p.instrs[1].dst) {
    const silgpu_prog_instr &op = p.instrs[2];
    auto operand = [&](int reg, const float *&ptr, int64_t &len) {
      const silgpu_prog_instr *ld = reg == p.instrs[0].dst   ? &p.instrs[0]
                                    : reg == p.instrs[1].dst ? &p.instrs[1]
                                                             : nullptr;
      if (ld == nullptr) return false;
      const int m = L.mode[ld->a];
      ptr = p.inputs[ld->a].ptr;
      len = m == kInContig ? n : m == kInScalar ? 1 : m == kInPeriod ? L.period[ld->a] : 0;
      return len > 0;
    };
    const float *pa = nullptr, *pb = nullptr;
    int64_t la = 0, lb = 0;
    if (operand(op.a, pa, la) && operand(op.b, pb, lb)) {
      switch (op.op) {
        case SILGPU_PI_ADD: return launch_binary_f32<SILGPU_ADD>(pa, la, pb, lb, d_out, n, c->stream);
        case SILGPU_PI_SUB: return launch_binary_f32<SILGPU_SUB>(pa, la, pb, lb, d_out, n, c->stream);
        case SILGPU_PI_MUL: return launch_binary_f32<SILGPU_MUL>(pa, la, pb, lb, d_out, n, c->stream);
        case SILGPU_PI_DIV: return launch_binary_f32<SILGPU_DIV>(pa, la, pb, lb, d_out, n, c->stream);
        default: return launch_binary_f32<SILGPU_POW>(pa, la, pb, lb, d_out, n, c->stream);
      }
    }
  }
  if (chain) {
    chain_launch C{};
    C.in = p.inputs[0].ptr;
    C.n_steps = p.n_instrs - 1;
    for (int s = 0; s < C.n_steps; ++s) {
      C.scale[s] = p.instrs[s + 1].imm;
      C.offset[s] = p.instrs[s + 1].imm2;
    }
    int64_t n4 = n / 4;
    if (n * 4 >= kStreamBytes)
      affine_chain_k<true><<<grid_for(n4, int64_t(kBlock) * kChainVec), kBlock, 0, c->stream>>>(
          C, reinterpret_cast<float4 *>(d_out), n4);
    else
      affine_chain_k<false><<<grid_for(n4, int64_t(kBlock) * kChainVec), kBlock, 0, c->stream>>>(
          C, reinterpret_cast<float4 *>(d_out), n4);
    SILGPU_LAUNCH_CHECK("affine_chain_k");
    return SILGPU_OK;
  }
  program_k<<<grid_for(n, int64_t(kBlock) * kVec), kBlock, 0, c->stream>>>(L, d_out, n);
  SILGPU_LAUNCH_CHECK("program_k");
  return SILGPU_OK;
}

}  // extern "C"

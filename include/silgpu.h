/*
 * silgpu.h — C ABI of the MI355X (gfx950) backend for the silarray hot path.
 *
 * The reference (yhirose/silarray) has no FFI: its operator boundary is the
 * header-only C++ class `sil::gpu` (include/gpu.h:266-1036) plus the
 * `gpu_context` singleton (include/gpu.h:49-260) and the unified-memory
 * `storage`/`buffer_pool` pair (include/unified_memory.h:17-79).  Every entry
 * point below replaces one of those; the reference interface it stands in for
 * is cited on each declaration.  The C++ mirror `silarray_amd/include/sil/gpu.h`
 * keeps the reference's method names and `storage` signatures and calls only
 * these functions.
 *
 * Conventions
 *   - Every function returns SILGPU_OK (0) or a negative status; the message of
 *     the last failure on the calling thread is returned by silgpu_last_error().
 *   - Pointers named d_* are device pointers (from silgpu_alloc or hipMalloc).
 *     Pointers named h_* are host pointers.
 *   - All launches are asynchronous on the library's single HIP stream and run
 *     in issue order, like the reference's single command buffer
 *     (include/gpu.h:66-77).  silgpu_sync() waits for them.
 *   - Sizes are element counts (int64_t) unless a name says bytes.
 *   - Nothing here allocates device memory except silgpu_alloc and the
 *     one-time scratch area reserved by silgpu_init.
 */
#ifndef SILGPU_H
#define SILGPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------- */
#define SILGPU_OK 0
#define SILGPU_ERR_INVALID (-1)     /* bad argument (shape, null pointer, range) */
#define SILGPU_ERR_HIP (-2)         /* a HIP runtime call or launch failed */
#define SILGPU_ERR_NOMEM (-3)       /* device or pinned allocation failed */
#define SILGPU_ERR_UNSUPPORTED (-4) /* valid request this build does not run */
#define SILGPU_ERR_NODEVICE (-5)    /* no HIP device visible */

/* ---- binary / unary operation codes ------------------------------------- */
/* Order follows the reference's ArithmeticOperation enum (include/array.h:570-576)
 * and PSO list (include/gpu.h:21-25). */
#define SILGPU_ADD 0
#define SILGPU_SUB 1
#define SILGPU_MUL 2
#define SILGPU_DIV 3
#define SILGPU_POW 4

#define SILGPU_SIGMOID 0 /* 1/(1+exp(-x)), include/gpu.h:314-316 */
#define SILGPU_RELU 1    /* max(x,0),      include/gpu.h:318-320 */

/* GEMM epilogues.  BIAS adds bias[col % bias_len] (include/gpu_kernels.metal:506-522);
 * BIAS_SIGMOID applies 1/(1+exp(-v)) after the bias (include/gpu_kernels.metal:524-542). */
#define SILGPU_EPI_NONE 0
#define SILGPU_EPI_BIAS 1
#define SILGPU_EPI_BIAS_SIGMOID 2
#define SILGPU_EPI_RELU 3
#define SILGPU_EPI_BIAS_RELU 4

/* ---- context, errors, memory -------------------------------------------- */

/* Message of the last failed call on this thread ("" if none). */
const char *silgpu_last_error(void);

/* Select device 0, create the stream, reserve scratch.  Idempotent.
 * Replaces gpu_context::instance() construction (include/gpu.h:59-62, 132-185)
 * and buffer_pool::instance() (include/unified_memory.h:33-36, 55-61). */
int silgpu_init(void);

/* Wait for all work issued so far.  Replaces gpu_context::flush()
 * (include/gpu.h:107-123) and sil::synchronize() (include/gpu.h:1375-1377). */
int silgpu_sync(void);

/* Device properties of the active device (CU count, clock in kHz, LDS bytes
 * per workgroup, gcnArchName).  No reference counterpart; used for roofline
 * reporting. */
int silgpu_device_info(int *cu_count, int *clock_khz, int *lds_bytes, char *arch,
                       size_t arch_len);

/* Pooled device allocation.  Replaces buffer_pool::acquire/release
 * (include/unified_memory.h:38-53) behind storage::make (:66-79).  Blocks are
 * reused by size class and returned to the pool by silgpu_free; the pool
 * never returns memory to HIP until silgpu_pool_trim(). */
int silgpu_alloc(size_t bytes, void **d_ptr);
int silgpu_free(void *d_ptr);
int silgpu_pool_trim(void);
/* Bytes currently handed out and bytes cached in the pool. */
int silgpu_pool_stats(size_t *in_use, size_t *cached);

/* Pinned host memory (hipHostMalloc) for the host mirror of a storage, pooled
 * by the device pool's size classes; silgpu_host_free returns the block to
 * the pool and silgpu_pool_trim() releases the cache.  Copies between pinned
 * blocks and HBM run as direct DMA.  The reference's unified memory
 * (include/unified_memory.h:38-79) needs no copies at all; this is the
 * staging side of the discrete-memory design. */
int silgpu_host_alloc(size_t bytes, void **h_ptr);
int silgpu_host_free(void *h_ptr);

/* Copies, ordered on the library stream.  h2d returns once the source may be
 * reused; d2h returns once the destination holds the data; d2d is async, its
 * two ranges must not overlap, and 16-byte-aligned ranges are moved by the
 * library's own streaming kernel (the rest by the runtime's copy).
 * Together they stand in for the host's direct access to MTLBuffer contents
 * (include/unified_memory.h:76, include/array.h:951-958). */
int silgpu_memcpy_h2d(void *d_dst, const void *h_src, size_t bytes);
int silgpu_memcpy_d2h(void *h_dst, const void *d_src, size_t bytes);
int silgpu_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes);

/* d[i] = value for i < n (4-byte elements).  Replaces the host fill in
 * array::constants (include/array.h:1268-1272) for device-resident data. */
int silgpu_fill_u32(void *d_dst, uint32_t value, int64_t n);

/* ---- elementwise -------------------------------------------------------- */

/* out[i] = a[i % a_len] op b[i % b_len] for i < n, op in SILGPU_ADD..POW.
 * Replaces gpu::add/sub/mul/div/pow (include/gpu.h:289-312) and
 * arithmetic_dispatch_ (include/gpu.h:1331-1369).  Float pow is powf; int
 * pow rounds powf of the float-converted operands (gpu_kernels.metal:860-862);
 * int division truncates. */
int silgpu_binary_f32(int op, const float *d_a, int64_t a_len, const float *d_b,
                      int64_t b_len, float *d_out, int64_t n);
int silgpu_binary_i32(int op, const int32_t *d_a, int64_t a_len, const int32_t *d_b,
                      int64_t b_len, int32_t *d_out, int64_t n);

/* Stride-based broadcast: out (contiguous, shape[0..ndim)) = a op b where a
 * and b are read through element strides (0 on broadcast axes).  ndim <= 8.
 * Covers the cases the reference materialises on the host
 * (include/array.h:2500-2518) and middle-axis broadcasts that its i%len rule
 * cannot express (include/gpu_kernels.metal:838-841). */
int silgpu_binary_strided_f32(int op, int ndim, const int64_t *shape, const float *d_a,
                              const int64_t *a_strides, const float *d_b,
                              const int64_t *b_strides, float *d_out);

/* out[i] = f(in[i]), f = SILGPU_SIGMOID | SILGPU_RELU.  Replaces gpu::sigmoid
 * and gpu::relu (include/gpu.h:314-320, 1008-1031). */
int silgpu_unary_f32(int op, const float *d_in, float *d_out, int64_t n);

/* out[i] = dout[i]*s*(1-s), s = sigmoid(x[i]).  Replaces gpu::sigmoid_backward
 * (include/gpu.h:945-962). */
int silgpu_sigmoid_backward_f32(const float *d_dout, const float *d_x, float *d_out,
                                int64_t n);

/* In place: data[i] = sigmoid(data[i] + bias[i % cols]).  Replaces
 * gpu::bias_sigmoid (include/gpu.h:965-982). */
int silgpu_bias_sigmoid_f32(float *d_data, const float *d_bias, int64_t n, int64_t cols);

/* out[i] = in[i]*scale + offset (one rounding: fused multiply-add).  Replaces
 * gpu::affine (include/gpu.h:985-1004). */
int silgpu_affine_f32(const float *d_in, float *d_out, int64_t n, float scale,
                      float offset);

/* Fused elementwise program: the lowering target of sil::eval() for chains of
 * elementwise nodes (include/array.h:1888-2022, 2836-2888), one HBM pass for a
 * whole chain.  A program is a list of register-machine instructions over
 * n_inputs input streams; every instruction rounds to fp32, no contraction,
 * so the result equals node-by-node fp32 evaluation. */
#define SILGPU_PROG_MAX_INPUTS 8
#define SILGPU_PROG_MAX_INSTRS 64
#define SILGPU_PROG_MAX_REGS 8
#define SILGPU_PROG_MAX_DIMS 6

/* instruction opcodes */
#define SILGPU_PI_LOAD 0    /* r[dst] = input[a] at this element */
#define SILGPU_PI_CONST 1   /* r[dst] = imm */
#define SILGPU_PI_ADD 2     /* r[dst] = r[a] + r[b] */
#define SILGPU_PI_SUB 3     /* r[dst] = r[a] - r[b] */
#define SILGPU_PI_MUL 4     /* r[dst] = r[a] * r[b] */
#define SILGPU_PI_DIV 5     /* r[dst] = r[a] / r[b] */
#define SILGPU_PI_POW 6     /* r[dst] = powf(r[a], r[b]) */
#define SILGPU_PI_ADDI 7    /* r[dst] = r[a] + imm */
#define SILGPU_PI_MULI 8    /* r[dst] = r[a] * imm */
#define SILGPU_PI_RSUBI 9   /* r[dst] = imm - r[a] */
#define SILGPU_PI_RDIVI 10  /* r[dst] = imm / r[a] */
#define SILGPU_PI_SIGMOID 11 /* r[dst] = 1/(1+exp(-r[a])) */
#define SILGPU_PI_RELU 12   /* r[dst] = max(r[a], 0) */
#define SILGPU_PI_FMAI 13   /* r[dst] = fma(r[a], imm, imm2) (reference affine node) */
#define SILGPU_PI_SIGBWD 14 /* r[dst] = r[b]*s*(1-s), s = sigmoid(r[a]) */

typedef struct silgpu_prog_instr {
  int32_t op;
  int32_t dst;
  int32_t a;
  int32_t b;
  float imm;
  float imm2;
} silgpu_prog_instr;

typedef struct silgpu_prog_input {
  const float *ptr;                          /* device pointer */
  int64_t strides[SILGPU_PROG_MAX_DIMS];     /* element strides, 0 = broadcast */
} silgpu_prog_input;

typedef struct silgpu_program {
  int32_t n_inputs;
  int32_t n_instrs;
  int32_t ndim;                              /* output rank (<= 6) */
  int32_t out_reg;                           /* register holding the result */
  int64_t shape[SILGPU_PROG_MAX_DIMS];       /* output shape, row-major */
  silgpu_prog_input inputs[SILGPU_PROG_MAX_INPUTS];
  silgpu_prog_instr instrs[SILGPU_PROG_MAX_INSTRS];
} silgpu_program;

int silgpu_program_f32(const silgpu_program *prog, float *d_out);

/* ---- reductions --------------------------------------------------------- */

/* *d_out = sum / min / max of d_in[0..n).  One launch, device-side final
 * reduction, fp64 accumulation for the sum.  Replaces gpu::sum_f32 /
 * min_f32 / max_f32 plus the host finish (include/gpu.h:323-354, 409-470;
 * include/array.h:1535-1545, 1612-1619, 1642-1649).  n == 0 gives 0 for sum
 * and SILGPU_ERR_INVALID for min/max. */
int silgpu_sum_f32(const float *d_in, int64_t n, float *d_out);
int silgpu_min_f32(const float *d_in, int64_t n, float *d_out);
int silgpu_max_f32(const float *d_in, int64_t n, float *d_out);

/* Sum over the middle axis of a contiguous [outer, axis_len, inner] array:
 * out[o, i] = sum_a in[o, a, i].  Covers array::sum(axis) for every axis
 * (include/array.h:1554-1583, 2275-2319): gpu::sum_axis0_f32
 * (include/gpu.h:385-406) is outer == 1, and the reference's CPU-only
 * sum(axis != 0) (include/array.h:2303-2316) is the rest. */
int silgpu_sum_axis_f32(const float *d_in, int64_t outer, int64_t axis_len,
                        int64_t inner, float *d_out);

/* out[r] = first index of the maximum of row r of a contiguous [rows, cols]
 * array (NaN never wins).  Replaces gpu::argmax_f32 (include/gpu.h:890-913);
 * long rows are split across workgroups. */
int silgpu_argmax_rows_f32(const float *d_in, int64_t rows, int64_t cols,
                           int32_t *d_out);

/* Failure reporting of the one-launch reductions (sum, min, max, argmax).
 * Their finishing workgroup waits on the device for the other workgroups'
 * partial results; the reference finishes on the host instead
 * (include/gpu.h:331-354, include/array.h:1535-1545) and never waits on the
 * device.  The wait is bounded by the device wall clock (50 ms); a finisher
 * that gives up records the failure in a host-mapped word, and the next
 * silgpu_sync (or sum/min/max/argmax call) returns SILGPU_ERR_HIP with a
 * message and clears the partial-result slots for later calls.
 *
 * Test hooks for that path, with no counterpart in the reference:
 *   silgpu_slot_wait_selftest launches a finisher over slots [0, nslots) that
 *   nothing writes, waiting wait_us before it gives up; with late_us > 0 a
 *   second workgroup publishes slot 0 after late_us (a producer later than
 *   the deadline).  *d_taken (device, uint32) is increased by the number of
 *   slots the finisher did receive.  Every wait in it ends on the wall clock.
 *   silgpu_slots_in_use synchronises and counts the slots that are not zero
 *   (zero between launches when nothing has failed). */
int silgpu_slot_wait_selftest(int nslots, int64_t wait_us, int64_t late_us,
                              uint32_t *d_taken);
int silgpu_slots_in_use(int64_t *count);

/* ---- row ops ------------------------------------------------------------ */

/* Row softmax of a contiguous [rows, cols] array: exp(x - rowmax) / sum.
 * Replaces gpu::softmax (include/gpu.h:916-942). */
int silgpu_softmax_rows_f32(const float *d_in, float *d_out, int64_t rows, int64_t cols);

/* Row layer_norm: (x - mean) / sqrt(var + eps) * gamma + beta with the
 * two-pass variance of cpu::layer_norm (include/cpu.h:352-373).  Replaces
 * gpu::layer_norm (include/gpu.h:473-501). */
int silgpu_layer_norm_rows_f32(const float *d_in, float *d_out, const float *d_gamma,
                               const float *d_beta, int64_t rows, int64_t cols,
                               float eps);

/* ---- matrix products ---------------------------------------------------- */

/* C[b] = epilogue(op(A[b]) * op(B[b])) for b < batch, row-major.
 *   op(A) is M x K: A[m*lda + k] (trans_a = 0) or A[k*lda + m] (trans_a = 1)
 *   op(B) is K x N: B[k*ldb + n] (trans_b = 0) or B[n*ldb + k] (trans_b = 1)
 *   C[m*ldc + n]; batch b adds b*stride_{a,b,c}.
 *   bias (EPI_BIAS*, may be NULL otherwise) is read as bias[n % bias_len].
 * One entry point for every reference GEMM: gpu::sgemm / sgemm_batched /
 * sgemm_steel / sgemm_steel_batched / sgemm_bias_steel /
 * sgemm_bias_sigmoid_steel / sgemv / mps::dot_f32_ex (include/gpu.h:509-535,
 * 549-590, 609-615, 1296-1328).  The library picks the kernel (fp32 MFMA
 * tiles, split-K, GEMV) from the shape. */
int silgpu_sgemm(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                 const float *d_A, int64_t lda, int64_t stride_a, const float *d_B,
                 int64_t ldb, int64_t stride_b, float *d_C, int64_t ldc,
                 int64_t stride_c, int64_t batch, const float *d_bias,
                 int64_t bias_len, int epilogue);

/* silgpu_sgemm with a forced kernel configuration, for tile sweeps.  No
 * reference counterpart.  tile: 1 = 128x128, 2 = 64x64, 3 = 32x128,
 * 4 = 128x64, 5 = 256x256 (workgroup tile of C); 6, 7, 8 = the small-M
 * kernel (M <= 32, batch 1, A not transposed; otherwise the 32x128 tile)
 * with 32, 64 or 128 columns per workgroup; 9 = 64x64 with each
 * workgroup's K range halved between two groups of waves (M, N, K
 * multiples of 64 and 16-byte aligned operands; otherwise the 64x64 tile);
 * 10 = the same with four groups (K a multiple of 128);
 * splits: K splits (>= 1; batch must be 1 for splits > 1).  Never routes to
 * the GEMV kernels. */
int silgpu_sgemm_tuned(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                       const float *d_A, int64_t lda, int64_t stride_a, const float *d_B,
                       int64_t ldb, int64_t stride_b, float *d_C, int64_t ldc,
                       int64_t stride_c, int64_t batch, const float *d_bias,
                       int64_t bias_len, int epilogue, int tile, int splits);

/* The general product, of which silgpu_sgemm is the common case:
 *   C[b] = epi(op(A[b]) * op(B[b])) for every batch index b = (o, i),
 *   o < batch_outer, i < batch_inner, with operand X[b] at
 *   X + o*stride_x_outer + i*stride_x_inner (element strides),
 * so a batch that runs over two axes with different strides (attention heads
 * split out of a [batch, seq, heads*dim] array) is one launch.  The
 * epilogue applied to each fp32 accumulator v, in this order:
 *   1. use_scale: v = fmaf(v, scale, scale_offset) (a scalar affine node of
 *      the graph folded into the product, rounded as that node rounds);
 *   2. bias (SILGPU_EPI_BIAS*): v += bias[n % bias_len];
 *   3. sigmoid or relu per `epilogue`;
 *   4. residual (non-NULL, batch 1 only): v = v + residual[m*ldr + n].
 * Serves array::dot / batched_dot / linear / linear_sigmoid lowered by
 * sil::eval (include/array.h:1360-1416, 1462-1472, 2174-2258) with the
 * graph's neighbouring scalar and residual nodes fused in. */
typedef struct silgpu_gemm_desc {
  int32_t trans_a, trans_b;
  int64_t M, N, K;
  const float *A;
  int64_t lda;
  const float *B;
  int64_t ldb;
  float *C;
  int64_t ldc;
  int64_t batch_outer, batch_inner;        /* both >= 1 for a non-empty product */
  int64_t stride_a_outer, stride_a_inner;
  int64_t stride_b_outer, stride_b_inner;
  int64_t stride_c_outer, stride_c_inner;
  int32_t epilogue;                        /* SILGPU_EPI_* */
  int32_t use_scale;
  float scale, scale_offset;
  const float *bias;
  int64_t bias_len;
  const float *residual;
  int64_t ldr;
} silgpu_gemm_desc;

int silgpu_gemm(const silgpu_gemm_desc *desc);

/* silgpu_gemm that allocates nothing.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * caller passes inputs and outputs as for silgpu_gemm; the K-split partial
 * planes and GEMV partials live in one fixed 32 MiB device array reserved
 * when the library is loaded, whose address silgpu_init looks up.
 *   - silgpu_init() must have returned SILGPU_OK first (SILGPU_ERR_INVALID
 *     otherwise); the call itself makes no hipMalloc/hipFree.
 *   - A plan whose partial planes exceed 32 MiB runs with fewer K splits
 *     (down to none), so its rounding may differ from silgpu_gemm's within
 *     the SGEMM tolerance; otherwise the result is bit-identical.  A vector
 *     product (M == 1) wider than 8M columns runs in pieces of 8M columns.
 *   - All calls on one device share the array, and it keeps the last call's
 *     contents: calls that overlap in time on one device (several host
 *     threads, several streams) race. */
int silgpu_gemm_noalloc(const silgpu_gemm_desc *desc);

/* The matrix products the last silgpu_sgemm / silgpu_sgemm_tuned /
 * silgpu_gemm / silgpu_gemm_noalloc call on this thread launched: *n of them
 * (0 for a vector product, which runs the GEMV kernels; 2 when the last
 * rows of C ran as a second product), and for each its tile configuration
 * (the numbering of silgpu_sgemm_tuned), the K splits it launched and its
 * rows of C.  The arrays hold at least two entries.  No reference
 * counterpart: a diagnostic for tests and tile sweeps. */
int silgpu_gemm_last_plan(int *n, int *tiles, int *splits, int *rows);

/* Fused attention: for every batch index b = (o, i) (o < batch_outer,
 * i < batch_inner) and query row r < Sq,
 *   O[b][r][:] = sum_j softmax_j(scale * Q[b][r] . K[b][j]) * V[b][j][:]
 * over keys j < Sk, head dim D (16, 32, 64 or 128), every operand row-major
 * with unit stride along D:  X[b][row][d] = X + o*stride_x_outer +
 * i*stride_x_inner + row*ldx + d (16-byte aligned rows are read as float4,
 * others element by element).  The scores are rounded as the product's
 * fp32 result times `scale` (fmaf(acc, scale, 0)), the softmax subtracts the
 * row maximum, and rows are normalised once at the end (online softmax), so
 * results match the unfused graph within fp32 rounding, not bit for bit.
 * No reference counterpart as one call: sil::eval lowers the reference
 * graph dot/batched_dot -> scalar scale -> softmax -> dot/batched_dot
 * (include/array.h:1360-1403, 1677-1709) onto it when the score matrix is
 * used by nothing else, so the [Sq, Sk] scores never reach HBM. */
typedef struct silgpu_attn_desc {
  int64_t Sq, Sk, D;
  int64_t batch_outer, batch_inner;
  float scale;
  const float *Q;
  int64_t ldq, stride_q_outer, stride_q_inner;
  const float *K;
  int64_t ldk, stride_k_outer, stride_k_inner;
  const float *V;
  int64_t ldv, stride_v_outer, stride_v_inner;
  float *O;
  int64_t ldo, stride_o_outer, stride_o_inner;
} silgpu_attn_desc;

int silgpu_attention_f32(const silgpu_attn_desc *desc);

/* 2-D convolution, stride 1, zero padding K/2 on every side (output H x W):
 *   out[n][oh][ow][co] = sum_{kh, kw < K, ci < C_in}
 *       in[n][oh + kh - K/2][ow + kw - K/2][ci] * w[co][kh][kw][ci]
 * with NHWC input [N][H][W][C_in], OHWI weight [C_out][K][K][C_in] and NHWC
 * output [N][H][W][C_out], all contiguous.  An implicit GEMM on the fp32
 * matrix cores (M = N*H*W output pixels, N = C_out, K = K*K*C_in; no im2col
 * buffer).  Replaces gpu::conv2d (include/gpu.h:815-833: conv2d_gemm,
 * conv2d_gemm_smallch3, MPSGraph) as array::conv2d lowers to it
 * (include/array.h:1508-1517, 2259-2273). */
int silgpu_conv2d_f32(const float *d_in, const float *d_w, float *d_out, int64_t N, int64_t H,
                      int64_t W, int64_t C_in, int64_t K, int64_t C_out);

/* y[1 x N] = x[1 x K] * B[K x N] (B row-major, ldb >= N).  Replaces gpu::sgemv
 * (include/gpu.h:549-574).  silgpu_sgemm routes M == 1 here as well. */
int silgpu_sgemv(const float *d_x, const float *d_B, int64_t ldb, float *d_y, int64_t N,
                 int64_t K);

/* ---- timing (no reference counterpart; used by bench.py) ---------------- */

/* Events recorded on the library stream, for kernel time of back-to-back
 * launches. */
int silgpu_event_create(void **ev);
int silgpu_event_destroy(void *ev);
int silgpu_event_record(void *ev);
int silgpu_event_elapsed_ms(void *ev_start, void *ev_end, float *ms);

/* The library's hipStream_t, for callers that interoperate with it. */
int silgpu_get_stream(void **stream);

#ifdef __cplusplus
}
#endif

#endif /* SILGPU_H */

/*
 * hmx.h -- C ABI of libhmx, the gfx950 (MI355X) execution target behind the
 * `helion_mlir_utils` entry points and the `gpu` value of HELION_MLIR_TARGET.
 *
 * Conventions (every function):
 *   - Returns an int status: HMX_OK (0) on success; otherwise
 *     hmx_last_error() holds a message for the calling thread.
 *   - Pointers are device pointers owned by the caller (torch tensors on the
 *     Python side). No data buffer is allocated inside: split-K partials go
 *     to the caller's `workspace` (hmx_gemm_noalloc: to the library's static
 *     per-device scratch). The one exception is code: the first call that
 *     needs a kernel compiled at run time compiles and loads it (hipRTC,
 *     hipModuleLoadData), once per process (hmx_jit_info); hmx_gemm_noalloc
 *     never does, and HMX_JIT=0 turns it off.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream)
 *     and runs asynchronously. Functions keep no mutable global state (only
 *     per-thread error messages and timing events), so they may be called
 *     from several threads at once.
 *   - Operands are dense: row-major with the given leading dimension, or a
 *     packed layout described by its HMX_B_* code. bf16 travels as raw bits.
 *   - Arguments a kernel cannot take are refused with HMX_ERR_INVALID before
 *     anything is launched; no call falls back to another implementation.
 *
 * Each entry point names the reference function it stands in for
 * (adam-smnk/helion-mlir-xsmm, file:line). The reference's own native ABI is
 * `void entry(void** packed)` (helion_mlir_backend/_compiler/native/call.cpp:33),
 * one per JIT-compiled Helion kernel; here each hot-path kernel family has
 * one typed entry point instead.
 */
#ifndef HMX_H
#define HMX_H

#ifndef __HIPCC_RTC__
#include <stdint.h>
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define HMX_ABI_VERSION 5

/* Status codes. */
#define HMX_OK 0
#define HMX_ERR_INVALID 1     /* an argument the kernels cannot take */
#define HMX_ERR_HIP 2         /* a HIP runtime error (launch, device) */
#define HMX_ERR_UNSUPPORTED 3 /* not a gfx950 device */

/* Storage dtypes. bf16 is carried as its raw 16 bits. */
#define HMX_DTYPE_F32 0
#define HMX_DTYPE_BF16 1

/* Activations fused into an epilogue, applied to the f32 value before the
 * single rounding to the output dtype. */
#define HMX_EPI_IDENTITY 0
#define HMX_EPI_RELU 1
#define HMX_EPI_SILU 2
#define HMX_EPI_SIGMOID 3
#define HMX_EPI_GELU 4       /* erf form */
#define HMX_EPI_GELU_TANH 5  /* tanh approximation */
#define HMX_EPI_TANH 6
#define HMX_EPI_LEAKY_RELU 7 /* epilogue_arg = negative slope */
#define HMX_EPI_PROGRAM 8    /* the elementwise program `program` */

/*
 * Epilogue programs: an elementwise function of f32 values, for epilogues
 * that are not one of the activations above (the reference applies any
 * callable to the f32 accumulator, helion_mlir_utils/matmul.py:321-327, and
 * `epilogue(y, extra)` in group_norm, normalization.py:121). A program is a
 * straight-line list of at most HMX_PROGRAM_MAX instructions over
 * HMX_PROGRAM_REGS f32 registers. On entry register 0 holds the value (the
 * GEMM's `(acc + bias) * scale + shift`, group_norm's normalized value),
 * register 1 the extra operand (group_norm's per-channel `extra`, else 0) and
 * the others 0; each instruction writes `dst`; the result is register
 * `result`, rounded once to the output dtype. Every operation rounds to f32
 * as the same torch operation on f32 tensors does; max/min/clamp/relu keep
 * NaN.
 */
#define HMX_PROGRAM_MAX 16
#define HMX_PROGRAM_REGS 8

/* Opcodes: dst = f(a) | f(a, b) | f(a, c0[, c1]), registers a, b. */
#define HMX_OP_COPY 0
#define HMX_OP_NEG 1
#define HMX_OP_ABS 2
#define HMX_OP_RELU 3
#define HMX_OP_SIGMOID 4
#define HMX_OP_TANH 5
#define HMX_OP_SILU 6
#define HMX_OP_GELU 7         /* erf form */
#define HMX_OP_GELU_TANH 8
#define HMX_OP_EXP 9
#define HMX_OP_LOG 10
#define HMX_OP_SQRT 11
#define HMX_OP_RSQRT 12
#define HMX_OP_RECIP 13
#define HMX_OP_ERF 14
#define HMX_OP_SIN 15
#define HMX_OP_COS 16
#define HMX_OP_LOG1P 17
#define HMX_OP_EXPM1 18
#define HMX_OP_FLOOR 19
#define HMX_OP_CEIL 20
#define HMX_OP_TRUNC 21
#define HMX_OP_ROUND 22       /* half to even */
#define HMX_OP_SOFTPLUS 23    /* c0 = beta, c1 = threshold */
#define HMX_OP_MISH 24
#define HMX_OP_HARDSWISH 25
#define HMX_OP_HARDSIGMOID 26
#define HMX_OP_ELU 27         /* c0 = alpha, c1 = output scale (SELU: its scale) */
#define HMX_OP_LEAKY_RELU 28  /* c0 = negative slope */
#define HMX_OP_CLAMP 29       /* c0 = lower, c1 = upper bound (+-inf: none) */
#define HMX_OP_ADD_C 30       /* a + c0 */
#define HMX_OP_MUL_C 31       /* a * c0 */
#define HMX_OP_DIV_C 32       /* a / c0 */
#define HMX_OP_RSUB_C 33      /* c0 - a */
#define HMX_OP_RDIV_C 34      /* c0 / a */
#define HMX_OP_POW_C 35       /* a ** c0 */
#define HMX_OP_ADD 36         /* a + b */
#define HMX_OP_SUB 37         /* a - b */
#define HMX_OP_MUL 38         /* a * b */
#define HMX_OP_DIV 39         /* a / b */
#define HMX_OP_MAX 40         /* max(a, b) */
#define HMX_OP_MIN 41         /* min(a, b) */
#define HMX_OP_POW 42         /* a ** b */
#define HMX_OP_COUNT 43

typedef struct hmx_instr {
  uint8_t op, dst, a, b;
  float c0, c1;
} hmx_instr;

typedef struct hmx_program {
  int32_t count;  /* instructions, 1 .. HMX_PROGRAM_MAX */
  int32_t result; /* the register holding the result */
  hmx_instr code[HMX_PROGRAM_MAX];
} hmx_program;

/* Layouts of the GEMM's B operand (logical B is [K, N]).
 *   ROW           [K, N] row-major, row stride ldb
 *   TRANS         [N, K] row-major, row stride ldb (nn.Linear weights)
 *   VNNI_PANELS   [N_pad/P, K_pad/2, P, 2]   P = b_panel  (pack_b_vnni_t)
 *   BLOCKED_VNNI  [N_pad/32, K_pad/32, 16, 32, 2]        (pack_b_blocked_vnni)
 *   PANELS        [N_pad/P, K_pad, P]        P = b_panel  (bench pack_b_panels)
 *   BLOCKED       [N_pad/32, K_pad/32, 32, 32]            (pack_b_blocked)
 * For the packed layouts `ldb` is ignored and `b_kpad` is K_pad. */
#define HMX_B_ROW 0
#define HMX_B_TRANS 1
#define HMX_B_VNNI_PANELS 2
#define HMX_B_BLOCKED_VNNI 3
#define HMX_B_PANELS 4
#define HMX_B_BLOCKED 5

/* Group-norm epilogue operand use (the `extra` per-channel operand). */
#define HMX_EXTRA_NONE 0
#define HMX_EXTRA_ADD 1
#define HMX_EXTRA_MUL 2

/* Elementwise ops. */
#define HMX_ELT_RELU 0
#define HMX_ELT_LEAKY_RELU 1 /* arg = negative slope */
#define HMX_ELT_SCALE 2      /* arg = scalar factor */

/* Pack and pad kinds (hmx_pack). */
#define HMX_PACK_PAD 0              /* [R, C] -> [R_pad, C_pad]            (pad_2d, matmul.py:87-89) */
#define HMX_PACK_A_BLOCKED 1        /* [M, K] -> [M/32, K/32, 32, 32]      (matmul.py:92-99) */
#define HMX_PACK_A_BLOCKED_T 2      /* [K, M] -> [M/32, K/32, 32, 32]      (matmul.py:102-109) */
#define HMX_PACK_B_BLOCKED 3        /* [K, N] -> [N/32, K/32, 32, 32]      (matmul.py:112-119) */
#define HMX_PACK_B_BLOCKED_T 4      /* [N, K] -> [N/32, K/32, 32, 32]      (matmul.py:122-129) */
#define HMX_PACK_B_BLOCKED_VNNI 5   /* [K, N] -> [N/32, K/32, 16, 32, 2]   (matmul.py:132-140) */
#define HMX_PACK_B_BLOCKED_VNNI_T 6 /* [N, K] -> [N/32, K/32, 16, 32, 2]   (matmul.py:143-153) */
#define HMX_PACK_B_VNNI_PANELS_T 7  /* [N, K] -> [N/P, K/2, P, 2]          (matmul.py:972-983) */
#define HMX_PACK_B_PANELS 8         /* [K, N] -> [N/P, K, P]   (benchmarks/helion_block_pack.py:40-51) */
#define HMX_PACK_A_PANELS 9         /* [M, K] -> [K/P, M, P]   (benchmarks/helion_block_pack.py:54-62) */
#define HMX_PACK_TRANSPOSE 10       /* [R, C] -> [C_pad, R_pad] of the transpose (zero padded) */

/* The calling thread's last error message ("" if none). */
const char* hmx_last_error(void);

/* HMX_ABI_VERSION of the loaded library. */
int hmx_abi_version(void);

/* Checks that the current HIP device is a gfx950 (MI355X-class) GPU and
 * writes its compute-unit count. Stands in for the target check of
 * resolve_target (helion_mlir_backend/_compiler/targets/__init__.py:61-85). */
int hmx_device_check(int* compute_units);

/* Profiling hook; no counterpart in the reference (its kernels run on the
 * CPU, timed by callers with perf_counter). Arms hipEvent_t timing events for
 * the calling thread: the next kernel any entry point enqueues records
 * `start_event` when it begins, and every kernel enqueued while armed records
 * `stop_event` when it ends (hipExtLaunchKernelGGL), so the pair spans exactly
 * the kernels of the calls made in between, without host time. Armed
 * launches are dispatched later than plain ones: time throughput disarmed.
 * Both NULL disarms. The events must have been created with timing enabled
 * and belong to the device the calls run on. Per-thread state, like the
 * error message. */
int hmx_time_launches(void* start_event, void* stop_event);

/* Run-time compiled epilogues, as the reference reports its JIT's work
 * (helion_mlir_backend.explain(), _compiler/call_trace.py:220): kernels
 * compiled with an epilogue program or a named activation built in (the
 * 16x16x32 GEMM's register epilogue and group_norm's whole-row kernel;
 * hipRTC, on first use of each kernel variant and epilogue), the
 * compilations or launches that failed (those calls ran the prebuilt
 * kernels, and the variant is not tried again), and the launches of compiled
 * kernels. Any pointer may be NULL. HMX_JIT=0 in the environment turns
 * run-time compilation off (read on every call). */
int hmx_jit_info(int64_t* compiled, int64_t* failed, int64_t* launches);

/* The log of the last failed run-time compilation or launch ("" if none):
 * a copy per thread, valid until the same thread calls this again. */
const char* hmx_jit_last_log(void);

/*
 * GEMM with fused epilogue:
 *   C[b] = act(((op(A[b]) @ B[b]) + bias) * scale + shift)
 * op(A) is A [M, K] (lda) or, with trans_a, the transpose of A [K, M].
 * bias/scale/shift are [N] vectors of vec_dtype or NULL; accumulation is f32
 * and C (c_dtype) is rounded once. `act` is `epilogue` (HMX_EPI_*); with
 * HMX_EPI_PROGRAM it is `program` (otherwise `program` is ignored). ab_dtype is HMX_DTYPE_BF16 (MFMA bf16) or
 * HMX_DTYPE_F32 (MFMA f32). `batch` slices are strided by stride_a/b/c
 * elements. `splits` > 1 divides K into that many chunks whose f32 partials
 * ([splits, batch, M, N] in `workspace`) are summed in a fixed order by a
 * second kernel: results do not depend on timing. splits = 0 lets the
 * library choose (see hmx_gemm_plan), for the current device's CU count.
 * tile_m/tile_n/tile_k request a workgroup tile (0 = default): the largest
 * instantiated tile within the request is used. At most 64 rows of row-major
 * bf16 A against B [N, K] (batch 1, K a multiple of 64; a decode-shaped
 * linear layer) with splits 0 or 1 and no tile requested (or the skinny
 * kernel's own 32 x 32 x 64) take a skinny kernel: one workgroup per 32
 * columns of C, K split over its waves and summed in a fixed order, no
 * workspace (hmx_gemm_plan reports tile 32 x 32 x 64). The workspace also
 * takes a bf16 operand the library transposes once before the product (a
 * row-major B with ragged K, an A stored [K, M] of 512 or more rows, columns
 * and K); hmx_gemm_plan counts it. A row-major A or a B [N, K] spanning 2^31
 * bytes or more runs as one launch per block of whole tiles.
 * Stands in for matmul (helion_mlir_utils/matmul.py:1446-1570), its
 * fused-pack kernel (259-328), the f32 fused and blocked kernels (156-228,
 * 862-904, 1332-1368), split-K (1195-1300), bmm (1842-1882, 1965-2006) and the
 * prepacked-B kernels (534-627, 1593-1671, 1788-1839).
 */
int hmx_gemm(int ab_dtype, int c_dtype,
             const void* a, int64_t lda, int trans_a,
             const void* b, int64_t ldb, int b_layout, int64_t b_panel, int64_t b_kpad,
             void* c, int64_t ldc,
             int64_t m, int64_t n, int64_t k,
             int64_t batch, int64_t stride_a, int64_t stride_b, int64_t stride_c,
             const void* bias, const void* scale, const void* shift, int vec_dtype,
             int epilogue, float epilogue_arg, const hmx_program* program,
             int splits, void* workspace, int64_t workspace_bytes,
             int tile_m, int tile_n, int tile_k,
             void* stream);

/* Bytes of device memory hmx_gemm_noalloc keeps per device for its
 * workspace (64 MiB: config 5's 16 split-K partials of [16, 256, 256] f32). */
#define HMX_GEMM_SCRATCH_BYTES (64ll << 20)

/* hmx_gemm without a caller workspace and without allocating anything: the
 * split-K partials and a transposed A or B go to a workspace the library holds per
 * device (a static device array of HMX_GEMM_SCRATCH_BYTES, taken on each
 * device's first call and kept until the process ends). No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The arguments are hmx_gemm's. splits = 0 plans within the scratch; a
 * launch that needs more workspace than it holds (explicit splits) is
 * refused with HMX_ERR_INVALID. Calls on one device share its scratch, so
 * calls that overlap on one device (other streams, other threads) race:
 * order them on one stream. Results equal hmx_gemm's for the same plan. It
 * compiles and loads no kernel at run time: an epilogue whose compiled kernel
 * an earlier call made uses it, any other runs the prebuilt kernels. */
int hmx_gemm_noalloc(int ab_dtype, int c_dtype,
                     const void* a, int64_t lda, int trans_a,
                     const void* b, int64_t ldb, int b_layout, int64_t b_panel, int64_t b_kpad,
                     void* c, int64_t ldc,
                     int64_t m, int64_t n, int64_t k,
                     int64_t batch, int64_t stride_a, int64_t stride_b, int64_t stride_c,
                     const void* bias, const void* scale, const void* shift, int vec_dtype,
                     int epilogue, float epilogue_arg, const hmx_program* program,
                     int splits,
                     int tile_m, int tile_n, int tile_k,
                     void* stream);

/* The launch hmx_gemm would make for these arguments on a device of
 * `compute_units` CUs (0 = the current device's; MI355X's 256 when no device
 * is visible), without launching: the K splits (after `splits` = 0 is
 * resolved; `max_workspace_bytes` < 0 means unlimited), the workgroup tile
 * and the workspace bytes needed. `epilogue` is the launch's HMX_EPI_* code:
 * an epilogue program plans f32 partials even unsplit (kernels that do not
 * run programs fused leave them to the split-K reduction) and never the
 * skinny kernel. Host-only. Passing the result back to
 * hmx_gemm -- its splits, its tile as tile_m/n/k and a workspace of its size --
 * makes exactly the planned launch. Stands in for the tile heuristics
 * _fused_pack_tiles / _split_k (helion_mlir_utils/matmul.py:368-446, 1257-1287). */
int hmx_gemm_plan(int ab_dtype, int64_t m, int64_t n, int64_t k, int64_t batch,
                  int trans_a, int b_layout, int splits, int64_t max_workspace_bytes,
                  int tile_m, int tile_n, int tile_k, int compute_units, int epilogue,
                  int* out_splits, int* out_tile_m, int* out_tile_n, int* out_tile_k,
                  int64_t* out_workspace_bytes);

/* Row softmax over the last dim of contiguous [M, N], f32 internally,
 * `exp(x - max) * (1 / sum)` rounded once. x == y is allowed (in place).
 * Stands in for softmax (helion_mlir_utils/normalization.py:28-87, 138-153). */
int hmx_softmax_rows(int dtype, const void* x, void* y, int64_t m, int64_t n,
                     void* stream);

/* RMSNorm of contiguous [M, N] rows: y = x * rsqrt(mean(x^2) + eps) * w,
 * f32 internally, rounded once; w is [N] of w_dtype (NULL = no weight).
 * x == y is allowed. The reference has no RMSNorm entry point; this is the
 * new `rms_norm` beside group_norm (helion_mlir_utils/normalization.py:156-196). */
int hmx_rmsnorm_rows(int dtype, const void* x, const void* w, int w_dtype, void* y,
                     int64_t m, int64_t n, float eps, void* stream);

/* GroupNorm of contiguous [M, G * S] (S = group_size):
 *   y = act(extra_op((x - mean) * rsqrt(var + eps) * w + b, extra))
 * statistics per (row, group) in f32, centered variance; w, b, extra are
 * [G * S] of vec_dtype (b and extra may be NULL). G = 1 is LayerNorm.
 * With activation HMX_EPI_PROGRAM the whole epilogue is `program` instead:
 * y = program(normalized value, extra) (extra_op must be HMX_EXTRA_NONE; a
 * NULL extra reads 0). x == y is allowed. Stands in for group_norm
 * (helion_mlir_utils/normalization.py:94-123, 156-196). */
int hmx_group_norm_rows(int dtype, const void* x, const void* w, const void* b,
                        const void* extra, int vec_dtype, void* y,
                        int64_t m, int64_t groups, int64_t group_size, float eps,
                        int extra_op, int activation, float activation_arg,
                        const hmx_program* program, void* stream);

/* y[i] = act(sum_j x[i, j]) of contiguous [M, N], f32 accumulation, y [M] in
 * dtype. Stands in for row_sum (helion_mlir_utils/reduction.py:79-121). */
int hmx_row_sum(int dtype, const void* x, void* y, int64_t m, int64_t n,
                int activation, float activation_arg, const hmx_program* program,
                void* stream);

/* y[j] = sum_i x[i, j] of contiguous [M, N] into f32 y [N], in two passes
 * (row chunks into f32 partials in `workspace`, then the chunks added in
 * order, so results do not depend on timing). Stands in for column_sum
 * (helion_mlir_utils/reduction.py:124-163). */
int hmx_column_sum(int dtype, const void* x, float* y, int64_t m, int64_t n,
                   void* workspace, int64_t workspace_bytes, void* stream);

/* The workspace hmx_column_sum needs for [M, N] (0: none). Host-only. */
int hmx_column_sum_plan(int64_t m, int64_t n, int64_t* workspace_bytes);

/* y[i] = act(sum_j x[i, j] * v[j]), v f32 [N], y [M] in dtype. Stands in for
 * row_dot (helion_mlir_utils/reduction.py:166-212). */
int hmx_row_dot(int dtype, const void* x, const float* v, void* y, int64_t m,
                int64_t n, int activation, float activation_arg,
                const hmx_program* program, void* stream);

/* y = A @ x of contiguous A [M, K] and x [K] (both dtype), f32 accumulation,
 * y [M] in dtype. Stands in for matvec (helion_mlir_utils/reduction.py:24-67). */
int hmx_matvec(int dtype, const void* a, const void* x, void* y, int64_t m,
               int64_t k, void* stream);

/* Elementwise op over `numel` contiguous elements (y may equal x). Stands in
 * for relu / leaky_relu / scalar_mul (helion_mlir_utils/elementwise.py:14-56). */
int hmx_elementwise(int op, int dtype, const void* x, void* y, int64_t numel,
                    float arg, void* stream);

/* Layout conversion of a contiguous 2-D source [rows, cols] (row stride ld)
 * into the packed layout `kind`, zero-padded to rows_pad x cols_pad of the
 * logical matrix (for *_T kinds and TRANSPOSE the logical matrix is the
 * source's transpose). `panel` is the
 * panel width of the PANELS kinds. The pack kernels of
 * helion_mlir_utils/matmul.py:78-153, 972-983 and
 * benchmarks/helion_block_pack.py:40-62. */
int hmx_pack(int kind, int dtype, const void* src, int64_t rows, int64_t cols,
             int64_t ld, void* dst, int64_t rows_pad, int64_t cols_pad,
             int64_t panel, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HMX_H */

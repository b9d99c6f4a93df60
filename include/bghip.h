/*
 * bghip.h -- C ABI of the MI355X (gfx950) realizer library `libbghip.so`.
 *
 * This is the drop-in boundary that replaces browsergrad's WebGPU realizer
 * bridge.  Every entry point below corresponds to one method of the
 * reference's bridge interface
 *   - TypeScript: `WebGpuRealizerBridge`
 *       packages/browsergrad-kernels/src/realizer.ts:77-280 (interface)
 *       packages/browsergrad-kernels/src/realizer.ts:902-1683 (implementation)
 *   - Python:     `WebGpuBridge` Protocol
 *       packages/browsergrad-jit/src/python/_bridge.py:61-289
 * and is what the N-API addon (browsergrad_amd/node) and the Python ctypes
 * bridge (browsergrad_amd/bridge.py) bind.  Functions marked "extension"
 * have no reference counterpart; they are added additively (new functions,
 * never changed signatures), the same stability rule the reference states
 * for its bridge (packages/browsergrad-kernels/README.md:729).
 *
 * Conventions
 *   - Every function returns an int status (BG_OK == 0).  On failure the
 *     message is available from bg_last_error(ctx); the message is
 *     op-qualified the way the reference's KernelError is
 *     (packages/browsergrad-kernels/src/types.ts:87-92).
 *   - Handles are uint64 ids minted from 1 per context, never reused
 *     (realizer.ts:906-937).  0 is the null handle.
 *   - One context = one device + one HIP stream.  A context is not
 *     thread-shared ("never thread-shared", realizer.ts:894-897).
 *   - Device buffers are owned by the context.  bg_release is idempotent
 *     (realizer.ts:1036-1041).
 *   - Shapes are int64 arrays, row-major (C order); rank <= BG_MAX_RANK.
 *   - All compute entry points are asynchronous on the context stream;
 *     bg_materialize and bg_synchronize block.
 */
#ifndef BGHIP_H
#define BGHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BG_MAX_RANK 8
#define BG_FUSED_MAX_INPUTS 8   /* fused_elementwise.ts:97-103 */
#define BG_FUSED_MAX_OPS 32     /* fused_elementwise.ts:104-110 */
#define BG_FUSED_MAX_IMMS 16

typedef struct bg_ctx bg_ctx;
typedef uint64_t bg_handle;

/* Status codes. */
enum {
  BG_OK = 0,
  BG_E_INVALID = 1,     /* bad argument (shape, count, range)            */
  BG_E_HANDLE = 2,      /* unknown or released handle (realizer.ts:995)  */
  BG_E_DTYPE = 3,       /* dtype not supported by this op                */
  BG_E_SHAPE = 4,       /* shape mismatch between handles and arguments  */
  BG_E_OOM = 5,         /* hipErrorOutOfMemory                           */
  BG_E_HIP = 6,         /* any other HIP runtime error                   */
  BG_E_UNSUPPORTED = 7  /* op/configuration refused (JitNotImplemented)  */
};

/* Dtypes.  Names follow NumPy (_ir.py:348-353); "bfloat16" is an extension. */
enum {
  BG_F32 = 0,
  BG_F16 = 1,
  BG_BF16 = 2,
  BG_BOOL = 3,
  BG_I32 = 4,
  BG_I64 = 5,
  BG_U8 = 6,
  BG_F64 = 7
};

/* Fused-elementwise opcodes.  The first six are the reference's
 * FUSED_ELEMENTWISE inner opcodes (fused_elementwise.ts:83-90,
 * _realize.py:1557-1600); the rest are extensions used by bg_fused_ex. */
enum {
  BG_OP_ADD = 0,
  BG_OP_MUL = 1,
  BG_OP_DIV = 2,
  BG_OP_NEG = 3,
  BG_OP_EXP = 4,
  BG_OP_LOG = 5,
  /* extensions */
  BG_OP_MAX = 6,
  BG_OP_MIN = 7,
  BG_OP_CMP_EQ = 8,   /* results are 0.0 / 1.0 in registers, bool on store */
  BG_OP_CMP_NE = 9,
  BG_OP_CMP_LT = 10,
  BG_OP_CMP_LE = 11,
  BG_OP_CMP_GT = 12,
  BG_OP_CMP_GE = 13,
  BG_OP_WHERE = 14,   /* a ? b : c  (a != 0)                              */
  BG_OP_IMM = 15,     /* value = imms[a]                                 */
  BG_OP_ROUND_F16 = 16,  /* f32 -> nearest-even f16 -> f32 (CAST round trip) */
  BG_OP_ROUND_BF16 = 17, /* f32 -> nearest-even bf16 -> f32                 */
  BG_OP_SUB = 18,
  BG_OP_TANH = 19,
  BG_OP_SQRT = 20,
  BG_OP_RECIP = 21,
  BG_OP_ABS = 22,
  BG_OP_COPY = 23,
  BG_OP_COUNT_ = 24
};

/* Reduction epilogues for bg_fused_ex. */
enum {
  BG_RED_NONE = 0,
  BG_RED_SUM = 1,
  BG_RED_MAX = 2,
  BG_RED_MEAN = 3,
  BG_RED_MIN = 4
};

/* GEMM epilogue activations for bg_matmul_ex. */
enum {
  BG_ACT_NONE = 0,
  BG_ACT_RELU = 1,     /* where(y > 0, y, 0): the reference's relu (_functional.py:99-112) */
  BG_ACT_GELU_TANH = 2 /* reference tanh-GELU (_functional.py:123-134), f32 */
};

/* One fused step.  Refs: ref < 0 -> external input (-ref - 1);
 * ref >= 0 -> output of step `ref`.  `b`/`c` are ignored for unary ops;
 * for BG_OP_IMM `a` indexes the immediate table. */
typedef struct bg_fused_op {
  int32_t code;
  int32_t a;
  int32_t b;
  int32_t c;
} bg_fused_op;

/* Extension descriptor: broadcasting inputs + optional reduction over the
 * innermost `reduce_cols` elements of the iteration space. */
typedef struct bg_fused_desc {
  int32_t n_inputs;
  const bg_handle* inputs;
  /* Element strides of each input along each dim of `shape`
   * (n_inputs * rank, row-major by input).  0 = broadcast along that dim.
   * NULL means every input is contiguous with exactly `shape`. */
  const int64_t* in_strides;
  int32_t n_ops;
  const bg_fused_op* ops;
  int32_t n_imms;
  const double* imms;
  int32_t rank;
  const int64_t* shape;   /* iteration shape */
  int32_t out_dtype;      /* BG_F32 / BG_F16 / BG_BF16 / BG_BOOL */
  int32_t reduce_op;      /* BG_RED_* over the last dim of `shape` */
  int32_t reduce_keepdims;
} bg_fused_desc;

/* Extension descriptor for GEMM: C = epilogue(A @ op(B)).
 *   A: [batch][M][K] with row stride lda (elements) and batch stride sa.
 *   B: trans_b == 0 -> [batch][K][N] row-major (ldb >= N)
 *      trans_b == 1 -> [batch][N][K] row-major (ldb >= K), i.e. x @ W.T
 *   epilogue order (the order AMP realizes it, _amp.py:183-261,
 *   _realize.py:395-412):  acc(f32) -> [round to f16 if round_f16] ->
 *   [+ bias[n] (f32)] -> [activation] -> store out_dtype. */
typedef struct bg_matmul_desc {
  bg_handle a;
  bg_handle b;
  bg_handle bias;        /* 0 = none; f32 [N] */
  int64_t batch;
  int64_t m, n, k;
  int64_t lda, ldb, ldc;
  int64_t stride_a, stride_b, stride_c;  /* batch strides in elements (0 = broadcast) */
  int64_t offset_a, offset_b;            /* element offsets into a / b */
  int32_t trans_b;
  int32_t in_dtype;      /* BG_F32 (f32 MFMA) / BG_F16 / BG_BF16 */
  int32_t out_dtype;     /* BG_F32 / BG_F16 / BG_BF16 */
  int32_t round_f16;     /* round accumulator to the intermediate dtype before bias */
  int32_t act;           /* BG_ACT_* */
  int32_t reserved;
} bg_matmul_desc;

/* Extras for bg_matmul_ex2.  The epilogue is
 *   y = act([round](acc) + bias) + residual
 * evaluated in f32 in that order, which is the reference's autocast
 * `x + linear(h)` graph: MATMUL -> ADD(bias) -> [relu | GELU] -> ADD(x)
 * (_realize.py:395-412, _functional.py:99-134; residual streams of the
 * GPT-2 block).
 * residual: 0 = none; float32 holding batch*m*n elements, read as a dense
 *   [batch][m][n] block; the output must then be dense too.
 * a_dtype / b_dtype: the dtype a / b are stored in (-1 = in_dtype).  For a
 *   16-bit GEMM an operand stored as f32 (or the other 16-bit type) is
 *   rounded to in_dtype to nearest even in a pre-pass, which is the
 *   autocast CAST (_amp.py:56-69) fused into the call; a [K][N] B
 *   (trans_b = 0) is converted and re-laid out in the same pass.  Such an
 *   operand must be a dense matrix or batch of matrices.
 * reserved: must be 0. */
typedef struct bg_matmul_ext {
  bg_handle residual;
  int32_t a_dtype;
  int32_t b_dtype;
  int32_t reserved[4];
} bg_matmul_ext;

/* Extension descriptor for attention.  Q/K/V/O are addressed with explicit
 * element strides so head-split views (reshape+permute of a fused QKV
 * projection) need no copy.  Softmax and accumulation are f32, and P is
 * rounded to the input dtype before P@V.
 * round_scores != 0: the score matrix S = Q K^T is rounded to the input
 *   dtype before scaling, as the reference's autocast MATMUL output is
 *   (_realize.py:395-412); a kernel that rounds S exactly runs.
 * round_scores == 0: S stays in f32.  The fastest kernel may then fold the
 *   scale into Q (Q' = Q * scale * log2(e), one 16-bit rounding of Q'), and
 *   does so only where Q' cannot overflow (bf16, or scale * log2(e) <= 1). */
typedef struct bg_attention_desc {
  bg_handle q, k, v;
  int64_t batch, heads, sq, sk, d;
  int64_t q_off, k_off, v_off;
  int64_t q_sb, q_sh, q_ss;   /* strides: batch, head, seq (dim stride is 1) */
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;   /* output strides; 0,0,0 -> contiguous [B,H,S,D] */
  float scale;
  int32_t causal;
  int32_t in_dtype;     /* BG_F16 / BG_BF16 (MFMA) or BG_F32 */
  int32_t out_dtype;
  int32_t round_scores;
  int32_t reserved;
} bg_attention_desc;

/* Resource snapshot (realizer.ts:287-298 WebGpuResourceSnapshot). */
typedef struct bg_snapshot {
  int64_t current_owned_bytes;
  int64_t peak_owned_bytes;
  int64_t total_allocated_bytes;
  int64_t total_released_bytes;
  int64_t alive_handle_count;
  int64_t pending_profile_count;
  int64_t pass_profile_count;
  int64_t pool_cached_bytes;     /* extension: bytes parked in the block cache */
  int64_t pool_hits;             /* extension */
  int64_t pool_misses;           /* extension */
  int32_t timing_mode;           /* 0 unavailable, 1 hip-event (timestamp analogue) */
  int32_t timestamp_query_available;
} bg_snapshot;

/* One profiled dispatch (runner.ts:409-507 DirectDispatchProfile). */
typedef struct bg_pass_profile {
  char label[48];
  double gpu_ms;
  int64_t bytes;   /* algorithmic bytes of the dispatch */
  int64_t flops;   /* algorithmic flops of the dispatch */
} bg_pass_profile;

/* One kernel launch as the library issued it (extension; the launch log of
 * bg_set_launch_log).  kernel: the kernel symbol (mangled, truncated to
 * 159 bytes); grid / block: launch geometry; dynamic_lds: dynamic LDS bytes
 * of the launch; static_lds, vgprs (architected VGPRs per lane), scratch
 * (private bytes per lane) and max_threads: the kernel's compiled
 * attributes (hipFuncGetAttributes). */
typedef struct bg_launch_record {
  char kernel[160];
  int64_t grid[3];
  int32_t block[3];
  int64_t dynamic_lds;
  int64_t static_lds;
  int32_t vgprs;
  int32_t scratch;
  int32_t max_threads;
  int32_t reserved;
} bg_launch_record;

/* ---- context (createWebGpuRealizerBridge, realizer.ts:898-1005) ------- */
int bg_ctx_create(int device, int profiling, bg_ctx** out);
int bg_ctx_destroy(bg_ctx* ctx);
const char* bg_last_error(const bg_ctx* ctx);
int bg_dtype_from_name(const char* name);    /* -1 if unknown */
int64_t bg_dtype_size(int dtype);            /* bytes per element, -1 if unknown */
int bg_synchronize(bg_ctx* ctx);
const char* bg_version(void);

/* ---- buffer lifecycle ------------------------------------------------- */
/* upload: realizer.ts:1007-1021 */
int bg_upload(bg_ctx* ctx, const void* data, size_t nbytes,
              const int64_t* shape, int rank, int dtype, bg_handle* out);
/* materialize: realizer.ts:1023-1034 (blocking here; bindings wrap it as a
 * Promise).  nbytes must equal the handle's byte length. */
int bg_materialize(bg_ctx* ctx, bg_handle h, void* dst, size_t nbytes);
/* release: realizer.ts:1036-1041, idempotent */
int bg_release(bg_ctx* ctx, bg_handle h);
/* extension: metadata of a live handle */
int bg_handle_info(bg_ctx* ctx, bg_handle h, int64_t* shape_out, int* rank,
                   int* dtype, int64_t* nbytes);
/* aliveHandleCount: realizer.ts:275 */
int bg_alive_handles(bg_ctx* ctx, int64_t* out);
/* resourceSnapshot: realizer.ts:277, 287-298 */
int bg_resource_snapshot(bg_ctx* ctx, bg_snapshot* out);
/* flushProfiles: realizer.ts:1678-1681.  Waits for the stream, resolves all
 * pending event pairs, and copies up to `cap` profiles (oldest first). */
int bg_flush_profiles(bg_ctx* ctx, bg_pass_profile* out, int cap, int* n_out);
/* extension: switch per-dispatch profiling on or off between calls.  The
 * reference fixes it at creation (options.profiling, realizer.ts:899, 914);
 * profiles already recorded stay pending until bg_flush_profiles. */
int bg_set_profiling(bg_ctx* ctx, int on);
/* extension: record every kernel the library launches on this context
 * (on != 0) until switched off; bg_take_launch_log copies up to cap records
 * (oldest first) into out, sets *n_out to the number copied (or, with out
 * NULL, to the number pending) and clears what it copied.  Kernels compiled
 * at run time (fused programs) are launched as code objects and are not
 * recorded.  Used by the certified-numerics entry points to describe the
 * schedule that actually ran. */
int bg_set_launch_log(bg_ctx* ctx, int on);
int bg_take_launch_log(bg_ctx* ctx, bg_launch_record* out, int cap, int* n_out);

/* ---- compute ------------------------------------------------------------ */
/* matmul: realizer.ts:1043-1060.  A[M,K] @ B[K,N] row-major; dtype is
 * "float32" in the reference; float16/bfloat16 accepted (MFMA, f32 acc). */
int bg_matmul(bg_ctx* ctx, bg_handle a, bg_handle b, int64_t m, int64_t k,
              int64_t n, int dtype, bg_handle* out);
/* fused_elementwise: realizer.ts:1062-1085; ops use BG_OP_ADD..BG_OP_LOG */
int bg_fused_elementwise(bg_ctx* ctx, const bg_handle* inputs, int n_inputs,
                         const bg_fused_op* ops, int n_ops,
                         const int64_t* shape, int rank, int dtype,
                         bg_handle* out);
/* cast: realizer.ts:1087-1120 (reference: f32->f32 only).  Here every pair
 * of {f32, f16, bf16} with round-to-nearest-even narrowing. */
int bg_cast(bg_ctx* ctx, bg_handle h, int src_dtype, int dst_dtype,
            const int64_t* shape, int rank, bg_handle* out);
/* flash_attention: realizer.ts:1122-1151.  q,k,v [b,h,s,d]; mask (0 = none)
 * is an additive f32 mask broadcastable as [1|b,1|h,sq,sk]. */
int bg_flash_attention(bg_ctx* ctx, bg_handle q, bg_handle k, bg_handle v,
                       bg_handle mask, int64_t b, int64_t h, int64_t sq,
                       int64_t sk, int64_t d, float scale, int dtype,
                       bg_handle* out);

/* conv1d / conv2d and their backward kernels: realizer.ts:114-238
 * (interface), 1153-1521 (implementation).  f32 only (dtype must be BG_F32,
 * the reference's assertF32).  Layouts: input [n, c_in, l_in] or
 * [n, c_in, h, w]; weight [c_out, c_in/groups, k] or [c_out, c_in/groups,
 * kh, kw]; bias [c_out] or 0 for none; dy [n, c_out, l_out] or
 * [n, c_out, out_h, out_w].  The output sizes are taken as given (the
 * reference does not derive them): positions whose window lies outside the
 * padded input read zeros.  backward_input returns dx in the input's
 * layout, backward_weight dw in the weight's, backward_bias db [c_out]. */
int bg_conv1d(bg_ctx* ctx, bg_handle input, bg_handle weight, bg_handle bias,
              int64_t n, int64_t c_in, int64_t l_in, int64_t c_out, int64_t k,
              int64_t stride, int64_t padding, int64_t dilation,
              int64_t groups, int64_t l_out, int dtype, bg_handle* out);
int bg_conv1d_backward_input(bg_ctx* ctx, bg_handle dy, bg_handle weight,
                             int64_t n, int64_t c_in, int64_t l_in,
                             int64_t c_out, int64_t k, int64_t stride,
                             int64_t padding, int64_t dilation, int64_t groups,
                             int64_t l_out, int dtype, bg_handle* out);
int bg_conv1d_backward_weight(bg_ctx* ctx, bg_handle dy, bg_handle input,
                              int64_t n, int64_t c_in, int64_t l_in,
                              int64_t c_out, int64_t k, int64_t stride,
                              int64_t padding, int64_t dilation,
                              int64_t groups, int64_t l_out, int dtype,
                              bg_handle* out);
int bg_conv1d_backward_bias(bg_ctx* ctx, bg_handle dy, int64_t n,
                            int64_t c_out, int64_t l_out, int dtype,
                            bg_handle* out);
int bg_conv2d(bg_ctx* ctx, bg_handle input, bg_handle weight, bg_handle bias,
              int64_t n, int64_t c_in, int64_t h, int64_t w, int64_t c_out,
              int64_t kh, int64_t kw, int64_t stride_h, int64_t stride_w,
              int64_t pad_h, int64_t pad_w, int64_t dilation_h,
              int64_t dilation_w, int64_t groups, int64_t out_h,
              int64_t out_w, int dtype, bg_handle* out);
int bg_conv2d_backward_input(bg_ctx* ctx, bg_handle dy, bg_handle weight,
                             int64_t n, int64_t c_in, int64_t h, int64_t w,
                             int64_t c_out, int64_t kh, int64_t kw,
                             int64_t stride_h, int64_t stride_w, int64_t pad_h,
                             int64_t pad_w, int64_t dilation_h,
                             int64_t dilation_w, int64_t groups,
                             int64_t out_h, int64_t out_w, int dtype,
                             bg_handle* out);
int bg_conv2d_backward_weight(bg_ctx* ctx, bg_handle dy, bg_handle input,
                              int64_t n, int64_t c_in, int64_t h, int64_t w,
                              int64_t c_out, int64_t kh, int64_t kw,
                              int64_t stride_h, int64_t stride_w,
                              int64_t pad_h, int64_t pad_w,
                              int64_t dilation_h, int64_t dilation_w,
                              int64_t groups, int64_t out_h, int64_t out_w,
                              int dtype, bg_handle* out);
int bg_conv2d_backward_bias(bg_ctx* ctx, bg_handle dy, int64_t n,
                            int64_t c_out, int64_t out_h, int64_t out_w,
                            int dtype, bg_handle* out);

/* ---- extensions --------------------------------------------------------- */
int bg_matmul_ex(bg_ctx* ctx, const bg_matmul_desc* desc, bg_handle* out);
/* bg_matmul_ex with the extras of bg_matmul_ext (residual epilogue,
 * operands cast in a pre-pass).  Extends bridge.matmul
 * (realizer.ts:1043-1060) for the walker's fused linear + residual and
 * autocast-cast + linear patterns. */
int bg_matmul_ex2(bg_ctx* ctx, const bg_matmul_desc* desc, const bg_matmul_ext* ext, bg_handle* out);
/* No counterpart in the reference.  bg_matmul_ex for callers that cannot
 * allocate device memory (HIP graph capture, serving loops that forbid
 * hipMalloc): a, b, bias (f32 [N] or NULL) and c are caller-owned device
 * pointers (desc->a, ->b, ->bias must be 0; offset_a / offset_b, lda, ldb,
 * ldc, strides as in bg_matmul_ex, ldc / stride_c 0 = contiguous), the
 * caller sizes them (no extent check is possible), and the call allocates
 * nothing: no handle, no profiling event, and the kernels' scratch comes
 * from a fixed 16 MiB array per GPU held until the process ends.  Problems
 * that need more scratch (split-K partials of long-K f32 GEMMs, the
 * re-laid-out B of x @ w, the f32 product before a separate GELU pass) are
 * refused with BG_E_UNSUPPORTED before anything is launched.  The array is
 * shared by every call on one GPU: calls that overlap on one GPU (different
 * contexts or threads) race; calls on one context are stream ordered. */
int bg_matmul_noalloc(bg_ctx* ctx, const bg_matmul_desc* desc, const void* a, const void* b,
                      const float* bias, void* c);
int bg_fused_ex(bg_ctx* ctx, const bg_fused_desc* desc, bg_handle* out);
int bg_attention_ex(bg_ctx* ctx, const bg_attention_desc* desc, bg_handle* out);
/* LayerNorm over rows x cols (tensor_plan.ts:2170-2208; oracle
 * _realize.py:1008-1034).  x: f32/f16/bf16, weight/bias f32 [cols]. */
int bg_layer_norm(bg_ctx* ctx, bg_handle x, bg_handle weight, bg_handle bias,
                  int64_t rows, int64_t cols, float eps, int out_dtype,
                  bg_handle* out);
/* LayerNorm backward, f32 throughout (the tensor-plan ops
 * LAYER_NORM_BACKWARD_INPUT / _WEIGHT / _BIAS, tensor_plan.ts:2209-2321;
 * oracle _realize.py:1036-1072).  dy, x: [rows, cols]; weight: [cols].
 * input -> [rows, cols]; weight and bias -> [cols] (sums over rows). */
int bg_layer_norm_backward_input(bg_ctx* ctx, bg_handle dy, bg_handle x,
                                 bg_handle weight, int64_t rows, int64_t cols,
                                 float eps, bg_handle* out);
int bg_layer_norm_backward_weight(bg_ctx* ctx, bg_handle dy, bg_handle x,
                                  int64_t rows, int64_t cols, float eps,
                                  bg_handle* out);
int bg_layer_norm_backward_bias(bg_ctx* ctx, bg_handle dy, int64_t rows,
                                int64_t cols, bg_handle* out);
/* Optimizer updates, f32 elementwise over n elements (the tensor-plan ops
 * SGD_UPDATE, ADAMW_UPDATE_{M,V,PARAM}, ADAM_UPDATE_{M,V,PARAM},
 * tensor_plan.ts:2000-2168 with argument rules :648-702; oracle
 * _realize.py:1637-1721).  Inputs, in the reference's order:
 *   SGD          param, grad             param - lr*(grad + wd*param)
 *   ADAMW_M      m, grad                 b1*m + (1-b1)*grad
 *   ADAMW_V      v, grad                 b2*v + (1-b2)*grad^2
 *   ADAMW_PARAM  param, grad, m', v'     param - lr*mh/(sqrt(vh)+eps) - lr*wd*param
 *   ADAM_M       param, grad, m          b1*m + (1-b1)*(grad + wd*param)
 *   ADAM_V       param, grad, v          b2*v + (1-b2)*(grad + wd*param)^2
 *   ADAM_PARAM   param, m', v'           param - lr*mh/(sqrt(vh)+eps)
 * with mh = m'/(1-b1^step), vh = v'/(1-b2^step).  The output is a new
 * handle of n f32 elements.  (extension: the reference exposes these only
 * as plan steps; bg_run_tensor_plan lowers them onto this entry point.) */
enum {
  BG_OPT_SGD = 0,
  BG_OPT_ADAMW_M = 1,
  BG_OPT_ADAMW_V = 2,
  BG_OPT_ADAMW_PARAM = 3,
  BG_OPT_ADAM_M = 4,
  BG_OPT_ADAM_V = 5,
  BG_OPT_ADAM_PARAM = 6
};
typedef struct bg_optim_args {
  double lr;
  double beta1;
  double beta2;
  double eps;
  double weight_decay;
  int64_t step; /* >= 1 for the PARAM kinds */
} bg_optim_args;
int bg_optimizer_update(bg_ctx* ctx, int kind, const bg_handle* inputs,
                        int n_inputs, const bg_optim_args* args, int64_t n,
                        bg_handle* out);
/* Any convolution of the tensor-plan route (CONV1D*, CONV2D*, CONV3D*,
 * CONV_TRANSPOSE2D*, tensor_plan.ts:554-641; argument rules :3228-3775;
 * oracle _realize.py:413-1005) through one descriptor.  The first `spatial`
 * entries of each array are used, in (D,) H, W order.  Inputs by op:
 *   FORWARD          a = x [n, c_in, in...], b = weight, bias (0 = none)
 *   BACKWARD_INPUT   a = dy [n, c_out, out...], b = weight   -> [n, c_in, in...]
 *   BACKWARD_WEIGHT  a = dy, b = x                           -> weight layout
 *   BACKWARD_BIAS    a = dy                                  -> [c_out]
 * weight is [c_out, c_in/groups, k...], or [c_in, c_out/groups, k...] when
 * `transposed` (ConvTranspose: y[n, co, q] = sum x[n, ci, p] w[ci, co', kv]
 * over q = p*stride - pad + kv*dilation; output_pad only sizes the output,
 * which is given).  (extension) */
enum {
  BG_CONV_FORWARD = 0,
  BG_CONV_BACKWARD_INPUT = 1,
  BG_CONV_BACKWARD_WEIGHT = 2,
  BG_CONV_BACKWARD_BIAS = 3
};
typedef struct bg_conv_desc {
  int32_t op;
  int32_t transposed;
  int32_t spatial; /* 1, 2 or 3 */
  int32_t pad0;
  int64_t n, c_in, c_out, groups;
  int64_t in[3];  /* input spatial size */
  int64_t out[3]; /* output spatial size */
  int64_t k[3], stride[3], pad[3], dilation[3], output_pad[3];
  bg_handle a, b, bias;
} bg_conv_desc;
int bg_conv_ex(bg_ctx* ctx, const bg_conv_desc* desc, bg_handle* out);
/* Strided copy (PERMUTE / SLICE / BROADCAST materialisation,
 * tensor_plan.ts:824-997): out[i0..i{r-1}] = src[offset + sum(i_j*strides[j])]
 * in the dtype of src, shape `shape`. */
int bg_copy_strided(bg_ctx* ctx, bg_handle src, int64_t offset,
                    const int64_t* shape, const int64_t* strides, int rank,
                    bg_handle* out);
/* Reshape without copy: a new handle aliasing nothing -- the data is copied
 * device-to-device only when shapes differ in byte size (refused).  Used by
 * the walker for RESHAPE of an owned intermediate. */
int bg_reshape(bg_ctx* ctx, bg_handle h, const int64_t* shape, int rank,
               bg_handle* out);
/* Reduction over the last axis (REDUCE sum/max/mean/min, tensor_plan.ts:999-1115). */
int bg_reduce_last(bg_ctx* ctx, bg_handle x, int64_t rows, int64_t cols,
                   int op, int keepdims, bg_handle* out);
/* Last-axis softmax (FUSED_SOFTMAX; softmax.ts:102-119, tensor_plan.ts:
 * 573-586): rows x cols, x f32/f16/bf16, output out_dtype. */
int bg_softmax_last(bg_ctx* ctx, bg_handle x, int64_t rows, int64_t cols,
                    int out_dtype, bg_handle* out);
/* Plan executor (run_tensor_plan / run_tensor_plan_resident,
 * realizer.ts:1557-1620; tensor_plan.ts:183-373).  `plan_json` uses the
 * reference wire format (snake_case or camelCase).  `input_ids[i]` is a
 * plan value_id and `input_handles[i]` a live handle bound to it (the
 * bindings upload host bytes first).  When `dst` is non-NULL the root is
 * materialised into it (dst_nbytes must match) and released; otherwise
 * the root handle is returned in *root_out and stays resident (the root
 * must then be an allocation of its own, not a view of an input:
 * tensor_plan.ts:238-266). */
int bg_run_tensor_plan(bg_ctx* ctx, const char* plan_json,
                       const int64_t* input_ids, const bg_handle* input_handles,
                       int n_inputs, int dtype, void* dst, size_t dst_nbytes,
                       bg_handle* root_out);
/* Semantic route (run_tensor_plan_semantic / _resident_semantic,
 * realizer.ts:1588-1652; tensor_plan_semantics.ts:96-260): as above, with the
 * PERMUTE meaning taken from `requests_json`, the versioned
 * dense-permutation-view-copy side table, which must match the plan's
 * PERMUTE steps one to one (their legacy `arg` erased to null). */
int bg_run_tensor_plan_semantic(bg_ctx* ctx, const char* plan_json,
                                const char* requests_json,
                                const int64_t* input_ids,
                                const bg_handle* input_handles, int n_inputs,
                                int dtype, void* dst, size_t dst_nbytes,
                                bg_handle* root_out);

/* Device-free plan check (extension; no context, no GPU): parses and
 * validates `plan_json` (and `requests_json` when non-NULL) exactly as
 * bg_run_tensor_plan does, applies the plan-level fusion, and writes into
 * `out` (capacity out_cap, always NUL-terminated) a JSON summary of the steps
 * the executor would run ({"steps":[{"value_id","op","inputs",...}],
 * "root_id"}), or the refusal message when the status is not BG_OK.
 * *needed (when non-NULL) receives the full length + 1. */
int bg_plan_inspect(const char* plan_json, const char* requests_json, char* out, size_t out_cap,
                    size_t* needed);

/* Launch plan of one call, computed on the host before anything runs
 * (extension; no context, no GPU): the kernels the call will launch, in
 * order, with their template arguments, grids and workgroup sizes.  It backs
 * the prepare step of the verified-artifact APIs, which fix a schedule before
 * execution and check the run against it (prepareSemanticGemmWgsl,
 * packages/browsergrad-kernels/src/semantic_gemm.ts:194-340;
 * prepareSemanticAttentionWgsl, semantic_attention.ts:245-413).  Operands
 * are taken to start at their descriptor offsets inside allocations made by
 * this library (256-byte aligned), as the semantic runs upload them.
 * Covered: float32 GEMMs without GELU (bg_matmul_launch_plan) and float32
 * attention with head dim 1..64 (bg_attention_launch_plan); anything else
 * returns BG_E_UNSUPPORTED. */
#define BG_PLAN_MAX_LAUNCHES 4
typedef struct bg_launch_plan_entry {
  char family[48];        /* kernel function name, without namespace or template arguments */
  int32_t n_targs;
  int32_t targs[8];       /* integer / bool template arguments in declaration order */
  int32_t block[3];
  int64_t grid[3];
} bg_launch_plan_entry;
typedef struct bg_launch_plan {
  int32_t n_launches;
  int32_t tile_m, tile_n, tile_k;  /* GEMM: output tile and k step; attention: queries per
                                      workgroup, keys per tile, padded head dim */
  int32_t k_slices;                /* GEMM split-K slices (1 = none) */
  int32_t reserved;
  int64_t lds_bytes;               /* LDS per workgroup of the main kernel */
  int64_t workspace_bytes;         /* context scratch the call takes */
  bg_launch_plan_entry launch[BG_PLAN_MAX_LAUNCHES];
} bg_launch_plan;
/* A refusal's message goes to err (capacity err_cap, NUL-terminated; may be NULL). */
int bg_matmul_launch_plan(const bg_matmul_desc* desc, bg_launch_plan* out, char* err, size_t err_cap);
int bg_attention_launch_plan(const bg_attention_desc* desc, bg_launch_plan* out, char* err, size_t err_cap);

/* Raw device pointer of a handle (extension; for harnesses that time
 * kernels with their own events).  Valid until the handle is released. */
int bg_device_ptr(bg_ctx* ctx, bg_handle h, void** ptr);
/* The HIP stream of the context (hipStream_t as void*). */
int bg_stream(bg_ctx* ctx, void** stream);

#ifdef __cplusplus
}
#endif

#endif /* BGHIP_H */

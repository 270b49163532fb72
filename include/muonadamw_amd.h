/*
 * muonadamw_amd.h -- C ABI of the MI355X (gfx950) MuonAdamW step.
 *
 * This is the boundary between a host layer (the Python drop-in package, or any
 * other language over its FFI) and the hand-written HIP kernels.  Signatures use
 * plain pointers, sizes and scalars only.  All device memory is owned by the
 * caller: the library never allocates device memory.  Every entry point is
 * stateless and re-entrant; ordering between calls comes only from the stream.
 *
 * Status convention (every int-returning entry point):
 *     0            success
 *     negative     invalid argument, detected on the host before any HIP call
 *     positive     a hipError_t returned by the HIP runtime, passed through
 * mamw_strerror() turns either kind into text.
 *
 * Element types: fp32 is `float`; bf16 buffers are passed as `uint16_t*`
 * holding the IEEE bfloat16 bit pattern.
 *
 * Reference interfaces replaced (reference = "MuonAdamW package/triton_muon_adamw/"):
 *   adamw/triton_adam.py:66-103   solve_adamw_step          -> mamw_adamw_tensor_step
 *   adamw/triton_adam.py:132-153  TritonAdamW.step loop     -> mamw_adamw_table_* + mamw_adamw_mt_step
 *   muon/triton_muon.py:95-117    solve_ns_kernel_1         -> mamw_ns_gram
 *   muon/triton_muon.py:191-212   solve_ns_kernel_2         -> mamw_ns_poly
 *   muon/triton_muon.py:281-310   solve_ns_kernel_3         -> mamw_ns_update
 *   muon/triton_muon.py:327-372   muon_step (+ :414-448 loop) -> mamw_muon_workspace_bytes + mamw_muon_step
 */
#ifndef MUONADAMW_AMD_H
#define MUONADAMW_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MAMW_ABI_VERSION 5

/* ---- status codes -------------------------------------------------------- */
#define MAMW_OK             0
#define MAMW_ERR_NULL      -1 /* a required pointer is NULL                          */
#define MAMW_ERR_COUNT     -2 /* tensor / matrix count out of range                  */
#define MAMW_ERR_NUMEL     -3 /* element count negative or beyond the supported size */
#define MAMW_ERR_SHAPE     -4 /* rows/cols non-positive or mixed within one call     */
#define MAMW_ERR_ALIGN     -5 /* pointer misaligned for its element type             */
#define MAMW_ERR_WORKSPACE -6 /* workspace NULL, misaligned or too small             */
#define MAMW_ERR_HYPER     -7 /* hyper-parameter out of range (ns_steps, ...)        */
#define MAMW_ERR_TABLE     -8 /* host table buffer too small                         */
#define MAMW_ERR_ALIAS     -9 /* buffers that must be distinct overlap               */
#define MAMW_ERR_SCRATCH  -10 /* step needs more than MAMW_NOALLOC_SCRATCH_BYTES     */

/* A hipStream_t.  NULL selects the null stream. */
typedef void* mamw_stream_t;

/* ABI version compiled into the library (MAMW_ABI_VERSION). */
int mamw_abi_version(void);

/* Static description of a status code; never NULL. */
const char* mamw_strerror(int status);

/* ==== AdamW ================================================================ *
 * Per element (fp32, no fused multiply-add), following triton_adam.py:53-59:
 *     m     = beta1*m + (1-beta1)*g
 *     v     = beta2*v + (1-beta2)*(g*g)
 *     p     = (1 - lr*weight_decay)*p - lr*((m/bias1) / (sqrt(v/bias2) + eps))
 * with bias1 = 1-beta1^t, bias2 = 1-beta2^t computed by the caller (the
 * reference computes them on the host in float64, triton_adam.py:147-148).
 * param, exp_avg and exp_avg_sq are updated in place; grad is only read.       */

typedef struct mamw_adamw_tensor {
    float*       param;      /* numel fp32, contiguous */
    const float* grad;       /* numel fp32, contiguous */
    float*       exp_avg;    /* numel fp32, contiguous */
    float*       exp_avg_sq; /* numel fp32, contiguous */
    int64_t      numel;      /* >= 0; 0 is a no-op      */
} mamw_adamw_tensor;

/* Element-type flags of a tensor (mamw_adamw_tensor_ex.flags) or matrix
 * (mamw_muon_matrix.flags).  Optimizer state (exp_avg, exp_avg_sq, momentum)
 * is fp32 in every case; the update is computed in fp32 and a bf16 parameter is
 * written back rounded to nearest-even.                                         */
#define MAMW_BF16_PARAM 0x1 /* param holds bf16 (uint16_t bit patterns) */
#define MAMW_BF16_GRAD  0x2 /* grad holds bf16                           */

/* A tensor of any element-type combination.  No counterpart in the reference
 * (whose kernels take the parameter's dtype for every buffer,
 * triton_adam.py:79-85,129-130): bf16 parameters and/or gradients with fp32
 * moments.                                                                    */
typedef struct mamw_adamw_tensor_ex {
    void*        param;      /* numel fp32, or bf16 with MAMW_BF16_PARAM */
    const void*  grad;       /* numel fp32, or bf16 with MAMW_BF16_GRAD  */
    float*       exp_avg;    /* numel fp32                                */
    float*       exp_avg_sq; /* numel fp32                                */
    int64_t      numel;      /* >= 0; 0 is a no-op                        */
    int32_t      flags;      /* MAMW_BF16_* bits; other bits rejected     */
    int32_t      reserved;   /* must be 0                                 */
} mamw_adamw_tensor_ex;

/* One tensor, one launch.  Replaces solve_adamw_step (triton_adam.py:66-103),
 * which views 1-D tensors as (1,N) and launches a (M, cdiv(N,512)) grid. */
int mamw_adamw_tensor_step(float* param, const float* grad, float* exp_avg,
                           float* exp_avg_sq, int64_t numel, float lr,
                           float bias1, float bias2, float beta1, float beta2,
                           float weight_decay, float eps, mamw_stream_t stream);

/* Multi-tensor AdamW: every tensor of a step in ONE launch.  Replaces the
 * per-parameter launch loop of TritonAdamW.step (triton_adam.py:132-153).
 *
 * 1. mamw_adamw_table_bytes: size of the packed table for n_tensors (one
 *    64-byte record per tensor plus one that mamw_adamw_mt_step_amp writes).
 * 2. mamw_adamw_table_pack (host only, no HIP call): validates the tensors and
 *    packs the table into host memory; returns the launch's block count.
 *    Memory one tensor writes (param, exp_avg, exp_avg_sq) overlapping memory
 *    any tensor of the table reads or writes is MAMW_ERR_ALIAS (the launch
 *    updates them all at once), a parameter listed twice included: split such
 *    a list over several tables, one launch each, for updates in sequence.
 * 3. The caller copies the table to device memory (16-byte aligned) and keeps
 *    it there while the pointers stay the same.
 * 4. mamw_adamw_mt_step: launches the update over every packed tensor.        */
int mamw_adamw_table_bytes(int n_tensors, size_t* bytes);
int mamw_adamw_table_pack(const mamw_adamw_tensor* tensors, int n_tensors,
                          void* host_table, size_t table_bytes,
                          int64_t* n_blocks);
/* mamw_adamw_table_pack for mamw_adamw_tensor_ex entries (same table format,
 * same mamw_adamw_mt_step); bf16 buffers need 2-byte alignment.               */
int mamw_adamw_table_pack_ex(const mamw_adamw_tensor_ex* tensors, int n_tensors,
                             void* host_table, size_t table_bytes,
                             int64_t* n_blocks);
int mamw_adamw_mt_step(const void* device_table, int n_tensors,
                       int64_t n_blocks, float lr, float bias1, float bias2,
                       float beta1, float beta2, float weight_decay, float eps,
                       mamw_stream_t stream);

/* mamw_adamw_mt_step for a gradient-scaler step, with the scaler's tensors
 * left on the device (no host synchronisation): the fused AdamW path of
 * torch/optim/adam.py:865-899 driven by torch/amp/grad_scaler.py:403-448
 * (the reference has no mixed-precision path).
 *   step:       device fp32 step counter, already incremented for this step;
 *               the bias corrections are 1 - beta^step, formed on the device
 *               in double from the double betas and rounded to fp32, as the
 *               host forms them for mamw_adamw_mt_step, by a one-wave kernel
 *               launched first that stores them in the table's trailing
 *               record (so calls sharing one table must not overlap).
 *               Required.
 *   grad_scale: device fp32; every gradient is divided by it.  NULL: none.
 *   found_inf:  device fp32; non-zero skips the update (parameters and
 *               moments untouched).  NULL: never skipped.
 * The caller decrements *step by *found_inf afterwards, as torch does.
 * device_table must be writable device memory (the trailing record is
 * written); every argument is validated, n_blocks included, before the first
 * launch.                                                                   */
int mamw_adamw_mt_step_amp(void* device_table, int n_tensors,
                           int64_t n_blocks, float lr, double beta1,
                           double beta2, float weight_decay, float eps,
                           const float* step, const float* grad_scale,
                           const float* found_inf, mamw_stream_t stream);

/* ==== Muon ================================================================= *
 * One Muon update of up to MAMW_MUON_MAX_BATCH matrices that share
 * {min(rows,cols), max(rows,cols)} (wide and tall may be mixed), following
 * torch/optim/_muon.py:304-318 as wrapped by PyTorchMuonAdamW
 * (optimizer.py:228-241) and re-implemented by muon_step (triton_muon.py:327-372):
 *     momentum = lerp(momentum, grad, 1-beta)                   (fp32)
 *     u        = nesterov ? lerp(grad, momentum, beta) : momentum
 *     X        = bf16(u), transposed when rows > cols            (m x n, m <= n)
 *     X        = X / max(||X||_F, eps)                           (bf16)
 *     repeat ns_steps:  A = X Xt;  B = b A + c A A;  X = a X + B X   (bf16, fp32 accumulate)
 *     param    = param*(1 - lr*weight_decay) - scaled_lr * X(transposed back)
 * The workspace (device memory, 256-byte aligned, at least
 * mamw_muon_workspace_bytes) holds the bf16 iterates; its contents need not be
 * initialised and are garbage afterwards.                                       */

#define MAMW_MUON_MAX_BATCH 32

typedef struct mamw_muon_matrix {
    float*       param;     /* rows x cols fp32, row-major, contiguous
                               (bf16 with MAMW_BF16_PARAM)             */
    const float* grad;      /* rows x cols fp32 (bf16 with MAMW_BF16_GRAD) */
    float*       momentum;  /* rows x cols fp32                        */
    float*       update;    /* optional (NULL = skip): receives the orthogonalised
                               update (rows x cols fp32, bf16-valued), the `out`
                               buffer of muon_step (triton_muon.py:341,368)      */
    int64_t      rows;
    int64_t      cols;
    float        scaled_lr; /* lr * adjust_lr(rows, cols)              */
    int32_t      flags;     /* MAMW_BF16_* bits (0: fp32 param and grad);
                               other bits rejected                      */
} mamw_muon_matrix;

int mamw_muon_workspace_bytes(int batch, int64_t rows, int64_t cols,
                              int ns_steps, size_t* bytes);

/* lr, weight_decay and beta are doubles because torch forms the derived
 * scalars in double before rounding them to fp32: the lerp weights 1-beta and
 * beta (_muon.py:310-311) and the decay factor 1 - lr*weight_decay (:317).   */
int mamw_muon_step(const mamw_muon_matrix* mats, int batch, double lr,
                   double weight_decay, double beta, int nesterov, float a,
                   float b, float c, int ns_steps, float eps, void* workspace,
                   size_t workspace_bytes, mamw_stream_t stream);

/* mamw_muon_step without a caller workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  No counterpart in the reference (its
 * launchers allocate scratch from torch per call, triton_muon.py:320-321,
 * 358-359,422).  The workspace is a file-scope device array of
 * MAMW_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, held from the
 * library's load until the process ends; its device address is resolved once
 * per device on the first call there.  The call allocates nothing (no
 * hipMalloc/hipFree, and no profiler events even while profiling is on).
 * Limits and sharing:
 *   - a batch whose mamw_muon_workspace_bytes exceeds the array is rejected
 *     with MAMW_ERR_SCRATCH (one 4096 x 14336 matrix needs 288 MiB; what
 *     fits: 1 of 4096 x 4096, 12 of 1024 x 4096, 22 of 768 x 3072, 28 of
 *     768 x 2304, 32 of 768 x 768);
 *   - every call on one GPU uses that GPU's one array, which keeps the last
 *     call's contents (nothing in it needs to start at zero: each step writes
 *     every workspace byte it reads first), so calls that overlap in time on
 *     one GPU race: issue them on one stream, or order them with events.
 * Arguments, validation and results are those of mamw_muon_step.            */
#define MAMW_NOALLOC_SCRATCH_BYTES (256u << 20) /* 256 MiB per GPU */
int mamw_muon_step_noalloc(const mamw_muon_matrix* mats, int batch, double lr,
                           double weight_decay, double beta, int nesterov,
                           float a, float b, float c, int ns_steps, float eps,
                           mamw_stream_t stream);

/* mamw_muon_step for a gradient-scaler step (torch/amp/grad_scaler.py:403-448;
 * the reference has no mixed-precision path): gradients are divided by the
 * device fp32 *grad_scale (NULL: not scaled); a non-zero device fp32
 * *found_inf (NULL: never) leaves the momentum, the parameters and the update
 * buffers untouched, with no host synchronisation.                         */
int mamw_muon_step_amp(const mamw_muon_matrix* mats, int batch, double lr,
                       double weight_decay, double beta, int nesterov, float a,
                       float b, float c, int ns_steps, float eps,
                       void* workspace, size_t workspace_bytes,
                       const float* grad_scale, const float* found_inf,
                       mamw_stream_t stream);

/* ==== Newton-Schulz building blocks (batched, bf16, fp32 accumulate) ======== *
 * Operate on `batch` contiguous zero-padded row-major matrices.  m and n must
 * be multiples of 128 and k a multiple of 64; the Python mirrors pad.  An
 * output whose byte range (over the whole batch) overlaps a buffer the same
 * call reads, or the other output, is rejected with MAMW_ERR_ALIAS.            */

/* A = X X^T  (X: m x k, A: m x m).  Replaces solve_ns_kernel_1
 * (triton_muon.py:95-117).  Only tiles on or above the diagonal are computed;
 * each is written to both triangles, so A is exactly symmetric.               */
int mamw_ns_gram(const uint16_t* X, uint16_t* A, int batch, int64_t m,
                 int64_t k, mamw_stream_t stream);

/* B = b A + c A A for symmetric A (m x m).  Replaces solve_ns_kernel_2
 * (triton_muon.py:191-212).  B is exactly symmetric.                          */
int mamw_ns_poly(const uint16_t* A, uint16_t* B, int batch, int64_t m,
                 float b, float c, mamw_stream_t stream);

/* out = a X + B X  (B: m x m symmetric, X: m x n).  Replaces solve_ns_kernel_3
 * (triton_muon.py:281-310).  XT must hold X^T (n x m); X itself is not read
 * (out may equal X); out must not overlap B or XT; out_t, if not NULL,
 * receives out^T (n x m) and must not overlap B, XT or out.                   */
int mamw_ns_update(const uint16_t* B, const uint16_t* X, const uint16_t* XT,
                   uint16_t* out, uint16_t* out_t, int batch, int64_t m,
                   int64_t n, float a, mamw_stream_t stream);

/* dst = src^T for `batch` bf16 matrices (src rows x cols, dst cols x rows);
 * src and dst must not overlap.                                              */
int mamw_transpose_bf16(const uint16_t* src, uint16_t* dst, int batch,
                        int64_t rows, int64_t cols, mamw_stream_t stream);

/* ==== Profiling (opt-in) ==================================================== *
 * Between mamw_prof_start() and mamw_prof_stop(), every kernel launched by the
 * library is timed with a pair of HIP events bound to its dispatch.
 * mamw_prof_collect() waits for those events and returns one record per launch
 * (in launch order), then forgets them; with capacity < count it returns
 * MAMW_ERR_TABLE, sets *count and keeps the records.  Not meant for code that
 * runs under HIP graph capture.                                               */
typedef struct mamw_prof_record {
    int32_t kernel;  /* see mamw_prof_kernel_name                                  */
    int32_t variant; /* GEMMs: 8*tile + 4*(A lower-triangle) + 2*(k-major) + (k-blocked) */
    double  flops;   /* algorithmic floating-point operations of the launch (0: n/a) */
    double  bytes;   /* algorithmic HBM bytes of the launch (0: not known here)      */
    float   ms;      /* dispatch duration                                            */
    int32_t pad;
} mamw_prof_record;

int mamw_prof_start(void);
int mamw_prof_stop(void);
int mamw_prof_collect(mamw_prof_record* out, int capacity, int* count);
const char* mamw_prof_kernel_name(int kernel);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* MUONADAMW_AMD_H */

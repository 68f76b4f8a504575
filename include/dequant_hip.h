/*
 * dequant_hip.h -- C ABI of the MI355X (gfx950) fused dequant + GEMV engine.
 *
 * This is the drop-in boundary for the decode path of the reference project
 * (KrishnaI2424/Dequant_Project). The reference binds three C++ launchers into
 * the pybind11 module `dequant_cuda`:
 *
 *   add_one(x)                                   kernels/dequant_cuda.h:10,  kernels/smoke.cu:15-25
 *   gemv(x, qweight, scales, zeros, bits,
 *        group_size, symmetric, interleaved)     kernels/dequant_cuda.h:13-15, kernels/dequant_gemv.cu:339-386
 *   dequantize(qweight, scales, zeros, bits,
 *              group_size, symmetric,
 *              interleaved, K)                   kernels/dequant_cuda.h:18-20, kernels/dequant_gemv.cu:310-337
 *   (module definition: kernels/bindings.cpp:5-17)
 *
 * Each is replaced below by an `extern "C"` entry point over plain device
 * pointers and sizes. No torch types cross this boundary; a torch extension,
 * ctypes, cgo or any other FFI can bind it. Nothing here allocates device
 * memory: the caller owns every buffer, as the reference's callers own the
 * tensors they pass (and the torch layer allocates the outputs, as the
 * reference's launchers do with torch::empty).
 *
 * Packed format (frozen; defined by the reference's dequant/packer.py:1-201):
 *   - a weight is [N, K]; the GEMV reduces over K; groups run along K;
 *   - qweight is [N, K / (32/bits)] 32-bit words (torch int32 holding the
 *     uint32 bit pattern, packer.py:159-161);
 *   - codes are unsigned; symmetric codes are pre-biased by 2^(bits-1);
 *   - "sequential": logical code i of a word sits at bit offset bits*i;
 *     "interleaved": slot s holds logical code T[s] with
 *        T4 = {0,2,4,6,1,3,5,7}, T2 = {0,4,8,12,1,5,9,13,2,6,10,14,3,7,11,15},
 *        T8 = {0,2,1,3}                               (packer.py:37-41);
 *   - scales (and zeros when asymmetric) are fp16 [N, K / group_size];
 *     per-channel quantization is passed as group_size == K
 *     (dequant/quant_linear.py:79).
 *
 * fp16 values travel as uint16_t bit patterns.
 *
 * Errors: every entry point returns DQ_OK (0) or a DQ_ERR_* status and
 * records a message (the reference's TORCH_CHECK text, e.g.
 * "gemv handles 1 <= M <= 8, got M=9; use the dequantize + F.linear fallback")
 * retrievable with dq_last_error() on the calling thread. Launch errors from
 * the HIP runtime come back as DQ_ERR_LAUNCH. Device-side faults surface
 * asynchronously, as with any HIP launch.
 *
 * Streams: every launch is asynchronous on `stream` (NULL = the legacy default
 * stream). No entry point synchronizes, allocates or reads device memory on
 * the host, so all of them may be captured into a HIP graph.
 */
#ifndef DEQUANT_HIP_H_
#define DEQUANT_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same type as hipStream_t (hip_runtime_api.h: typedef struct ihipStream_t* hipStream_t). */
typedef struct ihipStream_t* dq_stream_t;

enum dq_status {
  DQ_OK = 0,
  DQ_ERR_INVALID_ARGUMENT = 1, /* violates the packed format or the call contract */
  DQ_ERR_UNSUPPORTED = 2,      /* well-formed, but outside what the entry point handles (M > 8) */
  DQ_ERR_LAUNCH = 3,           /* the HIP runtime rejected a launch */
  DQ_ERR_HIP = 4               /* another HIP runtime call failed */
};

/* Largest batch (rows of x) the fused GEMV handles; kernels/dequant_gemv.cu:27
 * and dequant/quant_linear.py:39 (MAX_M = 8). */
#define DQ_MAX_M 8

/* Message describing the last non-OK status returned on this thread
 * (empty string if none). Valid until the next call on this thread. */
const char* dq_last_error(void);

/* Short name of a status code ("DQ_OK", "DQ_ERR_INVALID_ARGUMENT", ...). */
const char* dq_status_name(int status);

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int dq_version(void);

/* ---------------------------------------------------------------- tensors
 * Host-side description of one operand, used by dq_check_* to run the
 * reference's argument validation (kernels/dequant_gemv.cu:230-283, 310-317,
 * 342-361) in the reference's order and with the reference's messages. A
 * binding fills one per tensor; the checks read no device memory and make no
 * HIP call, so they run on machines without a GPU.
 */
enum dq_dtype { DQ_DTYPE_OTHER = 0, DQ_DTYPE_INT32 = 1, DQ_DTYPE_FLOAT16 = 2, DQ_DTYPE_FLOAT32 = 3 };

typedef struct dq_tensor {
  const void* data;   /* first element */
  int32_t is_device;  /* 1 if the memory is GPU memory ("a CUDA tensor" in torch terms) */
  int32_t device;     /* device ordinal when is_device */
  int32_t dtype;      /* enum dq_dtype */
  int32_t contiguous; /* 1 if row-major dense */
  int32_t ndim;
  int64_t sizes[4];   /* sizes[0..ndim-1] */
} dq_tensor;

/* Validation of dequant_cuda.gemv(x, qweight, scales, zeros, bits, group_size,
 * symmetric, interleaved): kernels/dequant_gemv.cu:342-361 then check_weight
 * :230-283. `zeros` may be NULL (= None). */
int dq_check_gemv(const dq_tensor* x, const dq_tensor* qweight, const dq_tensor* scales,
                  const dq_tensor* zeros, int64_t bits, int64_t group_size, int symmetric);

/* Validation of dequant_cuda.gemm_small(x, qweight, scales, zeros, bits,
 * group_size, symmetric, interleaved): the rules of dq_check_gemv with
 * 1 <= M <= DQ_MAX_GEMM_M (no reference counterpart; see dq_gemm_small). */
int dq_check_gemm_small(const dq_tensor* x, const dq_tensor* qweight, const dq_tensor* scales,
                        const dq_tensor* zeros, int64_t bits, int64_t group_size, int symmetric);

/* Validation of dequant_cuda.dequantize(..., K): kernels/dequant_gemv.cu:310-317
 * with check_weight :230-283. */
int dq_check_dequantize(const dq_tensor* qweight, const dq_tensor* scales, const dq_tensor* zeros,
                        int64_t bits, int64_t group_size, int symmetric, int64_t K);

/* Validation of dq_unpack's arguments (no reference counterpart; it applies
 * the qweight rules of check_weight, kernels/dequant_gemv.cu:233-246). */
int dq_check_unpack(const dq_tensor* qweight, int64_t bits, int64_t K);

/* ---------------------------------------------------------------- compute */

/* y[M, N] = fp16_rn( x[M, K] @ W^T ), W held packed; fp32 accumulation.
 * Replaces dequant_cuda.gemv (kernels/dequant_gemv.cu:339-386, kernel :144-217).
 *   x        fp16 [M, K], row-major, 16-byte aligned, 1 <= M <= DQ_MAX_M
 *   qweight  [N, K*bits/32] words, 16-byte aligned
 *   scales   fp16 [N, K/group_size]
 *   zeros    fp16 [N, K/group_size] if !symmetric, else NULL
 *   y        fp16 [M, N] output (written, never read)
 * group_size must divide K and be a multiple of 128/bits codes (one 16-byte
 * load), which excludes INT2 with group_size 32 (dequant_gemv.cu:357-361).
 * x must be smaller than 2 GiB. Weights of any size are taken: a weight whose
 * qweight or scales reach 2 GiB (the kernels' 32-bit buffer offsets) is
 * launched as row slices below that, writing disjoint columns of y. */
int dq_gemv(const uint16_t* x, const uint32_t* qweight, const uint16_t* scales,
            const uint16_t* zeros, uint16_t* y, int64_t M, int64_t N, int64_t K,
            int64_t bits, int64_t group_size, int symmetric, int interleaved,
            dq_stream_t stream);

/* One problem of a grouped GEMV launch: y[M, N] = x[M, K] @ W^T. */
typedef struct dq_gemv_problem {
  const uint16_t* x;        /* fp16 [M, K], 16-byte aligned */
  const uint32_t* qweight;  /* [N, K*bits/32], 16-byte aligned */
  const uint16_t* scales;   /* fp16 [N, K/group_size] */
  const uint16_t* zeros;    /* fp16 [N, K/group_size], or NULL when symmetric */
  uint16_t* y;              /* fp16 [M, N] */
  int64_t N;
  int64_t K;
  int64_t group_size;       /* == K for per-channel */
} dq_gemv_problem;

/* Most problems one dq_gemv_batched call takes. */
#define DQ_MAX_BATCH 16

/* Grouped fused dequant + GEMV: up to DQ_MAX_BATCH independent problems that
 * share M and the format (bits, symmetric, interleaved) in ONE kernel launch,
 * e.g. q|k|v or gate|up of a decoder layer, whose inputs coincide, or the
 * projections of several layers. Each problem obeys the rules of dq_gemv;
 * results match per-problem dq_gemv calls to within fp32 rounding of the
 * split-K partial sums (see dq_gemv_plan). `problems` is a host array read
 * during the call. No reference counterpart: the reference launches
 * one kernel per linear (dequant/quant_linear.py:72-82); this is the grouped
 * launch its decode path would use to avoid per-launch overhead. */
int dq_gemv_batched(const dq_gemv_problem* problems, int count, int64_t M, int64_t bits, int symmetric,
                    int interleaved, dq_stream_t stream);

/* Activation prologues of dq_gemv_prologue_batched. */
#define DQ_PROLOGUE_RMSNORM 1 /* y = W (rmsnorm(x; eps) * gamma): aux[i] = gamma, fp16 [K] */
#define DQ_PROLOGUE_SWIGLU 2  /* y = W (silu(x) * up): x = gate output, aux[i] = up, fp16 [M, K] */

/* Grouped GEMV (operand rules of dq_gemv_batched, M = 1) whose activations
 * first pass through a fused prologue, so the op before a Llama projection
 * costs no kernel of its own:
 *   DQ_PROLOGUE_RMSNORM  the RMSNorm in front of q|k|v and gate|up:
 *     y = W h, h = x / sqrt(mean(x^2) + eps) * gamma (mean over K, in fp32);
 *     computed as (W (x * gamma)) / sqrt(mean(x^2) + eps), with fp16
 *     products x * gamma;
 *   DQ_PROLOGUE_SWIGLU   the SwiGLU in front of down_proj:
 *     y = W h, h = fp16(fp16(silu(x)) * up), silu(g) = g / (1 + e^-g) in fp32.
 * aux[i] belongs to problem i (16-byte aligned). No reference counterpart: the
 * fusion of RMSNorm and SwiGLU into the projections is the reference's planned
 * next step (MODEL_SELECTION.md:211-218; byte_model.py:227-228 counts those
 * activation bytes); results match the unfused ops (torch RMSNorm / SiLU * up,
 * then dq_gemv_batched) to fp16 rounding of the activations. */
int dq_gemv_prologue_batched(const dq_gemv_problem* problems, const void* const* aux, int count, int64_t M,
                             int64_t bits, int symmetric, int interleaved, int prologue, float eps,
                             dq_stream_t stream);

/* Largest batch (rows of x) of dq_gemm_small. */
#define DQ_MAX_GEMM_M 64

/* Fused small GEMM: y[M, N] = fp16_rn( x[M, K] @ W16^T ), fp32 accumulation,
 * for 1 <= M <= DQ_MAX_GEMM_M, over up to DQ_MAX_BATCH problems of one format
 * (operand rules of dq_gemv_batched). W16 is the fp16 weight dq_dequantize
 * writes (packer.py:177-189), formed in registers and never stored. No
 * reference counterpart: it replaces, for batches of 9..64 rows, the
 * reference's dequantize + F.linear pair (dequant/quant_linear.py:131-132)
 * with one pass over the packed bytes; results equal that pair's up to the
 * order of the fp32 summation. */
int dq_gemm_small(const dq_gemv_problem* problems, int count, int64_t M, int64_t bits, int symmetric,
                  int interleaved, dq_stream_t stream);

/* dq_gemm_small for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops and harnesses that forbid hipMalloc); no
 * counterpart in the reference. Same operands, kernels and results as
 * dq_gemm_small, which allocates an 8 MiB scratch per stream on first use
 * for the split along K of launches with 16 < M; this entry point allocates
 * nothing: it uses the library's static 8 MiB device array, one per GPU,
 * held until the process ends. A launch plans its split within that array
 * (one needing more partial tiles takes fewer splits, down to none), so no
 * size exceeds it; M past DQ_MAX_GEMM_M is rejected as by dq_gemm_small.
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (on different streams) race. */
int dq_gemm_small_noalloc(const dq_gemv_problem* problems, int count, int64_t M, int64_t bits, int symmetric,
                          int interleaved, dq_stream_t stream);

/* Split along K that dq_gemm_small / dq_gemm_small_noalloc would use for
 * these problems (no reference counterpart; pure host logic), for profiling
 * and tuning tools: splits[i] = blocks per 64-column group of problem i along
 * K (1: unsplit, always for M <= 16). A launch with any problem above 1 runs
 * as two kernels (gemm_walk_kernel, then gemm_split_sum_kernel summing its
 * partial tiles). Weights past 2 GiB, which dq_gemm_small launches as row
 * slices, are planned here as one problem. */
int dq_gemm_small_plan(const dq_gemv_problem* problems, int count, int64_t M, int64_t bits, int* splits);

/* Geometry the launch of these problems would use (no reference
 * counterpart), for profiling and tuning tools; pure host logic. For each
 * problem i, waves_per_tile[i] waves (1, 2 or 4) share one tile along K;
 * the launch uses *rows_per_tile output rows per tile and the kernel
 *   *kernel_kind == 1: gemv_quad_kernel<bits, symmetric, interleaved,
 *                      rows_per_tile / 4, MG> (matrix cores; 2 <= M <= 8,
 *                      any group size; MG = 1 for M <= 4, else 2; for
 *                      M = 2 only launches that kind 7 does not take),
 *   *kernel_kind == 2: gemv_m1_kernel<bits, symmetric, interleaved,
 *                      rows_per_tile, false> (M = 1; VALU dot products), or
 *   *kernel_kind == 3: gemv_m1_kernel<bits, symmetric, interleaved,
 *                      rows_per_tile, true> (M = 1; dot products on the
 *                      matrix cores; not chosen by the current geometry),
 *   *kernel_kind == 4: gemv_m1_pipe_kernel<bits, symmetric, interleaved,
 *                      rows_per_tile> (M = 1, launches whose tiles are all
 *                      one wave wide: the next batch's loads are issued while
 *                      the current batch is computed),
 *   *kernel_kind == 6: gemv_m1_kernel's INT2 variant that keeps a wave's
 *                      activations across consecutive 8-row one-batch tiles
 *                      (K <= 4096, at least two rounds of its grid),
 *   *kernel_kind == 7: gemv_mx_pipe_kernel<bits, symmetric, interleaved,
 *                      rows_per_tile, 2> (M = 2, launches whose tiles are
 *                      all one wave wide: kind 4's walk with each weight
 *                      chunk dotted with both batch rows),
 *   *kernel_kind == 8: gemv_m1_pipe_split_kernel<bits, symmetric,
 *                      interleaved, rows_per_tile, waves_per_tile> (M = 1,
 *                      INT4 / INT8 launches of 4-row tiles whose K is split
 *                      over the same 2 or 4 waves in every problem, at most
 *                      1024 block-tiles: kind 4's walk over the K shares).
 * Kind 6 depends on the device's co-resident blocks; without a device the
 * plan assumes 256 CUs. (Kind 5, a block-staged INT2 variant, is no longer
 * returned: the pipelined kernel of kind 4 measured faster on its launches.)
 * The geometry is chosen per launch, so a problem's result is deterministic
 * for a given launch but may differ in the last bits between a grouped launch
 * and a single one. waves_per_tile must hold `count` ints. */
int dq_gemv_plan(const dq_gemv_problem* problems, int count, int64_t M, int64_t bits, int* waves_per_tile,
                 int* rows_per_tile, int* kernel_kind);

/* Profiling hook (no reference counterpart; the reference profiles with
 * Nsight, scripts/bench_dequant_kernel.py:205-229): when both are non-NULL
 * hipEvent_t handles, the NEXT dq_gemv / dq_gemv_batched launch on the calling
 * thread records `start_event` when its kernel starts executing and
 * `stop_event` when it ends (hipExtLaunchKernelGGL), so the pair times the
 * kernel alone, without launch gaps. The setting is consumed by that launch;
 * passing NULL, NULL clears it. Do not use while capturing a HIP graph. */
int dq_set_launch_events(void* start_event, void* stop_event);

/* out[N, K] = fp16_rn( (code - offset) * scale ), bit-exact with the
 * reference's packer.dequantize (dequant/packer.py:177-189). Replaces
 * dequant_cuda.dequantize (kernels/dequant_gemv.cu:310-337, kernel :113-140).
 * group_size must be a multiple of 32/bits (one word; :315-317).
 * out must be 16-byte aligned. */
int dq_dequantize(const uint32_t* qweight, const uint16_t* scales, const uint16_t* zeros,
                  uint16_t* out, int64_t N, int64_t K, int64_t bits, int64_t group_size,
                  int symmetric, int interleaved, dq_stream_t stream);

/* out[N, K] = the unsigned codes, int32, logical order; bit-exact with the
 * reference's packer.unpack (dequant/packer.py:164-174). No reference kernel:
 * the reference unpacks only inside its kernels; this exposes the unpack step
 * so that it can be checked bit for bit. out must be 16-byte aligned. */
int dq_unpack(const uint32_t* qweight, int32_t* out, int64_t N, int64_t K, int64_t bits,
              int interleaved, dq_stream_t stream);

/* out[i] = in[i] + 1 for fp32, the toolchain smoke kernel
 * (kernels/smoke.cu:9-25). Kept for export-surface parity. */
int dq_add_one(const float* in, float* out, int64_t n, dq_stream_t stream);

/* Measurement kernels for the benchmark's denominators (no reference
 * counterpart in the kernels; the reference measures its read ceiling with
 * torch ops, scripts/bandwidth_by_dtype.py:85-106, and quotes it in
 * hardware.md:71-100):
 *   dq_stream_read   reads `bytes` (a multiple of 16; data 16-byte aligned)
 *                    once, non-temporal, the chip sweeping the buffer in
 *                    address order in 1 KiB wave loads: the practical HBM
 *                    read ceiling. sink (>= 4 bytes of device
 *                    memory) is written only for a data pattern that real
 *                    buffers do not produce; it exists so the loads cannot
 *                    be dropped;
 *   dq_empty_kernel  one wave that does nothing: the launch gap of
 *                    back-to-back launches (e.g. in a HIP graph).
 * Both launch on `stream` and may be captured. */
int dq_stream_read(const void* data, int64_t bytes, uint32_t* sink, dq_stream_t stream);
int dq_empty_kernel(dq_stream_t stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* DEQUANT_HIP_H_ */

// Internal interface between the C ABI layer (dq_capi.cpp) and the HIP
// kernels (dq_kernels.hip). Arguments reaching these launchers have already
// been validated by the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dq {

// Largest number of GEMV problems one launch takes (they travel by value in
// the kernel argument block).
constexpr int kMaxBatch = 16;

// One y[M, N] = x[M, K] @ W^T problem of a (possibly grouped) launch.
struct GemvOperand {
  const uint16_t* x;        // fp16 [M, K]
  const uint32_t* qweight;  // [N, K*bits/32]
  const uint16_t* scales;   // fp16 [N, K/group_size]
  const uint16_t* zeros;    // fp16 [N, K/group_size] or nullptr (symmetric)
  uint16_t* y;              // fp16 [M, N]
  int64_t N, K, group_size;
  const uint16_t* aux = nullptr;  // prologue operand: RMSNorm gamma fp16 [K] or SwiGLU up fp16 [M, K]
  int64_t ldy = 0;                // row stride of y in elements; 0 = N (a row slice of a larger problem sets it)
};

// Profiling hook: when both events are non-null, the next GEMV launch on this
// thread is issued with hipExtLaunchKernelGGL and these start/stop events
// (they then bracket the kernel's own execution), after which they are cleared.
void set_launch_events(hipEvent_t start, hipEvent_t stop);

// Launch geometry a grouped GEMV would use: waves per tile along K for each
// problem (wk[0..count-1]), the launch's rows per tile, and which kernel runs:
// *mfma == 1: gemv_quad_kernel<bits, sym, inter, rows / 4, MG> (2 <= M <= 8);
// *mfma == 2: gemv_m1_kernel<bits, sym, inter, rows, false> (M = 1, VALU dots);
// *mfma == 3: gemv_m1_kernel<bits, sym, inter, rows, true> (M = 1, MFMA dots);
// *mfma == 4: gemv_m1_pipe_kernel<bits, sym, inter, rows> (M = 1, pipelined walk);
// *mfma == 6: gemv_m1_kernel's INT2 kept-activation variant (M = 1);
// *mfma == 7: gemv_mx_pipe_kernel<bits, sym, inter, rows, 2> (M = 2, one-wave tiles);
// *mfma == 8: gemv_m1_pipe_split_kernel<bits, sym, inter, rows, wk> (M = 1, split K).
void plan_gemv_batch(const GemvOperand* ops, int count, int64_t M, int bits, int* wk, int* rows, int* mfma);

// All problems of one launch share M and the format (bits, symmetry, layout).
hipError_t launch_gemv_batch(const GemvOperand* ops, int count, int64_t M, int bits, bool symmetric,
                             bool interleaved, hipStream_t stream);

// Activation prologues of launch_gemv_prologue_batch (every problem's `aux`
// must be set): y = W (rmsnorm(x) * gamma) with aux = gamma [K] and eps, or
// y = W (silu(x) * up) with aux = up [M, K] (x = the gate projection's output).
constexpr int kPrologueRmsNorm = 1;
constexpr int kPrologueSwiGlu = 2;

// launch_gemv_batch with an activation prologue; M = 1.
hipError_t launch_gemv_prologue_batch(const GemvOperand* ops, int count, int64_t M, int bits, bool symmetric,
                                      bool interleaved, int prologue, float eps, hipStream_t stream);

// Largest M the small fused GEMM takes (launch_gemm_batch).
constexpr int kMaxGemmM = 64;

// Scratch of the small GEMM's split along K (launch_gemm_batch): fp32
// partial tiles, written by one launch and summed by the next. Launches that
// share one scratch must not overlap.
constexpr int64_t kGemmScratchBytes = int64_t(8) << 20;

// y = x @ W16^T for 1 <= M <= kMaxGemmM with W16 the fp16 weight that
// dequantize materializes, built in registers (one pass over the packed
// bytes, fp32 accumulation on the matrix cores). Same operands as
// launch_gemv_batch. `scratch` (kGemmScratchBytes, or null: no split along
// K) serves launches with 16 < M.
hipError_t launch_gemm_batch(const GemvOperand* ops, int count, int64_t M, int bits, bool symmetric,
                             bool interleaved, void* scratch, hipStream_t stream);

// Split along K of a launch_gemm_batch launch with a scratch (pure host
// logic): gemm_walk_splits gives the launch's split factor S (1: unsplit, as
// for M <= 16 or without a scratch), gemm_problem_splits the blocks per column
// group of a problem with K columns under it. A problem with more than one
// runs as two kernel launches (the walk, then the sum of its partials).
int gemm_walk_splits(const GemvOperand* ops, int count, int64_t M, int bits, bool scratch);
int gemm_problem_splits(int64_t K, int bits, int S);

// Device address, on the current device, of the library's static scratch
// (kGemmScratchBytes) for dq_gemm_small_noalloc; allocates nothing.
hipError_t gemm_static_scratch(void** out);

struct DequantProblem {
  const uint32_t* qweight;
  const uint16_t* scales;
  const uint16_t* zeros;
  uint16_t* out;  // fp16 [N, K]
  int64_t N, K;
  int bits;
  int64_t group_size;
  bool symmetric, interleaved;
};

hipError_t launch_dequantize(const DequantProblem& p, hipStream_t stream);
hipError_t launch_unpack(const uint32_t* qweight, int32_t* out, int64_t N, int64_t K, int bits,
                         bool interleaved, hipStream_t stream);
hipError_t launch_add_one(const float* in, float* out, int64_t n, hipStream_t stream);

// Measurement kernels: a streaming read of `bytes` (a multiple of 16) and an
// empty kernel (one wave).
hipError_t launch_stream_read(const void* data, int64_t bytes, uint32_t* sink, hipStream_t stream);
hipError_t launch_empty(hipStream_t stream);

}  // namespace dq

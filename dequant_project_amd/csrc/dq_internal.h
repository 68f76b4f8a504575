// Internal interface between the C ABI layer (dq_capi.cpp) and the HIP
// kernels (dq_kernels.hip). Arguments reaching these launchers have already
// been validated by the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dq {

struct GemvProblem {
  const uint16_t* x;        // fp16 [M, K]
  const uint32_t* qweight;  // [N, K*bits/32]
  const uint16_t* scales;   // fp16 [N, K/group_size]
  const uint16_t* zeros;    // fp16 [N, K/group_size] or nullptr (symmetric)
  uint16_t* y;              // fp16 [M, N]
  int64_t M, N, K;
  int bits;
  int64_t group_size;
  bool symmetric, interleaved;
};

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

hipError_t launch_gemv(const GemvProblem& p, hipStream_t stream);
hipError_t launch_dequantize(const DequantProblem& p, hipStream_t stream);
hipError_t launch_unpack(const uint32_t* qweight, int32_t* out, int64_t N, int64_t K, int bits,
                         bool interleaved, hipStream_t stream);
hipError_t launch_add_one(const float* in, float* out, int64_t n, hipStream_t stream);

}  // namespace dq

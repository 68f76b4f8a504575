// C ABI of the fused dequant + GEMV engine (declared in include/dequant_hip.h).
//
// Two layers:
//   dq_check_*  validate operand descriptors in the order, and with the
//               messages, of the reference's host code
//               (kernels/dequant_gemv.cu:230-283 check_weight, :310-317
//               dequantize, :342-361 gemv). Pure host logic: no HIP call, so
//               they run on machines without a GPU.
//   dq_gemv / dq_gemv_batched / dq_dequantize / dq_unpack / dq_add_one
//               validate the scalar contract of a raw-pointer call (the rules
//               that do not need tensor metadata) and launch on `stream`.
// Errors are reported as a status code plus a thread-local message.

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <utility>
#include <vector>

#include "dequant_hip.h"
#include "dq_internal.h"

static_assert(DQ_MAX_BATCH == dq::kMaxBatch, "batch limits of the ABI and the kernels differ");
static_assert(DQ_PROLOGUE_RMSNORM == dq::kPrologueRmsNorm && DQ_PROLOGUE_SWIGLU == dq::kPrologueSwiGlu,
              "prologue codes of the ABI and the kernels differ");

namespace {

thread_local std::string g_error;

int fail(int status, const std::string& msg) {
  g_error = msg;
  return status;
}

template <typename... Ts>
std::string cat(const Ts&... parts) {
  std::ostringstream os;
  (os << ... << parts);
  return os.str();
}

// torch's IntArrayRef formatting: "[a, b, c]"
std::string sizes_str(const dq_tensor* t) {
  std::ostringstream os;
  os << "[";
  for (int i = 0; i < t->ndim && i < 4; ++i) os << (i ? ", " : "") << t->sizes[i];
  os << "]";
  return os.str();
}

bool same_sizes(const dq_tensor* a, const dq_tensor* b) {
  if (a->ndim != b->ndim) return false;
  for (int i = 0; i < a->ndim && i < 4; ++i)
    if (a->sizes[i] != b->sizes[i]) return false;
  return true;
}

bool same_device(const dq_tensor* a, const dq_tensor* b) {
  return a->is_device == b->is_device && (!a->is_device || a->device == b->device);
}

constexpr int64_t kMaxDim = int64_t(1) << 30;  // kernel index arithmetic stays in range

// kernels/dequant_gemv.cu:233-238
int check_bits_group_k(int64_t bits, int64_t group_size, int64_t K) {
  if (!(bits == 2 || bits == 4 || bits == 8))
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("bits must be 2, 4 or 8, got ", bits));
  if (group_size <= 0)
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("group_size must be positive, got ", group_size));
  if (!(K > 0 && K % group_size == 0))
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("K=", K, " is not divisible by group_size=", group_size));
  return DQ_OK;
}

// kernels/dequant_gemv.cu:259-261
int check_zeros_presence(bool has_zeros, bool symmetric) {
  if (has_zeros != !symmetric)
    return fail(DQ_ERR_INVALID_ARGUMENT,
                symmetric ? "symmetric=true takes no zeros" : "symmetric=false requires zeros");
  return DQ_OK;
}

// kernels/dequant_gemv.cu:240-246
int check_qweight(const dq_tensor* qw, int64_t bits, int64_t K) {
  const int64_t per = 32 / bits;
  if (!qw->is_device) return fail(DQ_ERR_INVALID_ARGUMENT, "qweight must be a CUDA tensor");
  if (qw->dtype != DQ_DTYPE_INT32) return fail(DQ_ERR_INVALID_ARGUMENT, "qweight must be int32");
  if (!qw->contiguous) return fail(DQ_ERR_INVALID_ARGUMENT, "qweight must be contiguous");
  if (qw->ndim != 2) return fail(DQ_ERR_INVALID_ARGUMENT, cat("qweight must be 2-D, got ", qw->ndim, "-D"));
  if (qw->sizes[1] * per != K)
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("qweight has ", qw->sizes[1], " words per row, which is ",
                                             qw->sizes[1] * per, " codes, but K=", K));
  return DQ_OK;
}

// check_weight, kernels/dequant_gemv.cu:230-283
int check_weight(const dq_tensor* qw, const dq_tensor* sc, const dq_tensor* ze, int64_t bits,
                 int64_t group_size, bool symmetric, int64_t K) {
  int st = check_bits_group_k(bits, group_size, K);
  if (st) return st;
  if ((st = check_qweight(qw, bits, K))) return st;

  const int64_t N = qw->sizes[0];
  const int64_t n_groups = K / group_size;
  if (!sc->is_device) return fail(DQ_ERR_INVALID_ARGUMENT, "scales must be a CUDA tensor");
  if (sc->dtype != DQ_DTYPE_FLOAT16) return fail(DQ_ERR_INVALID_ARGUMENT, "scales must be float16");
  if (!sc->contiguous) return fail(DQ_ERR_INVALID_ARGUMENT, "scales must be contiguous");
  if (!(sc->ndim == 2 && sc->sizes[0] == N && sc->sizes[1] == n_groups))
    return fail(DQ_ERR_INVALID_ARGUMENT,
                cat("scales must be [", N, ", ", n_groups, "], got ", sizes_str(sc)));
  if (!same_device(sc, qw))
    return fail(DQ_ERR_INVALID_ARGUMENT, "scales and qweight must be on the same device");

  if ((st = check_zeros_presence(ze != nullptr, symmetric))) return st;
  if (ze) {
    if (!ze->is_device) return fail(DQ_ERR_INVALID_ARGUMENT, "zeros must be a CUDA tensor");
    if (ze->dtype != DQ_DTYPE_FLOAT16) return fail(DQ_ERR_INVALID_ARGUMENT, "zeros must be float16");
    if (!ze->contiguous) return fail(DQ_ERR_INVALID_ARGUMENT, "zeros must be contiguous");
    if (!same_sizes(ze, sc))
      return fail(DQ_ERR_INVALID_ARGUMENT, cat("zeros must have the same shape as scales, got ", sizes_str(ze)));
    if (!same_device(ze, qw))
      return fail(DQ_ERR_INVALID_ARGUMENT, "zeros and qweight must be on the same device");
  }
  return DQ_OK;
}

// kernels/dequant_gemv.cu:357-361
int check_gemv_group(int64_t group_size, int64_t bits) {
  const int64_t cpl = 128 / bits;
  if (group_size % cpl != 0)
    return fail(DQ_ERR_INVALID_ARGUMENT,
                cat("group_size=", group_size, " must be a multiple of ", cpl,
                    " (the codes one lane loads per uint4) at ", bits,
                    " bits; this excludes INT2 with group_size 32"));
  return DQ_OK;
}

// kernels/dequant_gemv.cu:315-317
int check_dequant_group(int64_t group_size, int64_t bits) {
  const int64_t per = 32 / bits;
  if (group_size % per != 0)
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("group_size=", group_size, " must be a multiple of ", per,
                                             " values per uint32 word at ", bits, " bits"));
  return DQ_OK;
}

// kernels/dequant_gemv.cu:349-350
int check_m(int64_t M) {
  if (!(M >= 1 && M <= DQ_MAX_M))
    return fail(DQ_ERR_UNSUPPORTED, cat("gemv handles 1 <= M <= ", DQ_MAX_M, ", got M=", M,
                                        "; use the dequantize + F.linear fallback"));
  return DQ_OK;
}

// dq_gemm_small's batch range (no reference counterpart)
int check_gemm_m(int64_t M) {
  if (!(M >= 1 && M <= DQ_MAX_GEMM_M))
    return fail(DQ_ERR_UNSUPPORTED, cat("gemm_small handles 1 <= M <= ", DQ_MAX_GEMM_M, ", got M=", M,
                                        "; use the dequantize + F.linear fallback"));
  return DQ_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Limits of this implementation (no reference counterpart: the reference's
// kernels index with int and would overflow silently).
int check_extent(int64_t N, int64_t K) {
  if (N < 0) return fail(DQ_ERR_INVALID_ARGUMENT, cat("N must be non-negative, got ", N));
  if (N >= (int64_t(1) << 31) || K > kMaxDim)
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("shape [", N, ", ", K, "] exceeds the supported extent"));
  return DQ_OK;
}

// The GEMV kernels address every operand with 32-bit buffer offsets and use
// offsets at or above 2^31 as "out of range", so each operand of a launched
// problem stays below 2 GiB. Weights past that (an INT8 lm_head of
// 128256 x 16384 is 2.1 GB) are launched as row slices (slice_problems); the
// activations, M x K fp16, must fit as they are.
constexpr int64_t kOperandLimit = (int64_t(1) << 31) - 1;

int check_gemv_bytes(int64_t M, int64_t K) {
  if (M * K * 2 > kOperandLimit)
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("x of shape [", M, ", ", K, "] exceeds the 2 GiB operand limit of ",
                                             "the GEMV kernels"));
  return DQ_OK;
}

// Rows of one slice: every weight operand of the slice (qweight, scales,
// zeros) below 2 GiB; a multiple of 64 rows when that leaves any.
int64_t slice_rows(int64_t K, int64_t bits, int64_t group_size) {
  const int64_t wrow = K * bits / 8, mrow = K / group_size * 2;
  int64_t r = std::min(kOperandLimit / wrow, kOperandLimit / mrow);
  if (r >= 64) r = r / 64 * 64;
  return std::max<int64_t>(r, 1);
}

// `op` as row slices below the operand limit (one slice when it already is):
// slice j holds rows [r0, r0 + n) of qweight, scales and zeros and writes
// y[:, r0 : r0 + n], so its y row stride stays the whole problem's N.
void append_slices(const dq::GemvOperand& op, int64_t bits, std::vector<dq::GemvOperand>& out) {
  const int64_t rows = slice_rows(op.K, bits, op.group_size);
  const int64_t words = op.K * bits / 32, groups = op.K / op.group_size;
  for (int64_t r0 = 0; r0 < op.N; r0 += rows) {
    dq::GemvOperand sl = op;
    sl.N = std::min(rows, op.N - r0);
    sl.qweight = op.qweight + r0 * words;
    sl.scales = op.scales + r0 * groups;
    sl.zeros = op.zeros ? op.zeros + r0 * groups : nullptr;
    sl.y = op.y + r0;
    sl.ldy = op.ldy ? op.ldy : op.N;
    out.push_back(sl);
  }
}

// Launches a list of problems (already sliced) in groups of at most
// kMaxBatch; one launch unless slicing produced more problems than that.
template <typename Launch>
hipError_t launch_in_groups(const std::vector<dq::GemvOperand>& ops, Launch launch) {
  for (size_t i = 0; i < ops.size(); i += dq::kMaxBatch) {
    const hipError_t e = launch(ops.data() + i, static_cast<int>(std::min<size_t>(dq::kMaxBatch, ops.size() - i)));
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// The scalar contract of one raw-pointer GEMV problem.
int check_gemv_problem(const uint16_t* x, const uint32_t* qweight, const uint16_t* scales, const uint16_t* zeros,
                       const uint16_t* y, int64_t M, int64_t N, int64_t K, int64_t bits, int64_t group_size,
                       int symmetric) {
  if (!x || !qweight || !scales || !y)
    return fail(DQ_ERR_INVALID_ARGUMENT, "x, qweight, scales and y must not be NULL");
  if (!aligned16(x)) return fail(DQ_ERR_INVALID_ARGUMENT, "x must be 16-byte aligned");
  int st = check_bits_group_k(bits, group_size, K);
  if (st) return st;
  if ((st = check_zeros_presence(zeros != nullptr, symmetric != 0))) return st;
  if ((st = check_gemv_group(group_size, bits))) return st;
  if (!aligned16(qweight)) return fail(DQ_ERR_INVALID_ARGUMENT, "qweight must be 16-byte aligned");
  if ((st = check_extent(N, K))) return st;
  return check_gemv_bytes(M, K);
}

int launch_status(hipError_t e) {
  if (e == hipSuccess) return DQ_OK;
  return fail(DQ_ERR_LAUNCH, cat("HIP launch failed: ", hipGetErrorString(e)));
}

// Scratch of the small GEMM's split along K (dq::kGemmScratchBytes), one per
// device and stream, so that launches on different streams never share one:
// allocated on the stream's first dq_gemm_small with 16 < M and kept until
// the process ends. A stream first seen inside a graph capture gets its
// scratch too: the thread's capture mode is relaxed for the allocation, as
// torch's allocator does (the scratch needs no initial contents). If that
// fails the stream gets none and its launches run unsplit, with the same
// results.
void* gemm_scratch(hipStream_t stream) {
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, void*> table;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_pair(dev, stream);
  const auto it = table.find(key);
  if (it != table.end()) return it->second;
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  void* p = nullptr;
  const bool ok = hipMalloc(&p, dq::kGemmScratchBytes) == hipSuccess;
  (void)hipThreadExchangeStreamCaptureMode(&mode);
  (void)hipGetLastError();
  if (!ok) return nullptr;
  table.emplace(key, p);
  return p;
}

// dq_gemm_small and dq_gemm_small_noalloc: the same validation and kernels;
// the split scratch comes from the per-stream table (allocated on first use)
// or, allocating nothing, from the library's static per-device array.
int gemm_small_call(const dq_gemv_problem* problems, int count, int64_t M, int64_t bits, int symmetric,
                    int interleaved, dq_stream_t stream, bool noalloc) {
  g_error.clear();
  if (count < 1 || count > DQ_MAX_BATCH)
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("count must be in [1, ", DQ_MAX_BATCH, "], got ", count));
  if (!problems) return fail(DQ_ERR_INVALID_ARGUMENT, "problems must not be NULL");
  int st = check_gemm_m(M);
  if (st) return st;
  std::vector<dq::GemvOperand> ops;
  for (int i = 0; i < count; ++i) {
    const dq_gemv_problem& p = problems[i];
    if ((st = check_gemv_problem(p.x, p.qweight, p.scales, p.zeros, p.y, M, p.N, p.K, bits, p.group_size,
                                 symmetric))) {
      g_error = cat("problem ", i, ": ", g_error);
      return st;
    }
    if (p.N > 0) append_slices(dq::GemvOperand{p.x, p.qweight, p.scales, p.zeros, p.y, p.N, p.K, p.group_size},
                               bits, ops);
  }
  if (ops.empty()) return DQ_OK;
  const hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  void* scratch = nullptr;
  if (!noalloc) {
    scratch = gemm_scratch(hs);
  } else if (const hipError_t e = dq::gemm_static_scratch(&scratch); e != hipSuccess) {
    return fail(DQ_ERR_HIP, cat("gemm_small_noalloc: no address for the static scratch on this device: ",
                                hipGetErrorString(e)));
  }
  return launch_status(launch_in_groups(ops, [&](const dq::GemvOperand* o, int n) {
    return dq::launch_gemm_batch(o, n, M, static_cast<int>(bits), symmetric != 0, interleaved != 0, scratch, hs);
  }));
}

}  // namespace

extern "C" {

const char* dq_last_error(void) { return g_error.c_str(); }

const char* dq_status_name(int status) {
  switch (status) {
    case DQ_OK: return "DQ_OK";
    case DQ_ERR_INVALID_ARGUMENT: return "DQ_ERR_INVALID_ARGUMENT";
    case DQ_ERR_UNSUPPORTED: return "DQ_ERR_UNSUPPORTED";
    case DQ_ERR_LAUNCH: return "DQ_ERR_LAUNCH";
    case DQ_ERR_HIP: return "DQ_ERR_HIP";
    default: return "DQ_ERR_UNKNOWN";
  }
}

int dq_version(void) { return 100; }

}  // extern "C"

namespace {

// The tensor rules of dq_check_gemv / dq_check_gemm_small; `check_rows` is
// the batch-range rule of the entry point.
int check_packed_product(const dq_tensor* x, const dq_tensor* qweight, const dq_tensor* scales,
                         const dq_tensor* zeros, int64_t bits, int64_t group_size, int symmetric,
                         int (*check_rows)(int64_t)) {
  g_error.clear();
  if (!x || !qweight || !scales)
    return fail(DQ_ERR_INVALID_ARGUMENT, "x, qweight and scales descriptors must not be NULL");
  // kernels/dequant_gemv.cu:342-352
  if (!x->is_device) return fail(DQ_ERR_INVALID_ARGUMENT, "x must be a CUDA tensor");
  if (x->dtype != DQ_DTYPE_FLOAT16) return fail(DQ_ERR_INVALID_ARGUMENT, "x must be float16");
  if (!x->contiguous) return fail(DQ_ERR_INVALID_ARGUMENT, "x must be contiguous");
  if (x->ndim != 2) return fail(DQ_ERR_INVALID_ARGUMENT, cat("x must be 2-D [M, K], got ", x->ndim, "-D"));
  int st = check_rows(x->sizes[0]);
  if (st) return st;
  if (!aligned16(x->data)) return fail(DQ_ERR_INVALID_ARGUMENT, "x must be 16-byte aligned");
  const int64_t K = x->sizes[1];
  // :354 check_weight, :355 device, :357-361 group vs. 16-byte load
  if ((st = check_weight(qweight, scales, zeros, bits, group_size, symmetric != 0, K))) return st;
  if (!same_device(x, qweight))
    return fail(DQ_ERR_INVALID_ARGUMENT, "x and qweight must be on the same device");
  if ((st = check_gemv_group(group_size, bits))) return st;
  // this implementation's own requirements
  if (!aligned16(qweight->data)) return fail(DQ_ERR_INVALID_ARGUMENT, "qweight must be 16-byte aligned");
  if ((st = check_extent(qweight->sizes[0], K))) return st;
  return check_gemv_bytes(x->sizes[0], K);
}

}  // namespace

extern "C" {

int dq_check_gemv(const dq_tensor* x, const dq_tensor* qweight, const dq_tensor* scales,
                  const dq_tensor* zeros, int64_t bits, int64_t group_size, int symmetric) {
  return check_packed_product(x, qweight, scales, zeros, bits, group_size, symmetric, check_m);
}

int dq_check_gemm_small(const dq_tensor* x, const dq_tensor* qweight, const dq_tensor* scales,
                        const dq_tensor* zeros, int64_t bits, int64_t group_size, int symmetric) {
  return check_packed_product(x, qweight, scales, zeros, bits, group_size, symmetric, check_gemm_m);
}

int dq_check_dequantize(const dq_tensor* qweight, const dq_tensor* scales, const dq_tensor* zeros,
                        int64_t bits, int64_t group_size, int symmetric, int64_t K) {
  g_error.clear();
  if (!qweight || !scales)
    return fail(DQ_ERR_INVALID_ARGUMENT, "qweight and scales descriptors must not be NULL");
  int st = check_weight(qweight, scales, zeros, bits, group_size, symmetric != 0, K);
  if (st) return st;
  if ((st = check_dequant_group(group_size, bits))) return st;
  return check_extent(qweight->sizes[0], K);
}

int dq_check_unpack(const dq_tensor* qweight, int64_t bits, int64_t K) {
  g_error.clear();
  if (!qweight) return fail(DQ_ERR_INVALID_ARGUMENT, "qweight descriptor must not be NULL");
  if (!(bits == 2 || bits == 4 || bits == 8))
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("bits must be 2, 4 or 8, got ", bits));
  if (K <= 0 || K % (32 / bits) != 0)
    return fail(DQ_ERR_INVALID_ARGUMENT,
                cat("K=", K, " is not a positive multiple of ", 32 / bits, " values per word"));
  int st = check_qweight(qweight, bits, K);
  if (st) return st;
  return check_extent(qweight->sizes[0], K);
}

int dq_gemv(const uint16_t* x, const uint32_t* qweight, const uint16_t* scales, const uint16_t* zeros,
            uint16_t* y, int64_t M, int64_t N, int64_t K, int64_t bits, int64_t group_size, int symmetric,
            int interleaved, dq_stream_t stream) {
  g_error.clear();
  int st = check_m(M);
  if (st) return st;
  if ((st = check_gemv_problem(x, qweight, scales, zeros, y, M, N, K, bits, group_size, symmetric))) return st;
  if (N == 0) return DQ_OK;
  std::vector<dq::GemvOperand> ops;
  append_slices(dq::GemvOperand{x, qweight, scales, zeros, y, N, K, group_size}, bits, ops);
  return launch_status(launch_in_groups(ops, [&](const dq::GemvOperand* o, int n) {
    return dq::launch_gemv_batch(o, n, M, static_cast<int>(bits), symmetric != 0, interleaved != 0,
                                 reinterpret_cast<hipStream_t>(stream));
  }));
}

int dq_gemv_batched(const dq_gemv_problem* problems, int count, int64_t M, int64_t bits, int symmetric,
                    int interleaved, dq_stream_t stream) {
  g_error.clear();
  if (count < 1 || count > DQ_MAX_BATCH)
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("count must be in [1, ", DQ_MAX_BATCH, "], got ", count));
  if (!problems) return fail(DQ_ERR_INVALID_ARGUMENT, "problems must not be NULL");
  int st = check_m(M);
  if (st) return st;
  std::vector<dq::GemvOperand> ops;
  for (int i = 0; i < count; ++i) {
    const dq_gemv_problem& p = problems[i];
    if ((st = check_gemv_problem(p.x, p.qweight, p.scales, p.zeros, p.y, M, p.N, p.K, bits, p.group_size,
                                 symmetric))) {
      g_error = cat("problem ", i, ": ", g_error);
      return st;
    }
    if (p.N > 0) append_slices(dq::GemvOperand{p.x, p.qweight, p.scales, p.zeros, p.y, p.N, p.K, p.group_size},
                               bits, ops);
  }
  if (ops.empty()) return DQ_OK;
  return launch_status(launch_in_groups(ops, [&](const dq::GemvOperand* o, int n) {
    return dq::launch_gemv_batch(o, n, M, static_cast<int>(bits), symmetric != 0, interleaved != 0,
                                 reinterpret_cast<hipStream_t>(stream));
  }));
}

int dq_gemv_prologue_batched(const dq_gemv_problem* problems, const void* const* aux, int count, int64_t M,
                             int64_t bits, int symmetric, int interleaved, int prologue, float eps,
                             dq_stream_t stream) {
  g_error.clear();
  if (count < 1 || count > DQ_MAX_BATCH)
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("count must be in [1, ", DQ_MAX_BATCH, "], got ", count));
  if (!problems || !aux) return fail(DQ_ERR_INVALID_ARGUMENT, "problems and aux must not be NULL");
  if (prologue != DQ_PROLOGUE_RMSNORM && prologue != DQ_PROLOGUE_SWIGLU)
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("unknown prologue ", prologue));
  if (prologue == DQ_PROLOGUE_RMSNORM && !(eps >= 0.0f && eps < 1e30f))
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("eps must be finite and non-negative, got ", eps));
  if (M != 1) return fail(DQ_ERR_UNSUPPORTED, cat("fused prologues handle M = 1, got M=", M));
  std::vector<dq::GemvOperand> ops;
  for (int i = 0; i < count; ++i) {
    const dq_gemv_problem& p = problems[i];
    int st = check_gemv_problem(p.x, p.qweight, p.scales, p.zeros, p.y, M, p.N, p.K, bits, p.group_size,
                                symmetric);
    if (!st && !aux[i]) st = fail(DQ_ERR_INVALID_ARGUMENT, "aux must not be NULL");
    if (!st && !aligned16(aux[i])) st = fail(DQ_ERR_INVALID_ARGUMENT, "aux must be 16-byte aligned");
    if (st) {
      g_error = cat("problem ", i, ": ", g_error);
      return st;
    }
    if (p.N > 0) {
      dq::GemvOperand op{p.x, p.qweight, p.scales, p.zeros, p.y, p.N, p.K, p.group_size};
      op.aux = static_cast<const uint16_t*>(aux[i]);
      append_slices(op, bits, ops);
    }
  }
  if (ops.empty()) return DQ_OK;
  return launch_status(launch_in_groups(ops, [&](const dq::GemvOperand* o, int n) {
    return dq::launch_gemv_prologue_batch(o, n, M, static_cast<int>(bits), symmetric != 0, interleaved != 0,
                                          prologue, eps, reinterpret_cast<hipStream_t>(stream));
  }));
}

int dq_gemm_small(const dq_gemv_problem* problems, int count, int64_t M, int64_t bits, int symmetric,
                  int interleaved, dq_stream_t stream) {
  return gemm_small_call(problems, count, M, bits, symmetric, interleaved, stream, false);
}

int dq_gemm_small_noalloc(const dq_gemv_problem* problems, int count, int64_t M, int64_t bits, int symmetric,
                          int interleaved, dq_stream_t stream) {
  return gemm_small_call(problems, count, M, bits, symmetric, interleaved, stream, true);
}

int dq_gemm_small_plan(const dq_gemv_problem* problems, int count, int64_t M, int64_t bits, int* splits) {
  g_error.clear();
  if (count < 1 || count > DQ_MAX_BATCH)
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("count must be in [1, ", DQ_MAX_BATCH, "], got ", count));
  if (!problems || !splits) return fail(DQ_ERR_INVALID_ARGUMENT, "problems and splits must not be NULL");
  int st = check_gemm_m(M);
  if (st) return st;
  if (!(bits == 2 || bits == 4 || bits == 8))
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("bits must be 2, 4 or 8, got ", bits));
  dq::GemvOperand ops[DQ_MAX_BATCH];
  for (int i = 0; i < count; ++i) {
    const dq_gemv_problem& p = problems[i];
    if (p.K <= 0 || p.K % (128 / bits) != 0 || p.N < 0)
      return fail(DQ_ERR_INVALID_ARGUMENT, cat("problem ", i, ": K=", p.K, " must be a positive multiple of ",
                                               128 / bits, " and N=", p.N, " non-negative"));
    ops[i] = dq::GemvOperand{p.x, p.qweight, p.scales, p.zeros, p.y, p.N, p.K, p.group_size};
  }
  const int S = dq::gemm_walk_splits(ops, count, M, static_cast<int>(bits), true);
  for (int i = 0; i < count; ++i) splits[i] = S == 1 ? 1 : dq::gemm_problem_splits(ops[i].K, static_cast<int>(bits), S);
  return DQ_OK;
}

int dq_gemv_plan(const dq_gemv_problem* problems, int count, int64_t M, int64_t bits, int* waves_per_tile,
                 int* rows_per_tile, int* kernel_kind) {
  g_error.clear();
  if (count < 1 || count > DQ_MAX_BATCH)
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("count must be in [1, ", DQ_MAX_BATCH, "], got ", count));
  if (!problems || !waves_per_tile || !rows_per_tile || !kernel_kind)
    return fail(DQ_ERR_INVALID_ARGUMENT,
                "problems, waves_per_tile, rows_per_tile and kernel_kind must not be NULL");
  int st = check_m(M);
  if (st) return st;
  if (!(bits == 2 || bits == 4 || bits == 8))
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("bits must be 2, 4 or 8, got ", bits));
  dq::GemvOperand ops[DQ_MAX_BATCH];
  for (int i = 0; i < count; ++i) {
    const dq_gemv_problem& p = problems[i];
    if (p.K <= 0 || p.K % (128 / bits) != 0 || p.N < 0)
      return fail(DQ_ERR_INVALID_ARGUMENT, cat("problem ", i, ": K=", p.K, " must be a positive multiple of ",
                                               128 / bits, " and N=", p.N, " non-negative"));
    if (p.group_size <= 0 || p.K % p.group_size != 0 || p.group_size % (128 / bits) != 0)
      return fail(DQ_ERR_INVALID_ARGUMENT, cat("problem ", i, ": group_size=", p.group_size,
                                               " must divide K and be a multiple of ", 128 / bits));
    ops[i] = dq::GemvOperand{p.x, p.qweight, p.scales, p.zeros, p.y, p.N, p.K, p.group_size};
  }
  dq::plan_gemv_batch(ops, count, M, static_cast<int>(bits), waves_per_tile, rows_per_tile, kernel_kind);
  return DQ_OK;
}

int dq_set_launch_events(void* start_event, void* stop_event) {
  g_error.clear();
  if ((start_event == nullptr) != (stop_event == nullptr))
    return fail(DQ_ERR_INVALID_ARGUMENT, "start_event and stop_event must both be set or both be NULL");
  dq::set_launch_events(static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event));
  return DQ_OK;
}

int dq_dequantize(const uint32_t* qweight, const uint16_t* scales, const uint16_t* zeros, uint16_t* out,
                  int64_t N, int64_t K, int64_t bits, int64_t group_size, int symmetric, int interleaved,
                  dq_stream_t stream) {
  g_error.clear();
  int st = check_bits_group_k(bits, group_size, K);
  if (st) return st;
  if (!qweight || !scales || !out)
    return fail(DQ_ERR_INVALID_ARGUMENT, "qweight, scales and out must not be NULL");
  if ((st = check_zeros_presence(zeros != nullptr, symmetric != 0))) return st;
  if ((st = check_dequant_group(group_size, bits))) return st;
  if (!aligned16(out)) return fail(DQ_ERR_INVALID_ARGUMENT, "out must be 16-byte aligned");
  if ((st = check_extent(N, K))) return st;
  if (N == 0) return DQ_OK;
  dq::DequantProblem p{qweight, scales, zeros, out, N, K, static_cast<int>(bits), group_size,
                       symmetric != 0, interleaved != 0};
  return launch_status(dq::launch_dequantize(p, reinterpret_cast<hipStream_t>(stream)));
}

int dq_unpack(const uint32_t* qweight, int32_t* out, int64_t N, int64_t K, int64_t bits, int interleaved,
              dq_stream_t stream) {
  g_error.clear();
  if (!(bits == 2 || bits == 4 || bits == 8))
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("bits must be 2, 4 or 8, got ", bits));
  if (K <= 0 || K % (32 / bits) != 0)
    return fail(DQ_ERR_INVALID_ARGUMENT,
                cat("K=", K, " is not a positive multiple of ", 32 / bits, " values per word"));
  if (!qweight || !out) return fail(DQ_ERR_INVALID_ARGUMENT, "qweight and out must not be NULL");
  if (!aligned16(out)) return fail(DQ_ERR_INVALID_ARGUMENT, "out must be 16-byte aligned");
  int st = check_extent(N, K);
  if (st) return st;
  if (N == 0) return DQ_OK;
  return launch_status(dq::launch_unpack(qweight, out, N, K, static_cast<int>(bits), interleaved != 0,
                                         reinterpret_cast<hipStream_t>(stream)));
}

int dq_stream_read(const void* data, int64_t bytes, uint32_t* sink, dq_stream_t stream) {
  g_error.clear();
  if (bytes < 0 || bytes % 16 != 0)
    return fail(DQ_ERR_INVALID_ARGUMENT, cat("bytes must be a non-negative multiple of 16, got ", bytes));
  if (bytes == 0) return DQ_OK;
  if (!data || !sink) return fail(DQ_ERR_INVALID_ARGUMENT, "data and sink must not be NULL");
  if (!aligned16(data)) return fail(DQ_ERR_INVALID_ARGUMENT, "data must be 16-byte aligned");
  return launch_status(dq::launch_stream_read(data, bytes, sink, reinterpret_cast<hipStream_t>(stream)));
}

int dq_empty_kernel(dq_stream_t stream) {
  g_error.clear();
  return launch_status(dq::launch_empty(reinterpret_cast<hipStream_t>(stream)));
}

int dq_add_one(const float* in, float* out, int64_t n, dq_stream_t stream) {
  g_error.clear();
  if (n < 0) return fail(DQ_ERR_INVALID_ARGUMENT, cat("n must be non-negative, got ", n));
  if (n == 0) return DQ_OK;
  if (!in || !out) return fail(DQ_ERR_INVALID_ARGUMENT, "in and out must not be NULL");
  return launch_status(dq::launch_add_one(in, out, n, reinterpret_cast<hipStream_t>(stream)));
}

}  // extern "C"

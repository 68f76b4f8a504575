// gfx950 (CDNA4) kernels of the fused dequant + GEMV engine.
//
// Packed format (dequant/packer.py of the reference, frozen):
//   qweight [N, K/PER] 32-bit words, PER = 32/BITS codes per word; a word's
//   slot s sits at bit offset BITS*s and holds logical code L(s): L(s) = s for
//   "sequential", the packer.py:37-41 table for "interleaved". Codes are
//   unsigned; symmetric codes carry a +2^(BITS-1) bias. scales/zeros are fp16
//   [N, K/group_size]; groups run along K.
//
// What replaces what (reference kernels/dequant_gemv.cu):
//   gemv_m1_kernel     <- gemv_kernel<BITS,SYM,INTER,MT>, MT = 1   :144-217
//   gemv_quad_kernel   <- gemv_kernel<BITS,SYM,INTER,MT>, MT = 8   :144-217
//                         (2 <= M <= 8)
//   dequantize_kernel  <- dequantize_kernel<BITS,SYM,INTER>        :113-140
//   gemm_mfma_kernel   (new: the M > 8 product of quant_linear.py:131-132,
//                      dequantize + F.linear, in one pass for M <= 64;
//                      gemm_shared_x_kernel: its large M <= 32 launches)
//   unpack_kernel      (new: exposes the unpack step for bit-exact checks)
//   add_one_kernel     <- kernels/smoke.cu:9-13
//
// GEMV design (CDNA4, wave64):
//   * One launch takes a list of up to 16 problems of one format (a single
//     call is a list of one; q|k|v or gate|up of a decoder layer share one
//     launch). Work is cut into tiles of R rows; a 256-thread block holds
//     4/wk tiles and the wk waves of a tile split its K range, meeting in LDS.
//   * M = 1: lane l walks the 16-byte chunks cb + l + 64t of its rows, so
//     every global_load_dwordx4 of a wave reads 1 KiB of one row
//     contiguously. A chunk holds 128/BITS codes of one group
//     (group_size % (128/BITS) == 0). Each batch issues the activations, then
//     every zero, scale and weight load of its R rows, before any math.
//   * M = 1 unpacks to biased fp16 codes in one VALU op per pair: under an
//     exponent field of 25 - p, a code masked into mantissa bit p reads
//     exactly 2^(10-p) + q (v_and_or_b32; INT8: one v_perm_b32), and per row
//     and chunk sum (q - z) x = sum (bias + q) x - (sum bias x + z sum x) in
//     fp32, with the two activation sums shared by the tile's rows. Codes sit
//     at mantissa bits 4..9 (biases <= 64; INT8: 1024), which keeps the fp32
//     sums' cancellation far inside the reference's error bound, for any
//     zero point.
//   * 2 <= M <= 8 and the small GEMM unpack to exact fp16 (code - zero) pairs
//     in two VALU ops per pair:
//       v_and_or_b32  (w & mask) | 0x64006400  -> fp16 (1024 + q * 2^p) in both
//                     halves (q sits in mantissa bits [p, p+BITS), p <= 8);
//       v_pk_fma_f16  * 2^-p - (2^(10-p) + z)  -> fp16 (q - z), exact.
//     Zero points outside [-1024, 1024] (possible: the packer stores them
//     unclamped) cannot use that form; such tiles take q exactly and subtract
//     z * sum(x) in fp32 instead (uniform branch, rare).
//   * Pair i holds the word's slots (i, i + PER/2); the activations are
//     gathered into the same pair order, so sequential and interleaved
//     layouts cost the same.
//   * v_dot2_f32_f16 (a diagonal-of-v_mfma_f32_4x4x4_16b_f16 form exists and
//     measured slower) multiplies code pairs with activation pairs and accumulates in fp32;
//     per chunk, acc * scale is added in fp32 -- the reference's factorized
//     scale, within its elementwise fp32 error bound. 2 <= M <= 8 runs the
//     exact form on the matrix cores (gemv_quad_kernel).
//   * Rows are finished with a DPP wave64 reduction (row_shr 1/2/4/8,
//     row_bcast 15/31) instead of an LDS tree; fp16 (RNE) stores.
//
// All kernels are written for gfx950 only; no other target is built.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "dq_internal.h"

namespace dq {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float f16_to_f32(uint16_t u) {
  return static_cast<float>(__builtin_bit_cast(_Float16, u));
}
__device__ __forceinline__ uint16_t f32_to_f16_rn(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));  // v_cvt_f16_f32, RNE
}
__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ h2 splat(_Float16 v) { return h2{v, v}; }

// Slot -> logical code index inside one word (packer.py:37-41 for interleaved).
template <int BITS, bool INTER>
__device__ __forceinline__ constexpr int logical_of_slot(int s) {
  if constexpr (!INTER) {
    return s;
  } else if constexpr (BITS == 4) {
    constexpr int t[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    return t[s];
  } else if constexpr (BITS == 2) {
    constexpr int t[16] = {0, 4, 8, 12, 1, 5, 9, 13, 2, 6, 10, 14, 3, 7, 11, 15};
    return t[s];
  } else {
    constexpr int t[4] = {0, 2, 1, 3};
    return t[s];
  }
}

template <int BITS> struct Fmt {
  static constexpr int PER = 32 / BITS;   // codes per word
  static constexpr int CPL = 128 / BITS;  // codes per 16-byte chunk
  static constexpr int PAIRS = PER / 2;   // fp16 pairs per word
  static constexpr int BIAS = 1 << (BITS - 1);
  // Codes of pair i sit at mantissa bit p = pair_pow(i) of the magic halves.
  // Pairs with equal p form a class and share one (q - z) constant.
  static constexpr int NCLS = BITS == 2 ? 5 : (BITS == 4 ? 2 : 1);
  static constexpr __device__ int cls(int i) {
    return BITS == 8 ? 0 : (BITS == 4 ? (i & 1) : (i < 5 ? i : i - 5));
  }
  static constexpr __device__ int class_pow(int c) { return BITS == 4 ? 4 * c : 2 * c; }
};

// 0x64006400 held in a VGPR: with it in a register the masking below is one
// v_and_or_b32 (gfx9 VOP3 encodings take no literal constants, so with both
// constants literal the compiler would need a v_and_b32 plus a v_or_b32).
__device__ __forceinline__ uint32_t magic_vgpr() {
  uint32_t m;
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(m));
  return m;
}

// Word -> PER/2 magic pairs: both fp16 halves of pair i are 1024 + q * 2^p,
// the low half from slot i, the high half from slot i + PER/2.
template <int BITS>
__device__ __forceinline__ void magic_pairs(uint32_t w, uint32_t magic, uint32_t* p) {
  if constexpr (BITS == 8) {
    p[0] = __builtin_amdgcn_perm(0x64646464u, w, 0x04020400u);  // {0x64, b2, 0x64, b0}
    p[1] = __builtin_amdgcn_perm(0x64646464u, w, 0x04030401u);  // {0x64, b3, 0x64, b1}
  } else if constexpr (BITS == 4) {
    p[0] = (w & 0x000F000Fu) | magic;
    p[1] = (w & 0x00F000F0u) | magic;
    const uint32_t w8 = w >> 8;
    p[2] = (w8 & 0x000F000Fu) | magic;
    p[3] = (w8 & 0x00F000F0u) | magic;
  } else {
#pragma unroll
    for (int i = 0; i < 5; ++i) p[i] = (w & (0x00030003u << (2 * i))) | magic;
    const uint32_t w10 = w >> 10;
#pragma unroll
    for (int i = 0; i < 3; ++i) p[5 + i] = (w10 & (0x00030003u << (2 * i))) | magic;
  }
}

// ------------------------------------------------------------ wave reduction
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false));
}

// Sums over the 64 lanes of a wave, for N values at once (interleaving the N
// chains hides the DPP read-after-write wait states); totals land in lane 63.
template <int N>
__device__ __forceinline__ void wave_sum_lane63(float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_move<0x111, 0xf>(v[i]);  // row_shr:1
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_move<0x112, 0xf>(v[i]);  // row_shr:2
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_move<0x114, 0xf>(v[i]);  // row_shr:4
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_move<0x118, 0xf>(v[i]);  // row_shr:8: lane 16r+15 has row r
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_move<0x142, 0xa>(v[i]);  // row_bcast:15 into rows 1, 3
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_move<0x143, 0xc>(v[i]);  // row_bcast:31 into rows 2, 3
}

// Sums over the 64 lanes of a wave for R = 4 or 8 values, halving the values
// per lane at each exchange. The gfx950 permlane32 swap of (a, b) leaves
// a = rows {0, 1} of a then of b and b = rows {2, 3} of a then of b;
// permlane16 leaves a = rows (a0, b0, a2, b2) and b = (a1, b1, a3, b3).
// Swapping value i with value i + R/2 and adding gives, in lanes 0-31, value
// i summed over both halves of the wave and, in lanes 32-63, value i + R/2;
// the permlane16 swap of i with i + R/4 then leaves row g holding value
// i + g R/4 summed over its four lane-sets, and four in-row DPP steps finish.
// Lane 16 g + 15 ends with the totals of values g R/4 + i in v[i],
// i < R/4: 5R/4 + 4 instructions where wave_sum_lane63 takes 6R.
template <int R>
__device__ __forceinline__ void wave_sum_rows(float (&v)[R]) {
  static_assert(R == 4 || R == 8, "rows per tile");
#pragma unroll
  for (int i = 0; i < R / 2; ++i) {
    const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v[i]),
                                                    __builtin_bit_cast(uint32_t, v[i + R / 2]), false, false);
    const uint32_t a = p[0], b = p[1];  // element by element: see swap_sum16
    v[i] = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
  }
#pragma unroll
  for (int i = 0; i < R / 4; ++i) {
    const auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v[i]),
                                                    __builtin_bit_cast(uint32_t, v[i + R / 4]), false, false);
    const uint32_t a = p[0], b = p[1];
    v[i] = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
  }
#pragma unroll
  for (int i = 0; i < R / 4; ++i) v[i] += dpp_move<0x111, 0xf>(v[i]);  // row_shr:1
#pragma unroll
  for (int i = 0; i < R / 4; ++i) v[i] += dpp_move<0x112, 0xf>(v[i]);  // row_shr:2
#pragma unroll
  for (int i = 0; i < R / 4; ++i) v[i] += dpp_move<0x114, 0xf>(v[i]);  // row_shr:4
#pragma unroll
  for (int i = 0; i < R / 4; ++i) v[i] += dpp_move<0x118, 0xf>(v[i]);  // row_shr:8: lane 16g+15
}

// ---------------------------------------------------------------------- gemv
constexpr int kGemvThreads = 256;  // 4 waves
constexpr int kWavesPerBlock = kGemvThreads / 64;
constexpr uint32_t kBufferConfig = 0x00020000u;  // raw 32-bit buffer view (gfx9 descriptor word 3)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           static_cast<int>(kBufferConfig));
}

// Activation pair i of a word: (x[L(i)], x[L(i + PER/2)]) from the word's
// PER halves held as PER/2 dwords d[]; one v_perm_b32 unless the pair is
// already a dword (interleaved layouts).
template <int BITS, bool INTER>
__device__ __forceinline__ void x_pairs_from_dwords(const uint32_t* d, h2* xp) {
  using F = Fmt<BITS>;
#pragma unroll
  for (int i = 0; i < F::PAIRS; ++i) {
    const int lo = logical_of_slot<BITS, INTER>(i);
    const int hi = logical_of_slot<BITS, INTER>(i + F::PAIRS);
    if ((lo & 1) == 0 && hi == lo + 1) {
      xp[i] = as_h2(d[lo >> 1]);
    } else {
      const uint32_t sel = ((hi & 1) ? 0x07060000u : 0x05040000u) | ((lo & 1) ? 0x0302u : 0x0100u);
      xp[i] = as_h2(__builtin_amdgcn_perm(d[hi >> 1], d[lo >> 1], sel));
    }
  }
}

// Launch-wide description of up to kMaxBatch problems (passed by value). The
// host precomputes every quotient the kernel needs, so tile bookkeeping is
// shifts and adds.
struct KernelProblem {
  const uint32_t* qweight;
  const uint16_t* scales;
  const uint16_t* zeros;
  const uint16_t* x;
  uint16_t* y;
  const uint16_t* aux;   // prologue operand (gamma [K] or up [M, K]); unused without one
  int N, K;
  int n_groups;          // K / group_size
  int chunks_per_group;  // group_size / (128/BITS)
  int cpg_shift;         // log2(chunks_per_group) when a power of two, else -1
  int n_chunks;          // K / (128/BITS)
  int lwk;               // log2 of the waves sharing one tile along K (wk = 1, 2 or 4)
  int per_wave;          // ceil(n_chunks / wk): chunks of one wave's share
  int tiles;             // ceil(N / R)
  int ldy;               // row stride of y in elements (N unless the problem is a row slice of a larger one)
};

struct KernelBatch {
  KernelProblem p[kMaxBatch];
  int bt_start[kMaxBatch + 1];  // prefix sums of block-tiles (4/wk tiles each); blocks never mix problems
  int count;
  int M;
  float eps;  // RMSNorm prologue epsilon
  int run;    // gemv_m1_kernel<..., kXmKeep>: block-tiles per run of the walk
};

// Where block-tile `bt` of the launch sits, as seen by one wave. All fields
// are wave-uniform. The issue/load/math helpers below cover the chunks
// [cb, ce) only up to CMAX 16-byte columns per lane: callers split longer
// ranges into batches of 64 * CMAX chunks.
struct TilePos {
  int p;        // problem
  int row0;     // first row of this wave's tile
  int cb, ce;   // chunk range [cb, ce) of this wave (its share of K)
  int kw, wk;   // this wave's share index and the number of shares
  int active;   // the block-tile has a tile for this wave (an int: a struct copy then carries no padding bytes)
};

// `p` is the problem of the previous block-tile of this block (block-tiles
// are visited in increasing order, so the search only moves forward).
__device__ __forceinline__ TilePos locate(const KernelBatch& b, int bt, int wave, int R, int& p) {
  TilePos t;
  while (p + 1 < b.count && bt >= b.bt_start[p + 1]) ++p;
  const KernelProblem& d = b.p[p];
  t.p = p;
  t.wk = 1 << d.lwk;
  const int slot = wave >> d.lwk;
  t.kw = wave & (t.wk - 1);
  const int tile = ((bt - b.bt_start[p]) << (2 - d.lwk)) + slot;  // 4 / wk tiles per block-tile
  t.active = tile < d.tiles;
  t.row0 = tile * R;
  t.cb = t.kw * d.per_wave;
  t.ce = min(d.n_chunks, t.cb + d.per_wave);
  return t;
}

// Buffer offset of 16-byte column c of a batch, or an out-of-range offset
// (loads return zeros, nothing is read) for lanes past the wave's share.
constexpr uint32_t kOutOfRange = 0x80000000u;
__device__ __forceinline__ uint32_t column_offset(int c, int ce, uint32_t bytes_per_column) {
  return c < ce ? static_cast<uint32_t>(c) * bytes_per_column : kOutOfRange;
}

// Group of chunk c: a shift when chunks_per_group is a power of two
// (including every per-channel K that is one), else a division.
__device__ __forceinline__ uint32_t group_of(const KernelProblem& d, int c) {
  if (d.cpg_shift >= 0) return static_cast<uint32_t>(c) >> d.cpg_shift;
  return static_cast<uint32_t>(c) / static_cast<uint32_t>(d.chunks_per_group);
}

// The descriptor fields the M = 1 walks read per batch, copied one by one
// when a walk reaches a tile, so that they stay in registers across its
// batches (read through the kernel arguments instead, they were loaded, and
// waited on, every batch; gemv_mx_pipe_kernel, measured about 1% slower
// with the copy, keeps indexing). A whole-struct copy carried around the
// loop left the fields the walk never reads in a stack slot, which the
// compiler then placed in LDS (10 -> 20 KiB per block, written and read
// every batch).
__device__ __forceinline__ void take_problem(KernelProblem& dst, const KernelProblem& src) {
  dst.qweight = src.qweight;
  dst.scales = src.scales;
  dst.zeros = src.zeros;
  dst.x = src.x;
  dst.y = src.y;
  dst.aux = src.aux;
  dst.N = src.N;
  dst.K = src.K;
  dst.n_groups = src.n_groups;
  dst.chunks_per_group = src.chunks_per_group;
  dst.cpg_shift = src.cpg_shift;
  dst.n_chunks = src.n_chunks;
  dst.per_wave = src.per_wave;
  dst.ldy = src.ldy;
}

// The loads of one tile: R rows x CMAX 16-byte chunk columns per lane, plus
// the rows' fp16 scales (and zeros) of those chunks.
template <int BITS, int R, int CMAX>
struct TileLoads {
  u32x4 w[CMAX][R];
  // fp16 bit patterns, zero-extended: 16-bit elements invite the vectorizer
  // to pair neighbours into <2 x half> reads, which pins the struct in memory
  uint32_t s[CMAX][R];
  uint32_t z[CMAX][R];
};

// The loads of one M = 1 tile batch: zero points first, then scales,
// then weights. vmcnt retires in issue order, so the math of row r starts as
// soon as weight row r has arrived.
template <int BITS, bool SYM, int R>
__device__ __forceinline__ void issue_tile_m1(const KernelProblem& d, const TilePos& t, int lane,
                                              TileLoads<BITS, R, 1>& L) {
  const uint32_t row_bytes = static_cast<uint32_t>(d.K) * BITS / 8;
  const uint32_t meta_row_bytes = static_cast<uint32_t>(d.n_groups) * 2;
  const __amdgpu_buffer_rsrc_t wbuf = buffer_of(d.qweight, static_cast<uint32_t>(d.N) * row_bytes);
  const __amdgpu_buffer_rsrc_t sbuf = buffer_of(d.scales, static_cast<uint32_t>(d.N) * meta_row_bytes);
  const __amdgpu_buffer_rsrc_t zbuf = buffer_of(SYM ? d.scales : d.zeros, static_cast<uint32_t>(d.N) * meta_row_bytes);
  const int c = t.cb + lane;
  const uint32_t woff = column_offset(c, t.ce, 16u);
  const uint32_t moff = c < t.ce ? group_of(d, c) * 2u : kOutOfRange;
  uint32_t rowv[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rowv[r] = static_cast<uint32_t>(min(t.row0 + r, d.N - 1));  // past N: re-read N-1
#pragma unroll
  for (int r = 0; r < R; ++r)
    L.z[0][r] = SYM ? 0u : __builtin_amdgcn_raw_buffer_load_b16(zbuf, moff, rowv[r] * meta_row_bytes, 0);
#pragma unroll
  for (int r = 0; r < R; ++r) L.s[0][r] = __builtin_amdgcn_raw_buffer_load_b16(sbuf, moff, rowv[r] * meta_row_bytes, 0);
#pragma unroll
  for (int r = 0; r < R; ++r) L.w[0][r] = __builtin_amdgcn_raw_buffer_load_b128(wbuf, woff, rowv[r] * row_bytes, 2);
}

// Activation pairs of CMAX chunk columns of one batch row, in pair order.
template <int BITS, bool INTER, int CMAX>
__device__ __forceinline__ void load_x_columns(const KernelProblem& d, const TilePos& t, int lane, int m,
                                               h2 (&xr)[CMAX][4][Fmt<BITS>::PAIRS]) {
  using F = Fmt<BITS>;
  const __amdgpu_buffer_rsrc_t xbuf = buffer_of(d.x, static_cast<uint32_t>(m + 1) * static_cast<uint32_t>(d.K) * 2);
  const uint32_t mrow = static_cast<uint32_t>(m) * static_cast<uint32_t>(d.K) * 2;
#pragma unroll
  for (int ct = 0; ct < CMAX; ++ct) {
    const uint32_t xoff = column_offset(t.cb + lane + 64 * ct, t.ce, F::CPL * 2u);
    uint32_t xd[F::CPL / 2];
#pragma unroll
    for (int q = 0; q < F::CPL / 8; ++q) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xbuf, xoff + 16u * q, mrow, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) xd[4 * q + e] = v[e];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) x_pairs_from_dwords<BITS, INTER>(xd + j * (F::PER / 2), xr[ct][j]);
  }
}

// Activation prologues fused into the GEMV (one choice per launch):
//   kProNone     x as given;
//   kProRmsNorm  RMSNorm folded in: the activation pairs are x * gamma (fp16
//                products; gamma = aux, [K]) and ssq accumulates sum(x^2) in
//                fp32 over the wave's chunks; each row's dot product is
//                multiplied by 1/sqrt(sum(x^2)/K + eps) when its tile finishes
//                (the factor is common to the whole row of the product);
//   kProSwiGlu   SwiGLU folded in: x is the gate projection's output and aux
//                the up projection's ([M, K]); the pairs are
//                fp16(fp16(silu(gate)) * up) with silu(g) = g / (1 + e^-g) in
//                fp32, the roundings of the unfused fp16 ops.
enum : int { kProNone = 0, kProRmsNorm = kPrologueRmsNorm, kProSwiGlu = kPrologueSwiGlu };

__device__ __forceinline__ _Float16 silu_h(_Float16 g) {
  const float gf = static_cast<float>(g);
  const float e = __builtin_amdgcn_exp2f(-gf * 1.4426950408889634f);  // e^-g
  return static_cast<_Float16>(gf * __builtin_amdgcn_rcpf(1.0f + e));
}

__device__ __forceinline__ uint32_t swiglu_pair(uint32_t g, uint32_t u) {
  const h2 gh = as_h2(g);
  const h2 sh = h2{silu_h(gh.x), silu_h(gh.y)};
  return __builtin_bit_cast(uint32_t, sh * as_h2(u));  // fp16 product: the exact product rounded once
}

// Raw activation (and prologue operand) dwords of one chunk column per lane
// for batch row m: loads only, so they can be issued ahead of the tile's.
template <int BITS, int PRO>
struct XRaw {
  uint32_t x[Fmt<BITS>::CPL / 2];
  uint32_t a[PRO == kProNone ? 1 : Fmt<BITS>::CPL / 2];
};

template <int BITS, int PRO>
__device__ __forceinline__ void issue_x_pro(const KernelProblem& d, const TilePos& t, int lane, int m, int M,
                                            XRaw<BITS, PRO>& R) {
  using F = Fmt<BITS>;
  const uint32_t kb = static_cast<uint32_t>(d.K) * 2u;
  const __amdgpu_buffer_rsrc_t xbuf = buffer_of(d.x, static_cast<uint32_t>(M) * kb);
  const __amdgpu_buffer_rsrc_t abuf = buffer_of(d.aux, (PRO == kProSwiGlu ? static_cast<uint32_t>(M) : 1u) * kb);
  const uint32_t xoff = column_offset(t.cb + lane, t.ce, F::CPL * 2u);
  const uint32_t mrow = static_cast<uint32_t>(m) * kb;
#pragma unroll
  for (int q = 0; q < F::CPL / 8; ++q) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xbuf, xoff + 16u * q, mrow, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) R.x[4 * q + e] = v[e];
  }
  if constexpr (PRO != kProNone) {
#pragma unroll
    for (int q = 0; q < F::CPL / 8; ++q) {
      const u32x4 v =
          __builtin_amdgcn_raw_buffer_load_b128(abuf, xoff + 16u * q, PRO == kProSwiGlu ? mrow : 0u, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) R.a[4 * q + e] = v[e];
    }
  }
}

// The prologue's arithmetic on loaded dwords, then the pair order of the math.
template <int BITS, bool INTER, int PRO>
__device__ __forceinline__ void x_pairs_pro(XRaw<BITS, PRO>& R, h2 (&xr)[4][Fmt<BITS>::PAIRS], float& ssq) {
  using F = Fmt<BITS>;
#pragma unroll
  for (int i = 0; i < F::CPL / 2; ++i) {
    if constexpr (PRO == kProRmsNorm) {
      ssq = __builtin_amdgcn_fdot2(as_h2(R.x[i]), as_h2(R.x[i]), ssq, false);
      R.x[i] = __builtin_bit_cast(uint32_t, as_h2(R.x[i]) * as_h2(R.a[i]));
    } else if constexpr (PRO == kProSwiGlu) {
      R.x[i] = swiglu_pair(R.x[i], R.a[i]);
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) x_pairs_from_dwords<BITS, INTER>(R.x + j * (F::PER / 2), xr[j]);
}

// Reduce the R per-lane partial sums of a tile and store y. Block-wide LDS
// combine when the tile's K is split over wk > 1 waves (`part` is this
// iteration's half of a double buffer, so one barrier per tile suffices).
// After wave_sum_rows the tile's R outputs sit R/4 to a lane in lanes
// 15, 31, 47 and 63, which store them with one instruction (four lanes, one
// 4-byte store each at R = 8): R two-byte stores from a single lane were a
// third of the M = 1 kernel's memory instructions on 2 KiB rows.
// Rows r .. r + Q - 1 of y from one lane (Q = 1 or 2): one 4-byte store when
// both rows exist and y + r is aligned for it.
template <int Q>
__device__ __forceinline__ void store_rows(uint16_t* y, int r, int N, const float* v) {
  uint16_t* dst = y + r;
  if constexpr (Q == 2) {
    if (r + 2 <= N && (reinterpret_cast<uintptr_t>(dst) & 3) == 0) {
      *reinterpret_cast<uint32_t*>(dst) =
          static_cast<uint32_t>(f32_to_f16_rn(v[0])) | (static_cast<uint32_t>(f32_to_f16_rn(v[1])) << 16);
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < Q; ++i)
    if (r + i < N) dst[i] = f32_to_f16_rn(v[i]);
}

template <int R>
__device__ __forceinline__ void finish_tile(const KernelProblem& d, const TilePos& t, int wave, int lane,
                                            float (&yacc)[R], float (*part)[R]) {
  constexpr int Q = R / 4;  // rows per holder lane 16 g + 15, from row g Q of the tile
  wave_sum_rows<R>(yacc);
  const bool holder = (lane & 15) == 15;
  const int g = lane >> 4;
  if (t.wk == 1) {
    if (t.active && holder) store_rows<Q>(d.y, t.row0 + g * Q, d.N, yacc);
  } else {
    if (holder) {
#pragma unroll
      for (int i = 0; i < Q; ++i) part[wave][g * Q + i] = yacc[i];
    }
    __syncthreads();  // all 4 waves of the block run the same block-tile sequence
    if (t.active && t.kw == 0 && lane < R) {
      float v = 0.f;
      for (int j = 0; j < t.wk; ++j) v += part[wave + j][lane];
      if (t.row0 + lane < d.N) d.y[t.row0 + lane] = f32_to_f16_rn(v);
    }
  }
}

// ------------------------------------------------------------- gemv, M = 1
// The M = 1 hot path. Same tile walk and loads as gemv_kernel, with the math
// specialized for one activation row.
//
// Biased codes. A code masked into the mantissa of an fp16 half at bit p,
// under exponent field 25 - p, reads exactly 2^(10-p) + q (the half's value
// is 2^(10-p) * (1 + q 2^p / 2^10)); one v_and_or_b32 per pair then makes the
// fp16 operands and no multiply is needed. The bias and the zero point come
// off per row and chunk in fp32:
//   sum_k (q_k - z) x_k = sum_k (bias_k + q_k) x_k - (C + z S),
//   S = sum_k x_k,  C = sum_k bias_k x_k,
// with S and C taken once per lane and batch (the activations are shared by
// the tile's R rows). Every product is exact (fp16 operands, fp32 products)
// and the sums run in fp32; the bias terms cancel in the subtraction, so the
// sums' rounding error grows with the bias. The codes are therefore placed
// high in the mantissa:
//   INT4  every nibble at bit 4 (bias 64), from w << 4, w, w >> 4, w >> 8;
//   INT2  codes at bits 8 / 6 (bias 4 / 16), from w << 8, w << 4, w, w >> 4,
//         w >> 6;
//   INT8  the byte at bit 0 (bias 1024), by byte permutation.
// A CPU model of this summation order puts its error at under a quarter of
// the fp32 budget of the reference's kernel test (2^-20 sum |w||x|, its
// scripts/test_dequant_kernel.py:112-122; exact (q - z) products: ~1%) on
// the Llama shapes, and with that test's fp16 output term, under a third of
// its tolerance down to K = 128 (INT2: under a half). INT2's 2-bit codes
// gain least from a bias: with |q - z| <= 2 the earlier placement at bits
// 4 / 6 / 8 (bias 64 / 16 / 4, two shifts fewer per word) exceeded that
// tolerance up to 4.4x at K = 128 and 3.3x at K = 256 (rows whose codes sit
// mostly at the zero point), and a GPU test hit 2.4x at K = 128; every code
// at bit 8 (bias 4, 0.3x) took three shifts more per word than the current
// placement and cost the INT2 stacks 10%. The
// form holds for any zero point (the packer's zeros are unclamped,
// packer.py:136-137), so there is no separate path for large zero points.
//   * MF = false: products and sums with v_dot2_f32_f16 (VALU);
//     MF = true:  the dot products go to the matrix cores. The 64 lanes form
//     the 16 blocks of v_mfma_f32_4x4x4_16b_f16, four consecutive chunk
//     columns of one row each; with A = the lane's own activations and B =
//     its own biased codes, register (lane % 4) of the 4x4 result holds the
//     lane's own dot product (the diagonal), so the load pattern stays one
//     contiguous 1 KiB row segment per wave and load.
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ h4 cat2(h2 a, h2 b) { return __builtin_shufflevector(a, b, 0, 1, 2, 3); }

// Pair i of a word holds slots i and i + PER/2 (the pair order of
// x_pairs_from_dwords); its codes sit at mantissa bit pow(cls(i)).
template <int BITS> struct Biased {
  static constexpr int NCLS = BITS == 2 ? 2 : 1;
  static constexpr __device__ int cls(int i) { return BITS == 2 && (i == 1 || i == 3 || i == 5) ? 1 : 0; }
  static constexpr int pow(int c) { return BITS == 8 ? 0 : (BITS == 4 ? 4 : (c == 0 ? 8 : 6)); }
  static constexpr float bias(int c) { return static_cast<float>(1 << (10 - pow(c))); }
  static constexpr uint32_t magic(int c) {
    const uint32_t e = static_cast<uint32_t>(25 - pow(c));
    return (e << 10) | (e << 26);
  }
};

template <uint32_t V>
__device__ __forceinline__ uint32_t vgpr_const() {
  uint32_t m;
  asm volatile("v_mov_b32 %0, %1" : "=v"(m) : "i"(V));
  return m;
}

// The class magics held in VGPRs (as magic_vgpr, so that each pair is one
// v_and_or_b32 with the mask as its one scalar operand).
template <int BITS>
struct ClassMagics {
  uint32_t m[Biased<BITS>::NCLS];
  __device__ __forceinline__ void init() {
    m[0] = vgpr_const<Biased<BITS>::magic(0)>();
    if constexpr (Biased<BITS>::NCLS > 1) m[1] = vgpr_const<Biased<BITS>::magic(1)>();
    if constexpr (Biased<BITS>::NCLS > 2) m[2] = vgpr_const<Biased<BITS>::magic(2)>();
  }
};

// Word -> PER/2 biased pairs: both halves of pair i are bias + q, the low
// half from slot i, the high half from slot i + PER/2. Each half's codes sit
// at the same offsets, and no mask reaches bits a shift carried across the
// halves' boundary.
template <int BITS>
__device__ __forceinline__ void biased_pairs(uint32_t w, const ClassMagics<BITS>& cm, uint32_t* p) {
  if constexpr (BITS == 8) {
    p[0] = __builtin_amdgcn_perm(0x64646464u, w, 0x04020400u);  // {0x64, b2, 0x64, b0}: 1024 + q
    p[1] = __builtin_amdgcn_perm(0x64646464u, w, 0x04030401u);
  } else if constexpr (BITS == 4) {
    constexpr uint32_t kNib = 0x00F000F0u;  // bits 4-7 of each half
    p[0] = ((w << 4) & kNib) | cm.m[0];
    p[1] = (w & kNib) | cm.m[0];
    p[2] = ((w >> 4) & kNib) | cm.m[0];
    p[3] = ((w >> 8) & kNib) | cm.m[0];
  } else {
    // slot i sits at bit 2i of the low half and slot i + 8 at the same offset
    // of the high half: one shift moves both, to bit 8 (class 0) or 6 (class 1)
    constexpr uint32_t k8 = 0x03000300u, k6 = 0x00C000C0u;
    const uint32_t w8 = w << 8, w4 = w << 4, r4 = w >> 4, r6 = w >> 6;
    p[0] = (w8 & k8) | cm.m[0];  // slot 0: bit 0 -> 8
    p[1] = (w4 & k6) | cm.m[1];  // slot 1: bit 2 -> 6
    p[2] = (w4 & k8) | cm.m[0];  // slot 2: bit 4 -> 8
    p[3] = (w & k6) | cm.m[1];   // slot 3: bit 6
    p[4] = (w & k8) | cm.m[0];   // slot 4: bit 8
    p[5] = (r4 & k6) | cm.m[1];  // slot 5: bit 10 -> 6
    p[6] = (r4 & k8) | cm.m[0];  // slot 6: bit 12 -> 8
    p[7] = (r6 & k8) | cm.m[0];  // slot 7: bit 14 -> 8
  }
}

// S = sum(x) and C = sum(bias * x) over the lane's chunk, per class with
// v_dot2 against ones (exact products, fp32 sums).
template <int BITS>
__device__ __forceinline__ void bias_sums(const h2 (&xr)[4][Fmt<BITS>::PAIRS], float& S, float& C) {
  using F = Fmt<BITS>;
  using B = Biased<BITS>;
  const h2 one = splat(static_cast<_Float16>(1.0f));
  float sc[B::NCLS];
#pragma unroll
  for (int c = 0; c < B::NCLS; ++c) sc[c] = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < F::PAIRS; ++i) sc[B::cls(i)] = __builtin_amdgcn_fdot2(xr[j][i], one, sc[B::cls(i)], false);
  S = sc[0];
  C = B::bias(0) * sc[0];
#pragma unroll
  for (int c = 1; c < B::NCLS; ++c) {
    S += sc[c];
    C = __builtin_fmaf(B::bias(c), sc[c], C);
  }
}

// sum over the lane's chunk of (bias + q) x for one row.
template <int BITS, bool MF>
__device__ __forceinline__ float biased_dot_m1(const u32x4& w, const h2 (&xr)[4][Fmt<BITS>::PAIRS],
                                               const ClassMagics<BITS>& cm, int lane) {
  using F = Fmt<BITS>;
  if constexpr (MF) {
    f4 D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t mp[F::PAIRS];
      biased_pairs<BITS>(w[j], cm, mp);
#pragma unroll
      for (int i = 0; i < F::PAIRS; i += 2)
        D = __builtin_amdgcn_mfma_f32_4x4x4f16(cat2(xr[j][i], xr[j][i + 1]), cat2(as_h2(mp[i]), as_h2(mp[i + 1])), D,
                                               0, 0, 0);
    }
    const bool s1 = lane & 1, s2 = lane & 2;
    return s2 ? (s1 ? D[3] : D[2]) : (s1 ? D[1] : D[0]);
  } else {
    float v = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t mp[F::PAIRS];
      biased_pairs<BITS>(w[j], cm, mp);
#pragma unroll
      for (int i = 0; i < F::PAIRS; ++i) v = __builtin_amdgcn_fdot2(as_h2(mp[i]), xr[j][i], v, false);
    }
    return v;
  }
}

// One batch of a tile, given the batch's bias sums S and C:
// acc[r] = scale_r * (sum (bias + q) x - (C + z_r S)).
template <int BITS, bool SYM, int R, bool MF>
__device__ __forceinline__ void tile_math_m1_sums(const TileLoads<BITS, R, 1>& L,
                                                  const h2 (&xr)[4][Fmt<BITS>::PAIRS], float S, float C,
                                                  const ClassMagics<BITS>& cm, int lane, float (&acc)[R]) {
  using F = Fmt<BITS>;
  if constexpr (SYM) C = __builtin_fmaf(static_cast<float>(F::BIAS), S, C);  // z = 2^(b-1) for every row
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float corr = SYM ? C : __builtin_fmaf(f16_to_f32(static_cast<uint16_t>(L.z[0][r])), S, C);
    const float v = biased_dot_m1<BITS, MF>(L.w[0][r], xr, cm, lane) - corr;
    acc[r] = __builtin_fmaf(f16_to_f32(static_cast<uint16_t>(L.s[0][r])), v, acc[r]);
  }
}

template <int BITS, bool SYM, bool INTER, int R, bool MF>
__device__ __forceinline__ void tile_math_m1(const TileLoads<BITS, R, 1>& L, const h2 (&xr)[4][Fmt<BITS>::PAIRS],
                                             const ClassMagics<BITS>& cm, int lane, float (&acc)[R]) {
  float S, C;
  bias_sums<BITS>(xr, S, C);
  tile_math_m1_sums<BITS, SYM, R, MF>(L, xr, S, C, cm, lane, acc);
}

// finish_tile for the RMSNorm prologue: the R dot products and the wave's
// sum(x^2) are reduced together (and combined over the wk waves of a split
// K), then y = dot / sqrt(sum(x^2) / K + eps).
__device__ __forceinline__ float inv_rms(float ssq, int K, float eps) {
  return 1.0f / __builtin_sqrtf(ssq / static_cast<float>(K) + eps);
}

template <int R>
__device__ __forceinline__ void finish_tile_rms(const KernelProblem& d, const TilePos& t, int wave, int lane, float eps,
                                                const float (&yacc)[R], float ssq, float (*part)[R + 1]) {
  constexpr int Q = R / 4;  // rows per holder lane 16 g + 15, from row g Q of the tile
  float v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) v[r] = yacc[r];
  wave_sum_rows<R>(v);
  float sq[1] = {ssq};
  wave_sum_lane63<1>(sq);  // the wave's sum(x^2) in lane 63, then in every lane
  const float q = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sq[0]), 63));
  const bool holder = (lane & 15) == 15;
  const int g = lane >> 4;
  if (t.wk == 1) {
    const float f = inv_rms(q, d.K, eps);
    float o[Q];
#pragma unroll
    for (int i = 0; i < Q; ++i) o[i] = v[i] * f;
    if (t.active && holder) store_rows<Q>(d.y, t.row0 + g * Q, d.N, o);
  } else {
    if (holder) {
#pragma unroll
      for (int i = 0; i < Q; ++i) part[wave][g * Q + i] = v[i];
    }
    if (lane == 63) part[wave][R] = q;
    __syncthreads();  // all 4 waves of the block run the same block-tile sequence
    if (t.active && t.kw == 0 && lane < R) {
      float a = 0.f, q = 0.f;
      for (int j = 0; j < t.wk; ++j) {
        a += part[wave + j][lane];
        q += part[wave + j][R];
      }
      if (t.row0 + lane < d.N) d.y[t.row0 + lane] = f32_to_f16_rn(a * inv_rms(q, d.K, eps));
    }
  }
}

// Workgroup barrier for LDS traffic only. Its release / acquire fences are
// scoped to LDS, so a wave waits for its own LDS writes (lgkmcnt) but not for
// its global loads in flight; __syncthreads() fences every address space,
// i.e. waits for all of the wave's outstanding global loads before the
// barrier (checked in the generated code: vmcnt(0) there, only lgkmcnt(0)
// here).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Where an M = 1 launch's activations come from (gemv_m1_kernel's XM):
//   kXmLoad   every wave loads each batch's activations;
//   kXmKeep   tiles of one batch, each block walking a contiguous range of
//             block-tiles: a wave keeps the activation pairs of its last tile
//             in its own LDS slot (8 KiB for INT2) and their bias sums in
//             registers, and loads x again only when a tile reads other
//             columns or another x (the q | k | v and gate | up problems of a
//             layer share x, so most tiles of a long range reuse them).
enum : int { kXmLoad = 0, kXmKeep = 2 };

template <int BITS, bool SYM, bool INTER, int R, bool MF, int PRO, int XM>
__global__ void __launch_bounds__(kGemvThreads)
gemv_m1_kernel(const KernelBatch b) {
  using F = Fmt<BITS>;
  constexpr bool KEEP = XM == kXmKeep;
  static_assert(!KEEP || (PRO == kProNone && !MF), "kept activations: plain VALU launches");
  constexpr int PW = PRO == kProRmsNorm ? R + 1 : R;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  __shared__ float part[2][kWavesPerBlock][PW];
  ClassMagics<BITS> cm;
  cm.init();
  const int total = b.bt_start[b.count];
  int phase = 0;
  int p = 0;
  // block-tiles in runs of `run` consecutive ones, the runs strided over the
  // grid: run = 1 is the plain grid-stride walk. KEEP walks runs of b.run
  // (kKeepRun), so a wave's consecutive tiles are neighbours while the
  // block-tiles in flight across the chip stay one compact span of the launch
  // (a contiguous share per block spread them over the whole launch and cost
  // 7.7% on the C4 INT2 stack before any reuse)
  const int run = KEEP ? b.run : 1;
  // KEEP: the pairs (in this wave's LDS slot) and bias sums of the last
  // activations this wave loaded, and the x and chunk columns they came from
  __shared__ u32x4 xkeep[KEEP ? kWavesPerBlock * F::PAIRS * 64 : 1];
  float Sk = 0.f, Ck = 0.f;
  bool have = false;
  const void* kx = nullptr;
  int kcb = 0, kce = 0;
  int bt = static_cast<int>(blockIdx.x) * run;  // run r, element j: (r * gridDim.x + blockIdx.x) * run + j
  int in_run = 0;
  while (bt < total) {
    const TilePos t = locate(b, bt, wave, R, p);
    KernelProblem dl{};  // the tile's problem (take_problem; the fields it does not copy stay zero)
    take_problem(dl, b.p[t.p]);
    const KernelProblem& d = dl;
    float yacc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) yacc[r] = 0.f;
    float ssq = 0.f;  // RMSNorm prologue: this wave's sum(x^2)
    if (t.active) {
      for (int cbase = t.cb; cbase < t.ce; cbase += 64) {
        TilePos tb = t;
        tb.cb = cbase;
        tb.ce = min(t.ce, cbase + 64);
        // activations first: vmcnt retires in issue order and every row's
        // math needs them, so with them last no row could start before the
        // whole tile had arrived
        h2 xr[1][4][F::PAIRS];
        XRaw<BITS, PRO> raw;
        TileLoads<BITS, R, 1> L;
        if constexpr (KEEP) {
          // the tile's one batch (tb == t); a fresh load keeps the order of
          // the path below (activations first), the pairs replace the kept ones
          u32x4* kept = xkeep + wave * F::PAIRS * 64;  // piece q of lane l at q * 64 + l
          if (!have || d.x != kx || tb.cb != kcb || tb.ce != kce) {
            load_x_columns<BITS, INTER, 1>(d, tb, lane, 0, xr);
            issue_tile_m1<BITS, SYM, R>(d, tb, lane, L);
            __builtin_amdgcn_sched_barrier(0);
            bias_sums<BITS>(xr[0], Sk, Ck);
#pragma unroll
            for (int q = 0; q < F::PAIRS; ++q) {
              u32x4 v;
#pragma unroll
              for (int e = 0; e < 4; ++e)
                v[e] = __builtin_bit_cast(uint32_t, xr[0][(4 * q + e) / F::PAIRS][(4 * q + e) % F::PAIRS]);
              kept[q * 64 + lane] = v;
            }
            have = true;
            kx = d.x;
            kcb = tb.cb;
            kce = tb.ce;
          } else {
            // one wave's own LDS slot: its reads follow its earlier writes in order
#pragma unroll
            for (int q = 0; q < F::PAIRS; ++q) {
              const u32x4 v = kept[q * 64 + lane];
#pragma unroll
              for (int e = 0; e < 4; ++e) xr[0][(4 * q + e) / F::PAIRS][(4 * q + e) % F::PAIRS] = as_h2(v[e]);
            }
            issue_tile_m1<BITS, SYM, R>(d, tb, lane, L);
            __builtin_amdgcn_sched_barrier(0);
          }
        } else {
          if constexpr (PRO == kProNone)
            load_x_columns<BITS, INTER, 1>(d, tb, lane, 0, xr);
          else
            issue_x_pro<BITS, PRO>(d, tb, lane, 0, 1, raw);
          issue_tile_m1<BITS, SYM, R>(d, tb, lane, L);
          // keep every load of the batch ahead of its math: left alone, the
          // scheduler sinks the weight loads into the math to save registers,
          // leaving one or two rows in flight and the latency exposed per row
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (PRO != kProNone) x_pairs_pro<BITS, INTER, PRO>(raw, xr[0], ssq);
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.f;
        if constexpr (KEEP)
          tile_math_m1_sums<BITS, SYM, R, MF>(L, xr[0], Sk, Ck, cm, lane, acc);
        else
          tile_math_m1<BITS, SYM, INTER, R, MF>(L, xr[0], cm, lane, acc);
#pragma unroll
        for (int r = 0; r < R; ++r) yacc[r] += acc[r];
      }
    }
    if constexpr (PRO == kProRmsNorm)
      finish_tile_rms<R>(d, t, wave, lane, b.eps, yacc, ssq, part[phase]);
    else
      finish_tile<R>(d, t, wave, lane, yacc, part[phase]);
    if (t.wk > 1) phase ^= 1;
    if constexpr (KEEP) {
      if (++in_run == run) {
        in_run = 0;
        bt += (static_cast<int>(gridDim.x) - 1) * run + 1;
      } else {
        ++bt;
      }
    } else {
      bt += gridDim.x;
    }
  }
}

// ------------------------------------- gemv, M = 1, software-pipelined walk
// The M = 1 kernel above issues a batch's loads, then computes it: while a
// wave does its math it has no load in flight, so the bytes in flight per CU
// (what sets the achieved bandwidth once HBM latency is queue-bound) fall
// with the VALU time. This kernel keeps a batch in flight at all times with
// the same registers: row r of the next batch (which may belong to the next
// tile of the wave's walk, or to another problem) is issued as soon as row r
// of the current batch has been computed.
//
// Activations: the block stages each batch's 64 chunk columns once in LDS,
// already in pair order (thread t forms the pairs of word t % 4 of column
// t / 4), double-buffered, one LDS-only barrier per batch (the weight loads
// stay in flight across it). A wave reads its pairs with ds_read_b128 when a
// batch starts, so the next batch's activations need no second set of
// registers while the current batch's math runs (that set would drop the
// kernel to four waves per SIMD), and the pairs are formed once per block
// instead of once per wave.
//
// Launches whose tiles are one wave wide (wk = 1): the four waves of a block
// then walk the same batches of the same block-tiles (block-tiles never mix
// problems), so every wave meets every barrier; a wave whose slot of a
// block-tile is empty walks its batches with out-of-range loads and stores
// nothing.

// Load addressing of one batch: descriptors and row offsets are wave-uniform
// (SGPRs), the chunk-column offsets per lane. Rows of an empty slot and every
// load of a batch past the walk's end get out-of-range offsets: they return
// zeros and read nothing.
template <int R>
struct BatchAddr {
  __amdgpu_buffer_rsrc_t wbuf, sbuf, zbuf;
  uint32_t woff, moff;
  uint32_t wrow[R], mrow[R];
};

template <int BITS, bool SYM, int R>
__device__ __forceinline__ void batch_addr(const KernelProblem& d, int row0, int cbase, int ce, int lane, bool live,
                                           BatchAddr<R>& a) {
  const uint32_t row_bytes = static_cast<uint32_t>(d.K) * BITS / 8;
  const uint32_t meta_row_bytes = static_cast<uint32_t>(d.n_groups) * 2;
  a.wbuf = buffer_of(d.qweight, static_cast<uint32_t>(d.N) * row_bytes);
  a.sbuf = buffer_of(d.scales, static_cast<uint32_t>(d.N) * meta_row_bytes);
  a.zbuf = buffer_of(SYM ? d.scales : d.zeros, static_cast<uint32_t>(d.N) * meta_row_bytes);
  const int c = cbase + lane;
  const bool in = live && c < min(ce, cbase + 64);
  a.woff = in ? static_cast<uint32_t>(c) * 16u : kOutOfRange;
  a.moff = in ? group_of(d, c) * 2u : kOutOfRange;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t row = static_cast<uint32_t>(min(row0 + r, d.N - 1));  // past N: re-read N-1
    a.wrow[r] = row * row_bytes;
    a.mrow[r] = row * meta_row_bytes;
  }
}

template <bool SYM, int R>
__device__ __forceinline__ void issue_row(const BatchAddr<R>& a, int r, uint32_t& z, uint32_t& s, u32x4& w) {
  if constexpr (!SYM) z = __builtin_amdgcn_raw_buffer_load_b16(a.zbuf, a.moff, a.mrow[r], 0);
  s = __builtin_amdgcn_raw_buffer_load_b16(a.sbuf, a.moff, a.mrow[r], 0);
  w = __builtin_amdgcn_raw_buffer_load_b128(a.wbuf, a.woff, a.wrow[r], 2);
}

// One batch's activations in LDS, in pair order: chunk column c at
// c * kStride (a 16-byte pad per column spreads a wave's reads over the
// banks); thread t of the block forms word t % 4 of column t / 4.
template <int BITS>
struct PairStage {
  using F = Fmt<BITS>;
  static constexpr int kWordBytes = F::PER * 2;        // one word's activations (= its pairs)
  static constexpr int kColumnBytes = F::CPL * 2;      // 4 words
  static constexpr int kStride = kColumnBytes + 16;
  static constexpr int kBufBytes = 64 * kStride;
  static constexpr int kWordDwords = kWordBytes / 4;   // PER / 2
};

// Thread t's word of the batch starting at column cbase (columns >= ce and a
// batch past the walk's end load zeros): from x, or from the RMSNorm
// prologue's gamma (same layout, one row).
template <int BITS>
__device__ __forceinline__ void pair_stage_issue(const void* base, const KernelProblem& d, int cbase, int ce,
                                                 bool live, uint32_t (&raw)[PairStage<BITS>::kWordDwords]) {
  using PS = PairStage<BITS>;
  const __amdgpu_buffer_rsrc_t xbuf = buffer_of(base, static_cast<uint32_t>(d.K) * 2u);
  const int t = static_cast<int>(threadIdx.x);
  const int c = cbase + (t >> 2);
  const uint32_t off = live && c < ce ? static_cast<uint32_t>(c) * PS::kColumnBytes + (t & 3) * PS::kWordBytes
                                      : kOutOfRange;
  if constexpr (PS::kWordDwords == 2) {
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(xbuf, off, 0, 0);
    raw[0] = v[0];
    raw[1] = v[1];
  } else {
#pragma unroll
    for (int q = 0; q < PS::kWordDwords / 4; ++q) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xbuf, off + 16u * q, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) raw[4 * q + e] = v[e];
    }
  }
}

// The RMSNorm prologue on a staged word: the thread's sum(x^2) in fp32 (one
// v_dot2 per dword), then x * gamma as fp16 products (the arithmetic of
// x_pairs_pro).
template <int BITS>
__device__ __forceinline__ void pair_stage_rmsnorm(uint32_t (&raw)[PairStage<BITS>::kWordDwords],
                                                   const uint32_t (&gam)[PairStage<BITS>::kWordDwords],
                                                   float& ssq) {
#pragma unroll
  for (int i = 0; i < PairStage<BITS>::kWordDwords; ++i) {
    ssq = __builtin_amdgcn_fdot2(as_h2(raw[i]), as_h2(raw[i]), ssq, false);
    raw[i] = __builtin_bit_cast(uint32_t, as_h2(raw[i]) * as_h2(gam[i]));
  }
}

// The SwiGLU prologue on a staged word: x is the gate projection's output,
// the operand the up projection's (the arithmetic of x_pairs_pro).
template <int BITS>
__device__ __forceinline__ void pair_stage_swiglu(uint32_t (&raw)[PairStage<BITS>::kWordDwords],
                                                  const uint32_t (&up)[PairStage<BITS>::kWordDwords]) {
#pragma unroll
  for (int i = 0; i < PairStage<BITS>::kWordDwords; ++i) raw[i] = swiglu_pair(raw[i], up[i]);
}

template <int BITS, bool INTER>
__device__ __forceinline__ void pair_stage_write(unsigned char* buf, const uint32_t (&raw)[PairStage<BITS>::kWordDwords]) {
  using PS = PairStage<BITS>;
  h2 xp[Fmt<BITS>::PAIRS];
  x_pairs_from_dwords<BITS, INTER>(raw, xp);
  const int t = static_cast<int>(threadIdx.x);
  unsigned char* dst = buf + (t >> 2) * PS::kStride + (t & 3) * PS::kWordBytes;
  if constexpr (PS::kWordDwords == 2) {
    *reinterpret_cast<u32x2*>(dst) = u32x2{__builtin_bit_cast(uint32_t, xp[0]), __builtin_bit_cast(uint32_t, xp[1])};
  } else {
#pragma unroll
    for (int q = 0; q < PS::kWordDwords / 4; ++q) {
      u32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = __builtin_bit_cast(uint32_t, xp[4 * q + e]);
      *reinterpret_cast<u32x4*>(dst + 16 * q) = v;
    }
  }
}

template <int BITS>
__device__ __forceinline__ void pair_stage_read(const unsigned char* buf, int lane, h2 (&xr)[4][Fmt<BITS>::PAIRS]) {
  using F = Fmt<BITS>;
  using PS = PairStage<BITS>;
  const unsigned char* src = buf + lane * PS::kStride;
#pragma unroll
  for (int k = 0; k < PS::kColumnBytes / 16; ++k) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(src + 16 * k);
#pragma unroll
    for (int e = 0; e < 4; ++e) xr[(4 * k + e) / F::PAIRS][(4 * k + e) % F::PAIRS] = as_h2(v[e]);
  }
}

// PRO = kProRmsNorm: the staging threads apply the RMSNorm prologue to the
// words they stage (x * gamma, and their fp32 sum(x^2) accumulated over the
// tile's batches: every activation of the tile's K is staged once per
// block-tile, by one thread); at the tile's end the block sums those partial
// sums (every tile of a block-tile shares x) and each row's dot product is
// multiplied by 1 / sqrt(sum(x^2) / K + eps) before the fp16 store.
// PRO = kProSwiGlu: the staging threads form silu(gate) * up of the words
// they stage (x = gate, aux = up), once per block and batch instead of once
// per tile and lane.
template <int BITS, bool SYM, bool INTER, int R, int PRO = kProNone>
__global__ void __launch_bounds__(kGemvThreads)
gemv_m1_pipe_kernel(const KernelBatch b) {
  using F = Fmt<BITS>;
  using PS = PairStage<BITS>;
  constexpr bool RMS = PRO == kProRmsNorm;
  constexpr bool SWI = PRO == kProSwiGlu;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  __shared__ __align__(16) unsigned char xs[2 * PS::kBufBytes];
  __shared__ float rms_part[kWavesPerBlock];
  float ssq = 0.f;  // RMS: this thread's sum(x^2) over the current tile's staged words
  ClassMagics<BITS> cm;
  cm.init();
  const int total = b.bt_start[b.count];
  int p = 0;
  int bt = static_cast<int>(blockIdx.x);
  if (bt >= total) return;  // block-uniform: the whole block leaves
  TilePos t = locate(b, bt, wave, R, p);
  KernelProblem dc{};  // the tile's problem (take_problem; the fields it does not copy stay zero)
  take_problem(dc, b.p[p]);
  int cb = t.cb;
  int par = 0;
  BatchAddr<R> a;
  uint32_t raw[PS::kWordDwords], gam[RMS || SWI ? PS::kWordDwords : 1];  // gam: gamma or up
  uint32_t z[R], s[R];
  u32x4 w[R];
  // the first batch: activations staged, rows in flight
  pair_stage_issue<BITS>(dc.x, dc, cb, t.ce, true, raw);
  if constexpr (RMS || SWI) pair_stage_issue<BITS>(dc.aux, dc, cb, t.ce, true, gam);
  batch_addr<BITS, SYM, R>(dc, t.row0, cb, t.ce, lane, t.active, a);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    issue_row<SYM, R>(a, r, z[r], s[r], w[r]);
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (RMS) pair_stage_rmsnorm<BITS>(raw, gam, ssq);
  if constexpr (SWI) pair_stage_swiglu<BITS>(raw, gam);
  pair_stage_write<BITS, INTER>(xs, raw);
  lds_barrier();
  float yacc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) yacc[r] = 0.f;
  for (;;) {
    // where the next batch is: the next 64 columns of this tile, or the
    // first batch of the next block-tile (the same for the whole block)
    int ncb = cb + 64;
    int nbt = bt, np = p;
    TilePos nt = t;
    KernelProblem dn{};
    take_problem(dn, dc);
    const bool tile_end = ncb >= t.ce;
    if (tile_end) {
      nbt = bt + static_cast<int>(gridDim.x);
      if (nbt < total) {
        nt = locate(b, nbt, wave, R, np);
        ncb = nt.cb;
        take_problem(dn, b.p[np]);
      }
    }
    const bool nvalid = nbt < total;  // block-uniform
    // the current batch's pairs and bias sums
    h2 xr[4][F::PAIRS];
    pair_stage_read<BITS>(xs + par * PS::kBufBytes, lane, xr);
    float S, C;
    bias_sums<BITS>(xr, S, C);
    if constexpr (SYM) C = __builtin_fmaf(static_cast<float>(F::BIAS), S, C);
    // the next batch's activations (issued first: vmcnt retires in order),
    // then its rows as the current ones free their registers
    pair_stage_issue<BITS>(dn.x, dn, ncb, nt.ce, nvalid, raw);
    if constexpr (RMS || SWI) pair_stage_issue<BITS>(dn.aux, dn, ncb, nt.ce, nvalid, gam);
    batch_addr<BITS, SYM, R>(dn, nt.row0, ncb, nt.ce, lane, nvalid && nt.active, a);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float corr = SYM ? C : __builtin_fmaf(f16_to_f32(static_cast<uint16_t>(z[r])), S, C);
      const float v = biased_dot_m1<BITS, false>(w[r], xr, cm, lane) - corr;
      yacc[r] = __builtin_fmaf(f16_to_f32(static_cast<uint16_t>(s[r])), v, yacc[r]);
      issue_row<SYM, R>(a, r, z[r], s[r], w[r]);  // row r of the next batch, into the freed registers
      __builtin_amdgcn_sched_barrier(0);
    }
    if (tile_end) {
      wave_sum_rows<R>(yacc);
      if constexpr (RMS) {
        // the block-tile's sum(x^2): every staging thread's partial sum of its
        // words (computed once per block and activation vector instead, for
        // the problems of a launch that share x, it made the decode step 0.4%
        // faster and cost the 8-row instance a wave per SIMD)
        float sq[1] = {ssq};
        wave_sum_lane63<1>(sq);
        if (lane == 63) rms_part[wave] = sq[0];
        lds_barrier();  // every wave of the block ends its tile here
        const float f = inv_rms(rms_part[0] + rms_part[1] + rms_part[2] + rms_part[3], dc.K, b.eps);
#pragma unroll
        for (int i = 0; i < R / 4; ++i) yacc[i] *= f;
        ssq = 0.f;
      }
      if (t.active && (lane & 15) == 15)
        store_rows<R / 4>(dc.y, t.row0 + (lane >> 4) * (R / 4), dc.N, yacc);
#pragma unroll
      for (int r = 0; r < R; ++r) yacc[r] = 0.f;
    }
    if (!nvalid) break;
    par ^= 1;
    if constexpr (RMS) pair_stage_rmsnorm<BITS>(raw, gam, ssq);
    if constexpr (SWI) pair_stage_swiglu<BITS>(raw, gam);
    pair_stage_write<BITS, INTER>(xs + par * PS::kBufBytes, raw);
    lds_barrier();  // the other buffer was read before the previous barrier
    cb = ncb;
    bt = nbt;
    p = np;
    t = nt;
    take_problem(dc, dn);
  }
}

// gemv_m1_pipe_kernel's walk for launches that split K over WK = 2 or 4
// waves per tile (no prologue): a block-tile holds 4 / WK tiles, wave w
// takes share w % WK of tile w / WK, and every share of a block-tile has
// the same ceil(per_wave / 64) batches (a shorter last share loads zeros
// past its end). The block stages each batch's activations of all WK
// shares (WK words per thread, WK buffers per parity); each wave reads its
// share's buffer, so the activations are loaded once per block, not once per
// lane as in gemv_m1_kernel's split launches. At a tile's end the shares'
// sums meet in LDS (double-buffered by tile, an LDS-only barrier: the next
// batch's rows stay in flight) and share 0 adds them in share order and
// stores.
template <int BITS, bool SYM, bool INTER, int R, int WK>
__global__ void __launch_bounds__(kGemvThreads)
gemv_m1_pipe_split_kernel(const KernelBatch b) {
  static_assert(WK == 2 || WK == 4, "K shares per tile");
  using F = Fmt<BITS>;
  using PS = PairStage<BITS>;
  constexpr int Q = R / 4;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  __shared__ __align__(16) unsigned char xs[2 * WK * PS::kBufBytes];
  __shared__ float part[2][kWavesPerBlock][R];
  ClassMagics<BITS> cm;
  cm.init();
  const int total = b.bt_start[b.count];
  int p = 0;
  int bt = static_cast<int>(blockIdx.x);
  if (bt >= total) return;  // block-uniform: the whole block leaves
  TilePos t = locate(b, bt, wave, R, p);
  KernelProblem dc{};  // the tile's problem (take_problem; the fields it does not copy stay zero)
  take_problem(dc, b.p[p]);
  int j = 0;  // batch of the current tile (block-uniform)
  int par = 0, phase = 0;
  BatchAddr<R> a;
  uint32_t raw[WK][PS::kWordDwords];
  uint32_t z[R], s[R];
  u32x4 w[R];
  // share sh's word of batch jj of problem d (all threads of the block)
  const auto stage_issue = [&](const KernelProblem& d, int jj, bool live) {
#pragma unroll
    for (int sh = 0; sh < WK; ++sh) {
      const int c0 = sh * d.per_wave;
      pair_stage_issue<BITS>(d.x, d, c0 + 64 * jj, min(d.n_chunks, c0 + d.per_wave), live, raw[sh]);
    }
  };
  const auto stage_write = [&](int pa) {
#pragma unroll
    for (int sh = 0; sh < WK; ++sh) pair_stage_write<BITS, INTER>(xs + (pa * WK + sh) * PS::kBufBytes, raw[sh]);
  };
  // the first batch: activations staged, rows in flight
  stage_issue(dc, 0, true);
  batch_addr<BITS, SYM, R>(dc, t.row0, t.cb, t.ce, lane, t.active, a);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    issue_row<SYM, R>(a, r, z[r], s[r], w[r]);
    __builtin_amdgcn_sched_barrier(0);
  }
  stage_write(0);
  lds_barrier();
  float yacc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) yacc[r] = 0.f;
  for (;;) {
    // where the next batch is: batch j + 1 of this tile, or the first batch
    // of the next block-tile (the same for the whole block)
    const int nb = (dc.per_wave + 63) >> 6;
    int nj = j + 1, nbt = bt, np = p;
    TilePos nt = t;
    KernelProblem dn{};
    take_problem(dn, dc);
    const bool tile_end = nj >= nb;
    if (tile_end) {
      nj = 0;
      nbt = bt + static_cast<int>(gridDim.x);
      if (nbt < total) {
        nt = locate(b, nbt, wave, R, np);
        take_problem(dn, b.p[np]);
      }
    }
    const bool nvalid = nbt < total;  // block-uniform
    h2 xr[4][F::PAIRS];
    pair_stage_read<BITS>(xs + (par * WK + t.kw) * PS::kBufBytes, lane, xr);
    float S, C;
    bias_sums<BITS>(xr, S, C);
    if constexpr (SYM) C = __builtin_fmaf(static_cast<float>(F::BIAS), S, C);
    stage_issue(dn, nj, nvalid);
    batch_addr<BITS, SYM, R>(dn, nt.row0, nt.cb + 64 * nj, nt.ce, lane, nvalid && nt.active, a);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float corr = SYM ? C : __builtin_fmaf(f16_to_f32(static_cast<uint16_t>(z[r])), S, C);
      const float v = biased_dot_m1<BITS, false>(w[r], xr, cm, lane) - corr;
      yacc[r] = __builtin_fmaf(f16_to_f32(static_cast<uint16_t>(s[r])), v, yacc[r]);
      issue_row<SYM, R>(a, r, z[r], s[r], w[r]);  // row r of the next batch
      __builtin_amdgcn_sched_barrier(0);
    }
    if (tile_end) {
      wave_sum_rows<R>(yacc);
      const int g = lane >> 4;
      if ((lane & 15) == 15) {
#pragma unroll
        for (int i = 0; i < Q; ++i) part[phase][wave][g * Q + i] = yacc[i];
      }
      lds_barrier();  // every wave of the block ends its tile here
      if (t.active && t.kw == 0 && (lane & 15) == 15) {
        float o[Q];
#pragma unroll
        for (int i = 0; i < Q; ++i) {
          float v = 0.f;
#pragma unroll
          for (int sh = 0; sh < WK; ++sh) v += part[phase][wave + sh][g * Q + i];
          o[i] = v;
        }
        store_rows<Q>(dc.y, t.row0 + g * Q, dc.N, o);
      }
      phase ^= 1;
#pragma unroll
      for (int r = 0; r < R; ++r) yacc[r] = 0.f;
    }
    if (!nvalid) break;
    par ^= 1;
    stage_write(par);
    lds_barrier();  // the other buffer was read before the previous barrier
    j = nj;
    bt = nbt;
    p = np;
    t = nt;
    take_problem(dc, dn);
  }
}

// Batches of 2 <= M <= MX rows (the launcher uses MX = 2) on gemv_m1_pipe_kernel's walk:
// each weight row's biased pairs are formed once per chunk and dotted with
// every batch row's activations (v_dot2, one fp32 chain per row and batch
// row, the M = 1 kernel's arithmetic), the activations of all MX batch rows
// staged per block as there (MX buffers per batch, double-buffered) and the
// bias sums S, C taken per batch row. One-wave tiles only: launches that
// split K run gemv_quad_kernel. Batch rows past M load zeros and store
// nothing.
template <int BITS, bool SYM, bool INTER, int R, int MX>
__global__ void __launch_bounds__(kGemvThreads) gemv_mx_pipe_kernel(const KernelBatch b) {
  using F = Fmt<BITS>;
  using PS = PairStage<BITS>;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  __shared__ __align__(16) unsigned char xs[2 * MX * PS::kBufBytes];
  ClassMagics<BITS> cm;
  cm.init();
  const int total = b.bt_start[b.count];
  int p = 0;
  int bt = static_cast<int>(blockIdx.x);
  if (bt >= total) return;  // block-uniform: the whole block leaves
  TilePos t = locate(b, bt, wave, R, p);
  int cb = t.cb;
  int par = 0;
  BatchAddr<R> a;
  uint32_t raw[MX][PS::kWordDwords];
  uint32_t z[R], s[R];
  u32x4 w[R];
  auto stage_issue = [&](const KernelProblem& d, int cbase, int ce, bool live) {
#pragma unroll
    for (int m = 0; m < MX; ++m)
      pair_stage_issue<BITS>(d.x + static_cast<int64_t>(m) * d.K, d, cbase, ce, live && m < b.M, raw[m]);
  };
  auto stage_write = [&](int parity) {
#pragma unroll
    for (int m = 0; m < MX; ++m) pair_stage_write<BITS, INTER>(xs + (parity * MX + m) * PS::kBufBytes, raw[m]);
  };
  // the first batch: activations staged, rows in flight
  stage_issue(b.p[t.p], cb, t.ce, true);
  batch_addr<BITS, SYM, R>(b.p[t.p], t.row0, cb, t.ce, lane, t.active, a);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    issue_row<SYM, R>(a, r, z[r], s[r], w[r]);
    __builtin_amdgcn_sched_barrier(0);
  }
  stage_write(0);
  lds_barrier();
  float yacc[MX][R];
#pragma unroll
  for (int m = 0; m < MX; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) yacc[m][r] = 0.f;
  for (;;) {
    // where the next batch is: the next 64 columns of this tile, or the
    // first batch of the next block-tile (the same for the whole block)
    int ncb = cb + 64;
    int nbt = bt, np = p;
    TilePos nt = t;
    const bool tile_end = ncb >= t.ce;
    if (tile_end) {
      nbt = bt + static_cast<int>(gridDim.x);
      if (nbt < total) {
        nt = locate(b, nbt, wave, R, np);
        ncb = nt.cb;
      }
    }
    const bool nvalid = nbt < total;  // block-uniform
    // the current batch's pairs and bias sums, per batch row
    h2 xr[MX][4][F::PAIRS];
    float S[MX], C[MX];
#pragma unroll
    for (int m = 0; m < MX; ++m) {
      pair_stage_read<BITS>(xs + (par * MX + m) * PS::kBufBytes, lane, xr[m]);
      bias_sums<BITS>(xr[m], S[m], C[m]);
      if constexpr (SYM) C[m] = __builtin_fmaf(static_cast<float>(F::BIAS), S[m], C[m]);
    }
    // the next batch's activations, then its rows as the current ones free their registers
    stage_issue(b.p[np], ncb, nt.ce, nvalid);
    batch_addr<BITS, SYM, R>(b.p[np], nt.row0, ncb, nt.ce, lane, nvalid && nt.active, a);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      uint32_t mp[4][F::PAIRS];
#pragma unroll
      for (int j = 0; j < 4; ++j) biased_pairs<BITS>(w[r][j], cm, mp[j]);
      const float zf = SYM ? 0.f : f16_to_f32(static_cast<uint16_t>(z[r]));
      const float sf = f16_to_f32(static_cast<uint16_t>(s[r]));
#pragma unroll
      for (int m = 0; m < MX; ++m) {
        float v = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < F::PAIRS; ++i) v = __builtin_amdgcn_fdot2(as_h2(mp[j][i]), xr[m][j][i], v, false);
        const float corr = SYM ? C[m] : __builtin_fmaf(zf, S[m], C[m]);
        yacc[m][r] = __builtin_fmaf(sf, v - corr, yacc[m][r]);
      }
      issue_row<SYM, R>(a, r, z[r], s[r], w[r]);  // row r of the next batch, into the freed registers
      __builtin_amdgcn_sched_barrier(0);
    }
    if (tile_end) {
      const KernelProblem& d = b.p[t.p];
#pragma unroll
      for (int m = 0; m < MX; ++m) {
        wave_sum_rows<R>(yacc[m]);
        if (m < b.M && t.active && (lane & 15) == 15)
          store_rows<R / 4>(d.y + static_cast<int64_t>(m) * d.ldy, t.row0 + (lane >> 4) * (R / 4), d.N, yacc[m]);
#pragma unroll
        for (int r = 0; r < R; ++r) yacc[m][r] = 0.f;
      }
    }
    if (!nvalid) break;
    par ^= 1;
    stage_write(par);
    lds_barrier();  // the other buffers were read before the previous barrier
    cb = ncb;
    bt = nbt;
    p = np;
    t = nt;
  }
}

// ------------------------------------------------ quad kernel, 2 <= M <= 8
// v_mfma_f32_4x4x4_16b_f16 computes 16 independent products D_b += A_b B_b
// (4x4 by 4x4); lane 4b + j supplies row j of A_b and column j of B_b and
// holds column j of D_b (register i = row i). Lane l = (b = l/4, q = l%4):
//   B  chunk cs + b (16 bytes, 128/BITS codes) of weight row row0 + 4g + q,
//      one register set per quad g of the tile, so one load instruction reads
//      4 rows x 256 contiguous bytes (as a pure read that pattern reaches
//      81% of peak; the 16 rows x 64 bytes of a 16x16x32 operand reach 70%);
//   A  the same chunk's activations of batch row 4mg + q (zeros past M);
//   D  lane (b, j), register i: sum over chunk cs + b of
//      x[4mg + i] * (q - z)[row0 + 4g + j].
// A chunk's MFMAs start from zero and acc += scale * D folds it in with its
// row's group scale in fp32: the reference's factorized arithmetic (exact
// (q - z) x products, fp32 sums, one scale per group), as in the VALU
// kernels, for any group size. The 16 blocks hold different chunks; their
// sum is taken once per tile (DPP row_ror 4 / 8 inside 16-lane rows, then the
// gfx950 permlane16 / permlane32 swaps across rows).
//
// Zero points outside [-1024, 1024] (WIDE, rare, asymmetric only): those rows
// use q alone and z * sum(x) is subtracted in fp32, sum(x) per chunk and
// batch row from one more MFMA chain against ones.
// Activations of one k-step for the whole block, staged in LDS: each step the
// block loads, for each of its wk K-shares, the 16 chunks of x the step
// covers (4*MG batch rows; one coalesced 16-byte piece per lane and load),
// and every wave reads its A fragments from there. Without the staging each
// wave loaded its own copy per step: as many bytes as its weights (M <= 4,
// INT4), and the load-class ablation put that at a third of the kernel's time.
// Double-buffered by step parity, one barrier per step. Rows are padded by 16
// bytes so the 16-byte fragment reads of a lane quad hit distinct banks.
template <int BITS, int MG, int WK>
struct QuadStage {
  static constexpr int kChunkBytes = Fmt<BITS>::CPL * 2;          // one row's activations of one chunk
  static constexpr int kPieces = kChunkBytes / 16;                  // 16-byte pieces per chunk
  static constexpr int kRowBytes = 16 * kChunkBytes + 16;          // one row's 16 chunks, padded
  static constexpr int kRows = 4 * MG;
  static constexpr int kBufBytes = WK * kRows * kRowBytes;
  static constexpr int kTotal = WK * kRows * 16 * kPieces;          // pieces per step
  static constexpr int kPerLane = (kTotal + kGemvThreads - 1) / kGemvThreads;
};

template <int BITS, int MG, int WK>
__device__ __forceinline__ void stage_issue(const KernelProblem& d, int M, int s, u32x4 (&st)[QuadStage<BITS, MG, WK>::kPerLane]) {
  using QS = QuadStage<BITS, MG, WK>;
  const uint32_t kb = static_cast<uint32_t>(d.K) * 2u;
  const __amdgpu_buffer_rsrc_t xbuf = buffer_of(d.x, static_cast<uint32_t>(M) * kb);
#pragma unroll
  for (int i = 0; i < QS::kPerLane; ++i) {
    const int e = static_cast<int>(threadIdx.x) + kGemvThreads * i;
    const int piece = e % QS::kPieces, cl = (e / QS::kPieces) % 16, r = e / (QS::kPieces * 16);
    const int m = r % QS::kRows, j = r / QS::kRows;
    const int c = j * d.per_wave + 16 * s + cl;
    const bool ok = e < QS::kTotal && m < M && c < min(d.n_chunks, (j + 1) * d.per_wave);
    st[i] = __builtin_amdgcn_raw_buffer_load_b128(
        xbuf, ok ? static_cast<uint32_t>(m) * kb + static_cast<uint32_t>(c) * QS::kChunkBytes + 16u * piece
                 : kOutOfRange,
        0, 0);
  }
}

template <int BITS, int MG, int WK>
__device__ __forceinline__ void stage_write(unsigned char* buf, const u32x4 (&st)[QuadStage<BITS, MG, WK>::kPerLane]) {
  using QS = QuadStage<BITS, MG, WK>;
#pragma unroll
  for (int i = 0; i < QS::kPerLane; ++i) {
    const int e = static_cast<int>(threadIdx.x) + kGemvThreads * i;
    const int piece = e % QS::kPieces, cl = (e / QS::kPieces) % 16, r = e / (QS::kPieces * 16);
    if (e < QS::kTotal)
      *reinterpret_cast<u32x4*>(buf + r * QS::kRowBytes + cl * QS::kChunkBytes + 16 * piece) = st[i];
  }
}

// Sum of v over the 16 lanes sharing l % 4, returned in lanes 0..15 (row 0;
// the other rows get partial sums). The gfx950 permlane swaps exchange rows
// with a zero operand, so one output of each swap is the moved row and the
// other zeros: (even rows += odd rows), then (lower half += upper half).
// The pair a swap returns is copied out element by element into named
// values: used directly inside __builtin_bit_cast, this clang reads element
// 0 for both (checked in its LLVM IR).
__device__ __forceinline__ float swap_sum16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), 0u, false, false);
  const uint32_t a = r[0], b = r[1];
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float swap_sum32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), 0u, false, false);
  const uint32_t a = r[0], b = r[1];
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float quad_column_sum(float v) {
  v += dpp_move<0x124, 0xf>(v);  // row_ror:4
  v += dpp_move<0x128, 0xf>(v);  // row_ror:8: every lane of a 16-lane row has its row's sum
  return swap_sum32(swap_sum16(v));
}

// ------------------------------------------ quad kernel: the tile walk
// Persistent blocks walk block-tiles like the M = 1 kernels; a tile is 4 * NT
// rows and the WK waves of a tile split its chunks (in steps of 16), meeting
// in LDS. Every problem of a launch uses WK waves per tile (the staging layout
// holds WK K-shares). The walk keeps the next step in flight during the
// current step's math with the same registers, as gemv_m1_pipe_kernel does
// at M = 1: quad g of the next step (which may belong to the next tile of the
// walk, or to another problem) is issued as soon as quad g of the current
// step has been computed, the next step's activations are loaded before the
// math and written to the other staging buffer after it, and the per-step
// barrier orders LDS only (a __syncthreads would wait for the next step's
// loads too). Measured against the same kernel with a step's loads issued
// at the step and a __syncthreads per step: C2 at M = 4 15.3 -> 14.7 us per
// call, the C4 stack at M = 2 / 4 / 8 unchanged (52-54 / 51 / 39% in that
// A/B): those launches are not bound by one step's load latency.
// Zero points outside [-1024, 1024] (asymmetric only) are handled in the
// same pass: those rows use q alone and subtract z * sum(x), sum(x) per
// chunk taken (one more MFMA chain against ones) only in steps where a wave
// has such a row; every other row subtracts 0 * 0. A row's result does not
// depend on the other rows' zero points.
// The tile's problem descriptor is copied into registers when the walk
// reaches the tile: indexed by the step's problem instead, its fields were
// read back from the kernel arguments every step, five scalar-load round
// trips per step (C2 at M = 4: 13.5 -> 12.8-12.9 us per call, the C4 M = 8
// stack 1-4% faster). (The M = 1 walks copy field by field instead, see
// take_problem: a whole-struct copy placed their unread fields in LDS.)
template <int NT>
struct QuadAddr {
  __amdgpu_buffer_rsrc_t wbuf, sbuf, zbuf;
  uint32_t woff[NT], moff[NT];  // per lane: row and chunk column offsets, or out of range
};

template <int BITS, bool SYM, int NT>
__device__ __forceinline__ void quad_addr(const KernelProblem& d, const TilePos& t, int s, int blk, int q, bool live,
                                          QuadAddr<NT>& a) {
  const uint32_t row_bytes = static_cast<uint32_t>(d.K) * BITS / 8;
  const uint32_t meta_row = static_cast<uint32_t>(d.n_groups) * 2u;
  a.wbuf = buffer_of(d.qweight, static_cast<uint32_t>(d.N) * row_bytes);
  a.sbuf = buffer_of(d.scales, static_cast<uint32_t>(d.N) * meta_row);
  a.zbuf = buffer_of(SYM ? d.scales : d.zeros, static_cast<uint32_t>(d.N) * meta_row);
  const int c = t.cb + 16 * s + blk;
  const bool ok = live && t.active && c < t.ce;
  const uint32_t gmo = ok ? group_of(d, c) * 2u : 0u;
#pragma unroll
  for (int g = 0; g < NT; ++g) {
    const uint32_t n = static_cast<uint32_t>(min(t.row0 + 4 * g + q, d.N - 1));  // past N: re-read, never stored
    a.woff[g] = ok ? n * row_bytes + static_cast<uint32_t>(c) * 16u : kOutOfRange;
    a.moff[g] = ok ? n * meta_row + gmo : kOutOfRange;
  }
}

template <bool SYM, int NT>
__device__ __forceinline__ void quad_issue(const QuadAddr<NT>& a, int g, uint32_t& z, uint32_t& s, u32x4& w) {
  if constexpr (!SYM) z = __builtin_amdgcn_raw_buffer_load_b16(a.zbuf, a.moff[g], 0, 0);
  s = __builtin_amdgcn_raw_buffer_load_b16(a.sbuf, a.moff[g], 0, 0);
  w = __builtin_amdgcn_raw_buffer_load_b128(a.wbuf, a.woff[g], 0, 2);
}

// acc += scale * sum over the lane's chunk of x (q - z) for one quad of one
// step; WIDE: rows whose zero point is outside [-1024, 1024] use q alone and
// subtract z * xs (xs: sum(x) per chunk).
template <int BITS, bool SYM, int MG, bool WIDE>
__device__ __forceinline__ void quad_math(const u32x4& w, uint32_t zb, uint32_t sb,
                                          const h2 (&xp)[MG][Fmt<BITS>::CPL / 2], const f4 (&xs)[MG],
                                          const h2 (&pow_scale)[Fmt<BITS>::NCLS], uint32_t magic, f4 (&acc)[MG]) {
  using F = Fmt<BITS>;
  constexpr int CPL = F::CPL, NF = CPL / 4;
  _Float16 zh;
  bool exact = true;
  if constexpr (SYM) {
    zh = static_cast<_Float16>(static_cast<float>(F::BIAS));
  } else if constexpr (!WIDE) {
    zh = __builtin_bit_cast(_Float16, static_cast<uint16_t>(zb));
  } else {
    exact = (zb & 0x7FFFu) <= 0x6400u;
    zh = exact ? __builtin_bit_cast(_Float16, static_cast<uint16_t>(zb)) : static_cast<_Float16>(0.0f);
  }
  const h2 zz = splat(zh);
  h2 off[F::NCLS];
#pragma unroll
  for (int k = 0; k < F::NCLS; k += 2) {
    const _Float16 b0 = static_cast<_Float16>(static_cast<float>(1 << (10 - F::class_pow(k))));
    const _Float16 b1 =
        k + 1 < F::NCLS ? static_cast<_Float16>(static_cast<float>(1 << (10 - F::class_pow(k + 1)))) : b0;
    const h2 both = -(h2{b0, b1} + zz);
    off[k] = splat(both.x);
    if (k + 1 < F::NCLS) off[k + 1] = splat(both.y);
  }
  h2 dq[CPL / 2];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t mp[F::PAIRS];
    magic_pairs<BITS>(w[j], magic, mp);
#pragma unroll
    for (int i = 0; i < F::PAIRS; ++i)
      dq[j * F::PAIRS + i] = __builtin_elementwise_fma(as_h2(mp[i]), pow_scale[F::cls(i)], off[F::cls(i)]);
  }
  const float sc = f16_to_f32(static_cast<uint16_t>(sb));
#pragma unroll
  for (int mg = 0; mg < MG; ++mg) {
    f4 D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int f = 0; f < NF; ++f)
      D = __builtin_amdgcn_mfma_f32_4x4x4f16(cat2(xp[mg][2 * f], xp[mg][2 * f + 1]), cat2(dq[2 * f], dq[2 * f + 1]), D,
                                             0, 0, 0);
    if constexpr (WIDE) {
      const float zf = exact ? 0.0f : f16_to_f32(static_cast<uint16_t>(zb));
#pragma unroll
      for (int i = 0; i < 4; ++i) D[i] = __builtin_fmaf(-zf, xs[mg][i], D[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[mg][i] = __builtin_fmaf(sc, D[i], acc[mg][i]);
  }
}

// Two batch-row groups with one K share (the M = 5..8 launches of large
// problems, e.g. the C4 stack at M = 8) are asked to fit four waves per SIMD:
// 125 VGPRs without spills instead of 144 (three waves); the C4 M = 8 stack
// ran 34.7 / 35.3 -> 34.0 / 33.5 us/layer (same box, two alternations). The
// other instances keep the compiler's choice: asked the same, the INT2 ones
// and those with K shares spilled to scratch.
template <int BITS, bool SYM, bool INTER, int NT, int MG, int WK>
__global__ void __launch_bounds__(kGemvThreads)
__attribute__((amdgpu_waves_per_eu(BITS != 2 && MG == 2 && WK == 1 ? 4 : 1, 8)))
gemv_quad_kernel(const KernelBatch b) {
  using F = Fmt<BITS>;
  using QS = QuadStage<BITS, MG, WK>;
  constexpr int CPL = F::CPL, NF = CPL / 4;
  constexpr int NV = NT * MG * 4;  // outputs of one column q per tile: (g, mg, i)
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int blk = lane >> 2, q = lane & 3;
  __shared__ float part[2][kWavesPerBlock][NV][4];
  __shared__ __align__(16) unsigned char xlds[2 * QS::kBufBytes];
  const uint32_t magic = magic_vgpr();
  h2 pow_scale[F::NCLS];
#pragma unroll
  for (int c = 0; c < F::NCLS; ++c)
    pow_scale[c] = splat(static_cast<_Float16>(__builtin_ldexpf(1.0f, -F::class_pow(c))));
  const int total = b.bt_start[b.count];
  int bt = static_cast<int>(blockIdx.x);
  if (bt >= total) return;  // block-uniform: the whole block leaves
  int p = 0;
  TilePos t = locate(b, bt, wave, 4 * NT, p);
  KernelProblem dc = b.p[p];  // the tile's problem, held across its steps (reloaded when the walk moves on)
  int s = 0, par = 0, phase = 0;
  QuadAddr<NT> a;
  u32x4 st[QS::kPerLane];
  uint32_t zb[NT], sb[NT];
  u32x4 w[NT];
  // the first step: activations staged, quads in flight
  stage_issue<BITS, MG, WK>(dc, b.M, s, st);
  quad_addr<BITS, SYM, NT>(dc, t, s, blk, q, true, a);
#pragma unroll
  for (int g = 0; g < NT; ++g) {
    quad_issue<SYM, NT>(a, g, zb[g], sb[g], w[g]);
    __builtin_amdgcn_sched_barrier(0);
  }
  stage_write<BITS, MG, WK>(xlds, st);
  lds_barrier();
  f4 acc[NT][MG];
#pragma unroll
  for (int g = 0; g < NT; ++g)
#pragma unroll
    for (int mg = 0; mg < MG; ++mg) acc[g][mg] = f4{0.f, 0.f, 0.f, 0.f};
  for (;;) {
    // the next step: the next 16 chunk columns of this tile, or the first
    // step of the next block-tile (the same for the whole block)
    const int nsteps = dc.per_wave >> 4;
    int ns = s + 1, nbt = bt, np = p;
    TilePos nt = t;
    KernelProblem dn = dc;
    const bool tile_end = ns >= nsteps;
    if (tile_end) {
      ns = 0;
      nbt = bt + static_cast<int>(gridDim.x);
      if (nbt < total) {
        nt = locate(b, nbt, wave, 4 * NT, np);
        dn = b.p[np];
      }
    }
    const bool nvalid = nbt < total;  // block-uniform
    // the current step's activation pairs
    const unsigned char* buf = xlds + par * QS::kBufBytes;
    h2 xp[MG][CPL / 2];
#pragma unroll
    for (int mg = 0; mg < MG; ++mg) {
      uint32_t xd[CPL / 2];
#pragma unroll
      for (int k = 0; k < CPL / 8; ++k) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(buf + (t.kw * QS::kRows + 4 * mg + q) * QS::kRowBytes +
                                                        blk * QS::kChunkBytes + 16 * k);
#pragma unroll
        for (int e = 0; e < 4; ++e) xd[4 * k + e] = v[e];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) x_pairs_from_dwords<BITS, INTER>(xd + j * (F::PER / 2), xp[mg] + j * F::PAIRS);
    }
    // the next step's activations, then its quads as the current ones free their registers
    if (nvalid) stage_issue<BITS, MG, WK>(dn, b.M, ns, st);
    quad_addr<BITS, SYM, NT>(dn, nt, ns, blk, q, nvalid, a);
    __builtin_amdgcn_sched_barrier(0);
    // zero points outside [-1024, 1024] in any of the wave's rows of this
    // step (a wave-wide vote): sum(x) per chunk for their z * sum(x) term
    f4 xs[MG];
#pragma unroll
    for (int mg = 0; mg < MG; ++mg) xs[mg] = f4{0.f, 0.f, 0.f, 0.f};
    if constexpr (!SYM) {
      bool any = false;
#pragma unroll
      for (int g = 0; g < NT; ++g) any = any || (zb[g] & 0x7FFFu) > 0x6400u;
      if (__builtin_amdgcn_ballot_w64(any) != 0) {  // wave-uniform
        const h2 one = splat(static_cast<_Float16>(1.0f));
#pragma unroll
        for (int mg = 0; mg < MG; ++mg)
#pragma unroll
          for (int f = 0; f < NF; ++f)
            xs[mg] = __builtin_amdgcn_mfma_f32_4x4x4f16(cat2(xp[mg][2 * f], xp[mg][2 * f + 1]), cat2(one, one),
                                                        xs[mg], 0, 0, 0);
      }
    }
#pragma unroll
    for (int g = 0; g < NT; ++g) {
      quad_math<BITS, SYM, MG, !SYM>(w[g], zb[g], sb[g], xp, xs, pow_scale, magic, acc[g]);
      quad_issue<SYM, NT>(a, g, zb[g], sb[g], w[g]);  // quad g of the next step, into the freed registers
      __builtin_amdgcn_sched_barrier(0);
    }
    if (tile_end) {
      float tot[NV];
#pragma unroll
      for (int g = 0; g < NT; ++g)
#pragma unroll
        for (int mg = 0; mg < MG; ++mg)
#pragma unroll
          for (int i = 0; i < 4; ++i) tot[(g * MG + mg) * 4 + i] = quad_column_sum(acc[g][mg][i]);
      const KernelProblem& d = dc;
      // value v = (g, mg, i) is y[4 mg + i][row0 + 4 g + q]; lane (b = v % 4, q) of row 0 stores it
      if (t.wk == 1) {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          const int g = v / (MG * 4), m = 4 * ((v / 4) % MG) + (v % 4), n = t.row0 + 4 * g + q;
          if (blk == (v & 3) && t.active && m < b.M && n < d.N)
            d.y[static_cast<int64_t>(m) * d.ldy + n] = f32_to_f16_rn(tot[v]);
        }
      } else {
#pragma unroll
        for (int v = 0; v < NV; ++v)
          if (blk == (v & 3)) part[phase][wave][v][q] = tot[v];
        lds_barrier();  // all 4 waves of the block run the same step sequence
        if (t.active && t.kw == 0) {
#pragma unroll
          for (int v = 0; v < NV; ++v) {
            const int g = v / (MG * 4), m = 4 * ((v / 4) % MG) + (v % 4), n = t.row0 + 4 * g + q;
            if (blk == (v & 3) && m < b.M && n < d.N) {
              float sum = 0.f;
              for (int j = 0; j < t.wk; ++j) sum += part[phase][wave + j][v][q];
              d.y[static_cast<int64_t>(m) * d.ldy + n] = f32_to_f16_rn(sum);
            }
          }
        }
        phase ^= 1;
      }
#pragma unroll
      for (int g = 0; g < NT; ++g)
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) acc[g][mg] = f4{0.f, 0.f, 0.f, 0.f};
    }
    if (!nvalid) break;
    par ^= 1;
    stage_write<BITS, MG, WK>(xlds + par * QS::kBufBytes, st);
    lds_barrier();  // the other buffer was read before the previous barrier
    s = ns;
    bt = nbt;
    p = np;
    t = nt;
    dc = dn;
  }
}

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ h8 pack8(h2 a, h2 b, h2 c, h2 d) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  const h4 lo = __builtin_shufflevector(a, b, 0, 1, 2, 3);
  const h4 hi = __builtin_shufflevector(c, d, 0, 1, 2, 3);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// ---------------------------------------------------- small GEMM, M <= 64 (MFMA)
// y[m, n] = fp16( sum_k x[m, k] * W16[n, k] ) with W16 = fp16((q - z) * s),
// the fp16 weight packer.dequantize materializes (packer.py:177-189), built
// in registers: (q - z) exact in fp16 (as in the GEMV kernels) times the fp16
// scale with one v_pk_mul_f16 is the exact product rounded once to fp16, i.e.
// the same bits as dequantize's fp32 multiply and RNE store. So this computes
// the reference's M > 8 path (dequantize, then F.linear over the fp16 weight:
// quant_linear.py:131-132) in one pass over the packed bytes, with fp32
// accumulation on the matrix cores; only the summation order differs.
//
// v_mfma_f32_16x16x32_f16 with the activations as A (16 batch rows x 32 k)
// and W16 as B (32 k x 16 output columns), lane l = (kb = l/16, r = l%16):
//   B  8 weights of row n = row0 + r: fragment f of chunk 4t + kb
//   A  the matching 8 activations of batch row 16 mb + r
//   D  lane l holds y[16 mb + 4 kb + i][row0 + r], i = 0..3
// A tile is 16 rows; an iteration covers chunks 4t..4t+3 of them, and each of
// the MB activation tiles reuses the iteration's W16 fragments. Zero points
// outside [-1024, 1024] take W16 from fp32 arithmetic instead (wave-uniform
// branch, rare).
struct GemmProblem {
  const uint32_t* qweight;
  const uint16_t* scales;
  const uint16_t* zeros;
  const uint16_t* x;
  uint16_t* y;
  int N, K;
  int n_groups;   // K / group_size
  int cpg_shift;  // log2(chunks per group) when a power of two, else -1
  int cpg;        // chunks per group
  int n_chunks;   // K / (128/BITS)
  int n_iters;    // ceil(n_chunks / 4)
  int lwk;        // log2 of the waves sharing one tile along K
  int per_wave;   // ceil(n_iters / wk)
  int tiles;      // ceil(N / 16)
  int ldy;        // row stride of y in elements
  // gemm_walk_kernel's split along K across blocks
  int splits;     // blocks per column group (1: no split, y written directly)
  int ips;        // iterations per split (a multiple of kWalkDepth)
  int part_base;  // first partial tile of this problem in the scratch
};

struct GemmBatch {
  GemmProblem p[kMaxBatch];
  int bt_start[kMaxBatch + 1];
  int count;
  int M;
  float* part;     // split partial tiles (gemm_walk_kernel), or null
};

// W16 fragments of one lane's chunk (CPL codes = CPL/8 fragments of 8).
template <int BITS, bool SYM, bool WIDE>
__device__ __forceinline__ void w16_fragments(const u32x4& w, uint32_t sb, uint32_t zb, uint32_t magic,
                                              h8 (&wf)[Fmt<BITS>::CPL / 8]) {
  using F = Fmt<BITS>;
  constexpr int NP = F::CPL / 2;
  h2 dq[NP];
  if constexpr (!WIDE) {
    h2 pow_scale[F::NCLS];
#pragma unroll
    for (int c = 0; c < F::NCLS; ++c)
      pow_scale[c] = splat(static_cast<_Float16>(__builtin_ldexpf(1.0f, -F::class_pow(c))));
    const _Float16 zh = SYM ? static_cast<_Float16>(static_cast<float>(F::BIAS))
                            : __builtin_bit_cast(_Float16, static_cast<uint16_t>(zb));
    const h2 zz = splat(zh);
    h2 off[F::NCLS];
#pragma unroll
    for (int c = 0; c < F::NCLS; c += 2) {
      const _Float16 b0 = static_cast<_Float16>(static_cast<float>(1 << (10 - F::class_pow(c))));
      const _Float16 b1 =
          c + 1 < F::NCLS ? static_cast<_Float16>(static_cast<float>(1 << (10 - F::class_pow(c + 1)))) : b0;
      const h2 both = -(h2{b0, b1} + zz);
      off[c] = splat(both.x);
      if (c + 1 < F::NCLS) off[c + 1] = splat(both.y);
    }
    const h2 ss = splat(__builtin_bit_cast(_Float16, static_cast<uint16_t>(sb)));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t mp[F::PAIRS];
      magic_pairs<BITS>(w[j], magic, mp);
#pragma unroll
      for (int i = 0; i < F::PAIRS; ++i)
        dq[j * F::PAIRS + i] = __builtin_elementwise_fma(as_h2(mp[i]), pow_scale[F::cls(i)], off[F::cls(i)]) * ss;
    }
  } else {
    // fp32 (q - z) * s then fp16 RNE, dequantize_kernel's own arithmetic
    const float s = f16_to_f32(static_cast<uint16_t>(sb));
    const float z = SYM ? static_cast<float>(F::BIAS) : f16_to_f32(static_cast<uint16_t>(zb));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int i = 0; i < F::PAIRS; ++i) {
        const float qa = static_cast<float>((w[j] >> (BITS * i)) & ((1u << BITS) - 1u));
        const float qb = static_cast<float>((w[j] >> (BITS * (i + F::PAIRS))) & ((1u << BITS) - 1u));
        dq[j * F::PAIRS + i] = h2{static_cast<_Float16>(__fmul_rn(qa - z, s)), static_cast<_Float16>(__fmul_rn(qb - z, s))};
      }
    }
  }
#pragma unroll
  for (int f = 0; f < F::CPL / 8; ++f) wf[f] = pack8(dq[4 * f], dq[4 * f + 1], dq[4 * f + 2], dq[4 * f + 3]);
}

// 4 x 4 transpose over the four 16-lane rows of a wave: on entry register q
// of lane (row, i) holds element (q, row); on exit register j holds element
// (row, j) of the same lane position i. Two stages of gfx950 lane swaps:
// permlane32 swaps rows {2, 3} of one register with rows {0, 1} of another,
// permlane16 rows {1, 3} of one with rows {0, 2} of another.
__device__ __forceinline__ void swap_rows32(uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  const uint32_t x = r[0], y = r[1];
  a = x;
  b = y;
}
__device__ __forceinline__ void swap_rows16(uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
  const uint32_t x = r[0], y = r[1];
  a = x;
  b = y;
}
__device__ __forceinline__ void transpose_rows4(u32x4 (&v)[4]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint32_t a0 = v[0][e], a1 = v[1][e], a2 = v[2][e], a3 = v[3][e];
    swap_rows32(a0, a2);
    swap_rows32(a1, a3);
    swap_rows16(a0, a1);
    swap_rows16(a2, a3);
    v[0][e] = a0;
    v[1][e] = a1;
    v[2][e] = a2;
    v[3][e] = a3;
  }
}

template <int BITS, bool SYM, bool INTER, int MB, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) gemm_mfma_kernel(const GemmBatch b) {
  using F = Fmt<BITS>;
  constexpr int CPL = F::CPL, NF = CPL / 8;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, kb = lane >> 4;
  __shared__ float part[2][WAVES][MB * 4][64];
  const uint32_t magic = magic_vgpr();
  const int total = b.bt_start[b.count];
  int phase = 0;
  int p = 0;
  for (int bt = blockIdx.x; bt < total; bt += gridDim.x) {
    while (p + 1 < b.count && bt >= b.bt_start[p + 1]) ++p;
    const GemmProblem& d = b.p[p];
    const int wk = 1 << d.lwk;
    const int slot = wave >> d.lwk;
    const int kw = wave & (wk - 1);
    const int tile = (bt - b.bt_start[p]) * (WAVES >> d.lwk) + slot;  // WAVES / wk tiles per block-tile
    const bool active = tile < d.tiles;
    const int row0 = tile * 16;
    const int ib = kw * d.per_wave;
    const int ie = min(d.n_iters, ib + d.per_wave);
    f4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f4{0.f, 0.f, 0.f, 0.f};
    if (active && ib < ie) {
      const uint32_t row_bytes = static_cast<uint32_t>(d.K) * BITS / 8;
      const uint32_t meta_row = static_cast<uint32_t>(d.n_groups) * 2u;
      const __amdgpu_buffer_rsrc_t wbuf = buffer_of(d.qweight, static_cast<uint32_t>(d.N) * row_bytes);
      const __amdgpu_buffer_rsrc_t sbuf = buffer_of(d.scales, static_cast<uint32_t>(d.N) * meta_row);
      const __amdgpu_buffer_rsrc_t zbuf = buffer_of(SYM ? d.scales : d.zeros, static_cast<uint32_t>(d.N) * meta_row);
      const __amdgpu_buffer_rsrc_t xbuf =
          buffer_of(d.x, static_cast<uint32_t>(b.M) * static_cast<uint32_t>(d.K) * 2u);
      const uint32_t n = static_cast<uint32_t>(min(row0 + r, d.N - 1));  // past N: re-read, never stored
      const uint32_t wrow = n * row_bytes, mrow = n * meta_row;
      uint32_t xrow[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        xrow[mb] = static_cast<uint32_t>(min(16 * mb + r, b.M - 1)) * static_cast<uint32_t>(d.K) * 2u;
      // the fields the iterations read, as values (read through d, the group
      // fields were loaded from the kernel arguments, and waited on, every
      // iteration)
      const int n_chunks = d.n_chunks, n_groups = d.n_groups, cpg_shift = d.cpg_shift, cpg = d.cpg;
      for (int t = ib; t < ie; ++t) {
        const int c = 4 * t + kb;
        const bool cok = c < n_chunks;
        const uint32_t g = n_groups == 1 ? 0u
                           : (cpg_shift >= 0 ? static_cast<uint32_t>(c) >> cpg_shift
                                             : static_cast<uint32_t>(c) / static_cast<uint32_t>(cpg));
        const uint32_t zb = SYM ? 0u
                                : __builtin_amdgcn_raw_buffer_load_b16(zbuf, cok ? mrow + g * 2u : kOutOfRange, 0, 0);
        const uint32_t sb = __builtin_amdgcn_raw_buffer_load_b16(sbuf, cok ? mrow + g * 2u : kOutOfRange, 0, 0);
        const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(
            wbuf, cok ? wrow + static_cast<uint32_t>(c) * 16u : kOutOfRange, 0, 2);
        u32x4 xv[MB][CPL / 8];
        if constexpr (BITS == 4) {
          // load q reads piece kb of chunk 4t + q, so the four lanes of a row
          // read that chunk's 64 contiguous bytes (16 rows x 64 B per load, not
          // 16 rows x 4 pieces 64 B apart); a 4 x 4 transpose over the lane
          // rows kb then hands lane (kb, r) the four pieces of its own chunk
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int cq = 4 * t + q;
              xv[mb][q] = __builtin_amdgcn_raw_buffer_load_b128(
                  xbuf, cq < n_chunks ? xrow[mb] + static_cast<uint32_t>(cq) * 64u + 16u * kb : kOutOfRange, 0, 0);
            }
          }
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) transpose_rows4(xv[mb]);
        } else {
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int q = 0; q < CPL / 8; ++q)
              xv[mb][q] = __builtin_amdgcn_raw_buffer_load_b128(
                  xbuf, cok ? xrow[mb] + static_cast<uint32_t>(c) * (CPL * 2u) + 16u * q : kOutOfRange, 0, 0);
        }
        h8 wf[NF];
        const bool wide = !SYM && (zb & 0x7FFFu) > 0x6400u;
        if (!SYM && __builtin_amdgcn_ballot_w64(wide) != 0)
          w16_fragments<BITS, SYM, true>(w, sb, zb, magic, wf);
        else
          w16_fragments<BITS, SYM, false>(w, sb, zb, magic, wf);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          uint32_t xd[CPL / 2];
#pragma unroll
          for (int q = 0; q < CPL / 8; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) xd[4 * q + e] = xv[mb][q][e];
          h2 xp[CPL / 2];
#pragma unroll
          for (int j = 0; j < 4; ++j) x_pairs_from_dwords<BITS, INTER>(xd + j * (F::PER / 2), xp + j * F::PAIRS);
#pragma unroll
          for (int f = 0; f < NF; ++f)
            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                pack8(xp[4 * f], xp[4 * f + 1], xp[4 * f + 2], xp[4 * f + 3]), wf[f], acc[mb], 0, 0, 0);
        }
      }
    }
    // lane (kb, r) holds y[16 mb + 4 kb + i][row0 + r]
    const int ncol = row0 + r;
    if (wk == 1) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = 16 * mb + 4 * kb + i;
          if (active && m < b.M && ncol < d.N) d.y[static_cast<int64_t>(m) * d.ldy + ncol] = f32_to_f16_rn(acc[mb][i]);
        }
    } else {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[phase][wave][4 * mb + i][lane] = acc[mb][i];
      __syncthreads();  // all 4 waves of the block run the same block-tile sequence
      if (active && kw == 0) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float v = 0.f;
            for (int j = 0; j < wk; ++j) v += part[phase][wave + j][4 * mb + i][lane];
            const int m = 16 * mb + 4 * kb + i;
            if (m < b.M && ncol < d.N) d.y[static_cast<int64_t>(m) * d.ldy + ncol] = f32_to_f16_rn(v);
          }
      }
      phase ^= 1;
    }
  }
}

// Small GEMM for M <= 16 with the activations shared across tiles. A block
// of 16 waves holds 4 tiles of 16 rows x 4 K-shares (wave w: tile w / 4,
// K-share w % 4), the same split along K as gemm_mfma_kernel at wk = 4. Each
// iteration (4 chunks per lane, lane (kb, r) as there) the 256 threads of a
// K-share stage its 16 batch rows x 4 chunks of activations in LDS, one
// 16-byte piece per thread (a wave's load covers 4 rows x 256 contiguous
// bytes), and all 16 waves meet at an LDS-only barrier (the weight loads stay
// in flight); each wave reads its A fragments from LDS. gemm_mfma_kernel
// loads every wave's activations itself: four times the activation loads,
// which counters showed the texture-address units spending most of their
// time on. The four K-share partials of a tile meet in LDS.
constexpr int kSxMinBlocks = 192;  // three quarters of the MI355X's 256 CUs

// TPB tiles x 4 K-shares per block; MB activation tiles of 16 rows.
template <int BITS, int MB, int TPB>
struct SxStage {
  static constexpr int kWaves = 4 * TPB;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kShareThreads = 64 * TPB;                 // threads of one K-share
  static constexpr int kChunkBytes = Fmt<BITS>::CPL * 2;
  static constexpr int kPieces = kChunkBytes / 16;               // 16-byte pieces per chunk
  static constexpr int kRowBytes = 4 * kChunkBytes + 16;         // a batch row's 4 chunks, padded
  static constexpr int kShareBytes = 16 * MB * kRowBytes;        // 16 MB batch rows
  static constexpr int kBufBytes = 4 * kShareBytes;              // 4 K-shares
  static constexpr int kPieceCount = 16 * MB * 4 * kPieces;      // pieces of one share per iteration
  static constexpr int kPerThread = (kPieceCount + kShareThreads - 1) / kShareThreads;
};

template <int BITS, bool SYM, bool INTER, int MB, int TPB>
__global__ void __launch_bounds__(256 * TPB) gemm_shared_x_kernel(const GemmBatch b) {
  using F = Fmt<BITS>;
  using SX = SxStage<BITS, MB, TPB>;
  constexpr int CPL = F::CPL, NF = CPL / 8;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, kb = lane >> 4;
  const int slot = wave >> 2, kw = wave & 3;
  const int tk = slot * 64 + lane;  // this thread's index among the threads of its K-share
  __shared__ __align__(16) unsigned char xs_lds[2 * SX::kBufBytes];
  __shared__ float part[SX::kWaves][4 * MB][64];
  const uint32_t magic = magic_vgpr();
  const int total = b.bt_start[b.count];
  int parity = 0;
  int p = 0;
  for (int bt = blockIdx.x; bt < total; bt += gridDim.x) {
    while (p + 1 < b.count && bt >= b.bt_start[p + 1]) ++p;
    const GemmProblem& d = b.p[p];
    const int tile = (bt - b.bt_start[p]) * TPB + slot;
    const bool active = tile < d.tiles;
    const int row0 = tile * 16;
    const int ib = kw * d.per_wave;
    const int ie = min(d.n_iters, ib + d.per_wave);
    f4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f4{0.f, 0.f, 0.f, 0.f};
    const uint32_t row_bytes = static_cast<uint32_t>(d.K) * BITS / 8;
    const uint32_t meta_row = static_cast<uint32_t>(d.n_groups) * 2u;
    const __amdgpu_buffer_rsrc_t wbuf = buffer_of(d.qweight, static_cast<uint32_t>(d.N) * row_bytes);
    const __amdgpu_buffer_rsrc_t sbuf = buffer_of(d.scales, static_cast<uint32_t>(d.N) * meta_row);
    const __amdgpu_buffer_rsrc_t zbuf = buffer_of(SYM ? d.scales : d.zeros, static_cast<uint32_t>(d.N) * meta_row);
    const uint32_t kbytes = static_cast<uint32_t>(d.K) * 2u;
    const __amdgpu_buffer_rsrc_t xbuf = buffer_of(d.x, static_cast<uint32_t>(b.M) * kbytes);
    const uint32_t n = static_cast<uint32_t>(min(row0 + r, d.N - 1));  // past N: re-read, never stored
    const uint32_t wrow = n * row_bytes, mrow = n * meta_row;
    // the fields the iterations read, as values (read through d, they were
    // loaded from the kernel arguments, and waited on, every iteration)
    const int per_wave = d.per_wave, n_chunks = d.n_chunks, n_groups = d.n_groups, cpg_shift = d.cpg_shift,
              cpg = d.cpg;
    // every wave, active or not, runs every iteration of the block's problem
    // (the K-shares stage together and meet at each iteration's barrier)
    for (int t = 0; t < per_wave; ++t) {
      unsigned char* buf = xs_lds + parity * SX::kBufBytes;
      parity ^= 1;
      const bool iok = ib + t < ie;
      // this K-share's activations of the iteration: piece e of 16 MB rows x 4 chunks
      u32x4 st[SX::kPerThread];
#pragma unroll
      for (int i = 0; i < SX::kPerThread; ++i) {
        const int e = tk + SX::kShareThreads * i;
        const int piece = e % SX::kPieces, cc = (e / SX::kPieces) % 4, m = e / (SX::kPieces * 4);
        const int c = 4 * (ib + t) + cc;
        const bool ok = e < SX::kPieceCount && iok && m < b.M && c < n_chunks;
        st[i] = __builtin_amdgcn_raw_buffer_load_b128(
            xbuf, ok ? static_cast<uint32_t>(m) * kbytes + static_cast<uint32_t>(c) * SX::kChunkBytes + 16u * piece
                     : kOutOfRange,
            0, 0);
      }
      const int c = 4 * (ib + t) + kb;
      const bool cok = active && iok && c < n_chunks;
      const uint32_t g = n_groups == 1 ? 0u
                         : (cpg_shift >= 0 ? static_cast<uint32_t>(c) >> cpg_shift
                                           : static_cast<uint32_t>(c) / static_cast<uint32_t>(cpg));
      const uint32_t zb = SYM ? 0u : __builtin_amdgcn_raw_buffer_load_b16(zbuf, cok ? mrow + g * 2u : kOutOfRange, 0, 0);
      const uint32_t sb = __builtin_amdgcn_raw_buffer_load_b16(sbuf, cok ? mrow + g * 2u : kOutOfRange, 0, 0);
      const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(
          wbuf, cok ? wrow + static_cast<uint32_t>(c) * 16u : kOutOfRange, 0, 2);
      __builtin_amdgcn_sched_barrier(0);  // every global load of the iteration is in flight before the staging waits
#pragma unroll
      for (int i = 0; i < SX::kPerThread; ++i) {
        const int e = tk + SX::kShareThreads * i;
        const int piece = e % SX::kPieces, cc = (e / SX::kPieces) % 4, m = e / (SX::kPieces * 4);
        if (e < SX::kPieceCount)
          *reinterpret_cast<u32x4*>(buf + kw * SX::kShareBytes + m * SX::kRowBytes + cc * SX::kChunkBytes +
                                     16 * piece) = st[i];
      }
      lds_barrier();
      h8 wf[NF];
      const bool wide = !SYM && (zb & 0x7FFFu) > 0x6400u;
      if (!SYM && __builtin_amdgcn_ballot_w64(wide) != 0)
        w16_fragments<BITS, SYM, true>(w, sb, zb, magic, wf);
      else
        w16_fragments<BITS, SYM, false>(w, sb, zb, magic, wf);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        // chunk kb of the iteration, batch row 16 mb + r, in the weights' pair order
        uint32_t xd[CPL / 2];
        const unsigned char* xrow =
            buf + kw * SX::kShareBytes + (16 * mb + r) * SX::kRowBytes + kb * SX::kChunkBytes;
#pragma unroll
        for (int q = 0; q < CPL / 8; ++q) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(xrow + 16 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e) xd[4 * q + e] = v[e];
        }
        h2 xp[CPL / 2];
#pragma unroll
        for (int j = 0; j < 4; ++j) x_pairs_from_dwords<BITS, INTER>(xd + j * (F::PER / 2), xp + j * F::PAIRS);
#pragma unroll
        for (int f = 0; f < NF; ++f)
          acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              pack8(xp[4 * f], xp[4 * f + 1], xp[4 * f + 2], xp[4 * f + 3]), wf[f], acc[mb], 0, 0, 0);
      }
    }
    // lane (kb, r) holds y[16 mb + 4 kb + i][row0 + r]; the 4 K-shares of a tile meet in LDS
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[wave][4 * mb + i][lane] = acc[mb][i];
    __syncthreads();
    if (active && kw == 0) {
      const int ncol = row0 + r;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = part[wave][4 * mb + i][lane] + part[wave + 1][4 * mb + i][lane] +
                          part[wave + 2][4 * mb + i][lane] + part[wave + 3][4 * mb + i][lane];
          const int m = 16 * mb + 4 * kb + i;
          if (m < b.M && ncol < d.N) d.y[static_cast<int64_t>(m) * d.ldy + ncol] = f32_to_f16_rn(v);
        }
    }
    __syncthreads();  // the partials are read before the next tile writes them
  }
}

// Small GEMM for 16 < M <= 64, walked by column groups with every batch row
// in each wave. A block of 4 waves owns 64 output columns (wave w: columns
// 16 w .. 16 w + 15, lane (kb, r) as in gemm_mfma_kernel) for all MB
// activation tiles of 16 rows, over the whole of K: each weight chunk is
// dequantized once and feeds MB MFMAs, and the four waves share one copy of
// the activations. (Blocks of one activation tile each dequantized every
// weight MB times: at M = 64 that math alone took 147 us per Llama-3-8B
// layer.) Activations go through LDS in stages of 128 k-values (INT2: 256):
// the 256 threads load a stage two stages ahead (one wave load covers whole
// rows, contiguous), put each word's activations in the weights' pair order
// (x_pairs_from_dwords) and store it one stage ahead into one of two
// buffers, so a wave reads its A fragments with one ds_read_b128 each. In
// LDS, 16-byte piece p of batch row q sits at slot p ^ (q % 16) of the row:
// the 16 rows one fragment read spans then fall in distinct banks. Weights
// run kWalkDepth iterations ahead in a register ring. One LDS-only barrier
// per stage; the loads stay in flight across it.
constexpr int kWalkDepth = 4;
constexpr int kTileCols = 64;  // output columns per block
constexpr int kWaitVm0 = 0x0F70;  // s_waitcnt vmcnt(0) (expcnt, lgkmcnt left at their maxima)

template <int BITS, int MB>
struct WalkStage {
  static constexpr int PER = Fmt<BITS>::PER;
  static constexpr int CPL = Fmt<BITS>::CPL;
  static constexpr int IK = 4 * CPL;                  // k-values per iteration (4 chunks)
  static constexpr int K = IK < 128 ? 128 : IK;       // k-values per stage
  static constexpr int SI = K / IK;                   // iterations per stage
  static constexpr int kRows = 16 * MB;
  static constexpr int kRowPieces = 2 * K / 16;       // 16-byte pieces of a row's stage
  static constexpr int kBufBytes = kRows * kRowPieces * 16;
  static constexpr int kUnitPieces = PER * 2 > 16 ? PER * 2 / 16 : 1;  // pieces holding whole words
  static constexpr int kUnits = kRows * kRowPieces / kUnitPieces;     // units per stage
  static constexpr int kLoads = kUnits / 256;         // units per thread per stage
  static constexpr int U = kWalkDepth / SI;           // stages per unrolled loop trip
  static_assert(kUnits % 256 == 0 && U >= 2 && U % 2 == 0, "walk geometry");
};

// One unit (kUnitPieces pieces of 16 bytes: whole words) of activations,
// reordered into the pairs x_pairs_from_dwords forms for each word.
template <int BITS, bool INTER, int UP>
__device__ __forceinline__ void pair_order_unit(const u32x4 (&v)[UP], u32x4 (&out)[UP]) {
  using F = Fmt<BITS>;
  constexpr int DW = 4 * UP;  // dwords of the unit
  uint32_t d[DW];
#pragma unroll
  for (int q = 0; q < UP; ++q)
#pragma unroll
    for (int e = 0; e < 4; ++e) d[4 * q + e] = v[q][e];
  h2 xp[DW];
#pragma unroll
  for (int j = 0; j < DW / (F::PER / 2); ++j) x_pairs_from_dwords<BITS, INTER>(d + j * (F::PER / 2), xp + j * F::PAIRS);
#pragma unroll
  for (int q = 0; q < UP; ++q)
    out[q] = u32x4{__builtin_bit_cast(uint32_t, xp[4 * q]), __builtin_bit_cast(uint32_t, xp[4 * q + 1]),
                   __builtin_bit_cast(uint32_t, xp[4 * q + 2]), __builtin_bit_cast(uint32_t, xp[4 * q + 3])};
}

template <int BITS, bool SYM, bool INTER, int MB>
__global__ void __launch_bounds__(256) gemm_walk_kernel(const GemmBatch b) {
  using F = Fmt<BITS>;
  using WS = WalkStage<BITS, MB>;
  constexpr int CPL = F::CPL, NF = CPL / 8, NP = CPL / 8;
  constexpr int SI = WS::SI, UP = WS::kUnitPieces, XL = WS::kLoads, D = kWalkDepth;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, kb = lane >> 4;
  __shared__ __align__(16) unsigned char xs_lds[2 * WS::kBufBytes];
  const int bt = blockIdx.x;
  int p = 0;
  while (p + 1 < b.count && bt >= b.bt_start[p + 1]) ++p;
  const GemmProblem& d = b.p[p];
  // block -> (column group, split along K); the splits of a group are adjacent
  const int splits = d.splits;
  const int grp = (bt - b.bt_start[p]) / splits;
  const int split = (bt - b.bt_start[p]) - grp * splits;
  const int col0 = grp * kTileCols + wave * 16;
  const uint32_t row_bytes = static_cast<uint32_t>(d.K) * BITS / 8;
  const uint32_t meta_row = static_cast<uint32_t>(d.n_groups) * 2u;
  const __amdgpu_buffer_rsrc_t wbuf = buffer_of(d.qweight, static_cast<uint32_t>(d.N) * row_bytes);
  const __amdgpu_buffer_rsrc_t sbuf = buffer_of(d.scales, static_cast<uint32_t>(d.N) * meta_row);
  const __amdgpu_buffer_rsrc_t zbuf = buffer_of(SYM ? d.scales : d.zeros, static_cast<uint32_t>(d.N) * meta_row);
  const uint32_t kbytes = static_cast<uint32_t>(d.K) * 2u;
  const __amdgpu_buffer_rsrc_t xbuf = buffer_of(d.x, static_cast<uint32_t>(b.M) * kbytes);
  const uint32_t n = static_cast<uint32_t>(min(col0 + r, d.N - 1));  // past N: re-read, never stored
  const uint32_t wrow = n * row_bytes, mrow = n * meta_row;
  // uniform values in scalars, so that no iteration reloads them from the argument block
  const int n_chunks = __builtin_amdgcn_readfirstlane(d.n_chunks);
  const int kdim = __builtin_amdgcn_readfirstlane(d.K);
  const int gmode = __builtin_amdgcn_readfirstlane(d.n_groups == 1 ? 0 : (d.cpg_shift >= 0 ? 1 : 2));
  const int cpg_shift = __builtin_amdgcn_readfirstlane(d.cpg_shift);
  const uint32_t cpg = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(d.cpg));
  // this block's iterations [i0, i1): stage s of the walk is global stage i0 / SI + s
  const int i0 = split * d.ips;
  const int i1 = min((n_chunks + 3) >> 2, i0 + d.ips);
  const int c_end = min(n_chunks, 4 * i1);  // chunks past the split read as zeros
  const int k_end = min(kdim, i1 * WS::IK);
  const int st0 = i0 / SI;
  const int n_st = (i1 - i0 + SI - 1) / SI;
  // this thread's units of a stage: unit e = 256 q + tid of the rows, in row order
  const int tid = threadIdx.x;
  uint32_t xoff[XL];
  int xpiece[XL], xlds[XL], xswz[XL];
#pragma unroll
  for (int q = 0; q < XL; ++q) {
    const int e = 256 * q + tid;
    const int rho = e / (WS::kRowPieces / UP);
    const int pc = (e % (WS::kRowPieces / UP)) * UP;
    xpiece[q] = pc;
    xlds[q] = rho * WS::kRowPieces * 16;
    xswz[q] = rho & 15;
    xoff[q] = rho < b.M ? static_cast<uint32_t>(rho) * kbytes + 16u * static_cast<uint32_t>(pc) : kOutOfRange;
  }
  auto issue_x = [&](int s, u32x4 (&xa)[XL][UP]) {
#pragma unroll
    for (int q = 0; q < XL; ++q)
#pragma unroll
      for (int h = 0; h < UP; ++h) {
        const bool ok = (xoff[q] != kOutOfRange) & ((st0 + s) * WS::K + 8 * (xpiece[q] + h + 1) <= k_end);
        xa[q][h] = __builtin_amdgcn_raw_buffer_load_b128(
            xbuf, ok ? xoff[q] + 16u * h + static_cast<uint32_t>(st0 + s) * (2u * WS::K) : kOutOfRange, 0, 0);
      }
  };
  auto store_x = [&](int buf_idx, const u32x4 (&xa)[XL][UP]) {
    unsigned char* buf = xs_lds + buf_idx * WS::kBufBytes;
#pragma unroll
    for (int q = 0; q < XL; ++q) {
      u32x4 v[UP];
      pair_order_unit<BITS, INTER, UP>(xa[q], v);
#pragma unroll
      for (int h = 0; h < UP; ++h)
        *reinterpret_cast<u32x4*>(buf + xlds[q] + 16 * ((xpiece[q] + h) ^ xswz[q])) = v[h];
    }
  };
  // scale and zero point in 32-bit registers of which the math reads the low
  // half only (16-bit arrays were packed in pairs right at the load, which
  // waits for it and, loads completing in order, for every load before it)
  auto issue_w = [&](int i, u32x4& w, uint32_t& sb, uint32_t& zb) {
    const int c = 4 * (i0 + i) + kb;
    const bool cok = c < c_end;
    const uint32_t g = gmode == 0 ? 0u
                       : (gmode == 1 ? static_cast<uint32_t>(c) >> cpg_shift : static_cast<uint32_t>(c) / cpg);
    zb = SYM ? 0u : __builtin_amdgcn_raw_buffer_load_b16(zbuf, cok ? mrow + g * 2u : kOutOfRange, 0, 0);
    sb = __builtin_amdgcn_raw_buffer_load_b16(sbuf, cok ? mrow + g * 2u : kOutOfRange, 0, 0);
    w = __builtin_amdgcn_raw_buffer_load_b128(wbuf, cok ? wrow + static_cast<uint32_t>(c) * 16u : kOutOfRange, 0, 2);
  };
  const uint32_t magic = magic_vgpr();
  f4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f4{0.f, 0.f, 0.f, 0.f};
  u32x4 xa[2][XL][UP];
  u32x4 wr[D];
  uint32_t sr[D], zr[D];
  issue_x(0, xa[0]);
  issue_x(1, xa[1]);
#pragma unroll
  for (int j = 0; j < D; ++j) issue_w(j, wr[j], sr[j], zr[j]);
  store_x(0, xa[0]);
  // every load before the walk done: the compiler's wait counts then hold no
  // pending load for the registers the first stages read
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  lds_barrier();
  // whole trips of U stages with no branch inside: stages past K load zeros
  // (a branch would put the loads' phis at a join, where the compiler widens
  // the 16-bit metadata and so waits for the loads just issued)
  for (int s0 = 0; s0 < n_st; s0 += WS::U) {
#pragma unroll
    for (int u = 0; u < WS::U; ++u) {
      const int s = s0 + u;
      {
        // stage s + 1 (loaded two stages ago) into the buffer stage s - 1 used:
        // every wave passed the barrier after stage s - 1, and the stores
        // then complete during this stage's math, not at its closing barrier
        store_x((u + 1) & 1, xa[(u + 1) & 1]);
        issue_x(s + 2, xa[u & 1]);  // this set's stage s was stored a stage ago
        const unsigned char* base = xs_lds + (u & 1) * WS::kBufBytes;
#pragma unroll
        for (int si = 0; si < SI; ++si) {
          const int slot = (u * SI + si) % D;
          // the A fragments first, so that the dequantization covers the LDS latency
          h8 a[MB][NF];
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            const unsigned char* xrow = base + (16 * mb + r) * (WS::kRowPieces * 16);
#pragma unroll
            for (int f = 0; f < NF; ++f)
              a[mb][f] = *reinterpret_cast<const h8*>(xrow + 16 * (((si * 4 + kb) * NP + f) ^ r));
          }
          h8 wf[NF];
          const bool wide = !SYM && (zr[slot] & 0x7FFFu) > 0x6400u;
          if (!SYM && __builtin_amdgcn_ballot_w64(wide) != 0)
            w16_fragments<BITS, SYM, true>(wr[slot], sr[slot], zr[slot], magic, wf);
          else
            w16_fragments<BITS, SYM, false>(wr[slot], sr[slot], zr[slot], magic, wf);
          issue_w(s * SI + si + D, wr[slot], sr[slot], zr[slot]);
          // the MB accumulation chains interleaved
#pragma unroll
          for (int f = 0; f < NF; ++f)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
              acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mb][f], wf[f], acc[mb], 0, 0, 0);
        }
        lds_barrier();
      }
    }
  }
  // lane (kb, r) holds y[16 mb + 4 kb + i][col0 + r]
  const int ncol = col0 + r;
  if (splits == 1) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 16 * mb + 4 * kb + i;
        if (m < b.M && ncol < d.N) d.y[static_cast<int64_t>(m) * d.ldy + ncol] = f32_to_f16_rn(acc[mb][i]);
      }
    return;
  }
  // Split along K: the partial tile goes to the scratch in the waves' own
  // layout (wave, activation tile, lane: one 16-byte store of a lane's four
  // sums); gemm_split_sum_kernel, the next launch, adds a group's partials
  // in split order and writes y. (Finishing in this launch, the last block
  // of a group to arrive at a counter adding them, cost three dependent
  // memory round trips per launch: 6-8 us on the Llama-3-8B shapes at
  // M = 64, more than the second launch.)
  float* tile = b.part + static_cast<int64_t>(d.part_base + grp * splits + split) * (16 * MB * kTileCols);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) reinterpret_cast<f4*>(tile)[(wave * MB + mb) * 64 + lane] = acc[mb];
}

// Second launch of a split gemm_walk_kernel launch: block g of problem p
// sums the partial tiles of column group g over the splits, in split order,
// and writes y; thread (wave, lane) takes the sums that lane of that wave
// held, so y is written as an unsplit block writes it.
template <int MB>
__global__ void __launch_bounds__(256) gemm_split_sum_kernel(const GemmBatch b) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 15, kb = lane >> 4;
  int p = 0;
  while (p + 1 < b.count && static_cast<int>(blockIdx.x) >= b.bt_start[p + 1]) ++p;
  const GemmProblem& d = b.p[p];
  const int splits = d.splits;
  const int grp = blockIdx.x - b.bt_start[p];
  constexpr int TILE = 16 * MB * kTileCols;
  const f4* tiles = reinterpret_cast<const f4*>(b.part + static_cast<int64_t>(d.part_base + grp * splits) * TILE);
  f4 sum[MB];
  for (int q0 = 0; q0 < splits; q0 += 4) {  // four splits' loads in flight at a time, added in split order
    f4 t[4][MB];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        t[j][mb] = q0 + j < splits ? tiles[static_cast<int64_t>(q0 + j) * (TILE / 4) + (wave * MB + mb) * 64 + lane]
                                   : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (q0 + j < splits) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) sum[mb] = q0 + j == 0 ? t[j][mb] : sum[mb] + t[j][mb];
      }
  }
  const int ncol = grp * kTileCols + wave * 16 + r;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * mb + 4 * kb + i;
      if (m < b.M && ncol < d.N) d.y[static_cast<int64_t>(m) * d.ldy + ncol] = f32_to_f16_rn(sum[mb][i]);
    }
}

// ---------------------------------------------------------------- dequantize
constexpr int kElemThreads = 256;

// Rows are walked along the grid's y dimension (a row index is uniform per
// block: no per-thread division) and a row's 32-bit words along x. A word
// lies in one group (group_size % (32/BITS) == 0): its group is a shift of
// the word index when words per group is a power of two (gshift >= 0), 0 for
// per-channel weights (one group), else a 32-bit division.
template <int BITS, bool SYM, bool INTER>
__global__ void __launch_bounds__(kElemThreads)
dequantize_kernel(const uint32_t* __restrict__ qweight, const uint16_t* __restrict__ scales,
                  const uint16_t* __restrict__ zeros, uint16_t* __restrict__ out, int N, int K, int group_size,
                  int gshift) {
  using F = Fmt<BITS>;
  const int wpr = K / F::PER;  // words per row
  const int ng = K / group_size;
  const int wpg = group_size / F::PER;
  for (int n = blockIdx.y; n < N; n += gridDim.y) {
    const uint32_t* qrow = qweight + static_cast<int64_t>(n) * wpr;
    const uint16_t* srow = scales + static_cast<int64_t>(n) * ng;
    const uint16_t* zrow = SYM ? nullptr : zeros + static_cast<int64_t>(n) * ng;
    uint16_t* orow = out + static_cast<int64_t>(n) * K;
    for (int w = blockIdx.x * kElemThreads + threadIdx.x; w < wpr; w += gridDim.x * kElemThreads) {
      const int g = ng == 1 ? 0 : (gshift >= 0 ? (w >> gshift) : w / wpg);
      const float s = f16_to_f32(srow[g]);
      const float off = SYM ? static_cast<float>(F::BIAS) : f16_to_f32(zrow[g]);
      const uint32_t word = qrow[w];
      uint16_t v[F::PER];
#pragma unroll
      for (int sl = 0; sl < F::PER; ++sl) {
        const float code = static_cast<float>((word >> (BITS * sl)) & ((1u << BITS) - 1u));
        // (code - off) then a separate fp32 multiply, then fp16 RNE: packer.py:183-189
        const float d = code - off;
        v[logical_of_slot<BITS, INTER>(sl)] = f32_to_f16_rn(__fmul_rn(d, s));
      }
      uint16_t* o = orow + static_cast<int64_t>(w) * F::PER;
      if constexpr (F::PER == 4) {
        *reinterpret_cast<uint2*>(o) = make_uint2(v[0] | (uint32_t(v[1]) << 16), v[2] | (uint32_t(v[3]) << 16));
      } else {
#pragma unroll
        for (int q = 0; q < F::PER / 8; ++q)
          *reinterpret_cast<uint4*>(o + 8 * q) = make_uint4(
              v[8 * q + 0] | (uint32_t(v[8 * q + 1]) << 16), v[8 * q + 2] | (uint32_t(v[8 * q + 3]) << 16),
              v[8 * q + 4] | (uint32_t(v[8 * q + 5]) << 16), v[8 * q + 6] | (uint32_t(v[8 * q + 7]) << 16));
      }
    }
  }
}

// -------------------------------------------------------------------- unpack
template <int BITS, bool INTER>
__global__ void __launch_bounds__(kElemThreads)
unpack_kernel(const uint32_t* __restrict__ qweight, int32_t* __restrict__ out, int64_t total_words, int K) {
  using F = Fmt<BITS>;
  const int64_t words_per_row = K / F::PER;
  for (int64_t widx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; widx < total_words;
       widx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = widx / words_per_row;
    const int k0 = static_cast<int>(widx - n * words_per_row) * F::PER;
    const uint32_t w = qweight[widx];
    int32_t v[F::PER];
#pragma unroll
    for (int sl = 0; sl < F::PER; ++sl)
      v[logical_of_slot<BITS, INTER>(sl)] = static_cast<int32_t>((w >> (BITS * sl)) & ((1u << BITS) - 1u));
    int32_t* o = out + n * K + k0;
#pragma unroll
    for (int q = 0; q < F::PER / 4; ++q)
      *reinterpret_cast<int4*>(o + 4 * q) = make_int4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
  }
}

// ------------------------------------------------------------------- add_one
__global__ void __launch_bounds__(kElemThreads)
add_one_kernel(const float* __restrict__ in, float* __restrict__ out, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    out[i] = in[i] + 1.0f;
}

// --------------------------------------------------------------- measurement
// The benchmark's denominators (no reference counterpart in the kernels; the
// reference measures its read ceiling with torch ops,
// scripts/bandwidth_by_dtype.py:85-106):
//   stream_read_kernel  reads `bytes` once: wave w reads 1 KiB segments w,
//                       w + W, w + 2W, ... (W waves in the grid) with one
//                       non-temporal 16-byte load per lane, so the whole chip
//                       sweeps the buffer in address order. Of the layouts
//                       measured on the part (1-8 KiB per wave and load set,
//                       2-8 waves per SIMD, strided or contiguous), this one
//                       read fastest (~90% of the 8 TB/s peak over 4 GiB);
//   empty_kernel        does nothing: the per-launch gap of back-to-back
//                       launches in a HIP graph.
// The xor of everything read decides one store that a real buffer never
// triggers, so the loads cannot be dropped.
constexpr uint32_t kReadMagic = 0x9e3779b9u;

__global__ void __launch_bounds__(256) stream_read_kernel(const unsigned char* __restrict__ src, int64_t bytes,
                                                          uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x * 4 + (threadIdx.x >> 6)));
  const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
  const int64_t segments = (bytes + 1023) / 1024;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t sg = wave; sg < segments; sg += waves) {
    const int64_t left = bytes - sg * 1024;  // the last segment may be partial: loads past it return zeros
    const __amdgpu_buffer_rsrc_t r = buffer_of(src + sg * 1024, static_cast<uint32_t>(left < 1024 ? left : 1024));
    acc ^= __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<uint32_t>(lane) * 16u, 0, 2);
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == kReadMagic && acc.x == kReadMagic) sink[0] = acc.y;
}

__global__ void empty_kernel() {}


// ----------------------------------------------------------------- launchers
namespace {

int64_t elementwise_blocks(int64_t items) {
  const int64_t b = (items + kElemThreads - 1) / kElemThreads;
  return b < 1 ? 1 : (b > 65536 ? 65536 : b);  // grid-stride loops cover the rest
}

// Launch geometry of a grouped GEMV with M = 1 (the VALU kernel), chosen per
// launch from the problems' shapes:
//   R    rows per tile: 8 when the launch has at least kWideTiles tiles of 8
//        rows (long stacks of projections: the activation pairs are reused 8x
//        and one DPP reduction chain serves 8 rows), else 4.
//   wk   waves sharing one tile along K (1, 2 or 4): the smallest that gives
//        the launch kTargetWaves(bits) waves, capped per problem so that each
//        wave keeps at least kMinColumns 16-byte columns of its rows. INT8 has
//        the least VALU work per byte and wants the most waves in flight.
//   grid persistent: the co-resident blocks of the kernel (occupancy query,
//        cached per instance), capped by the number of block-tiles.
// Geometry changes only the order of fp32 additions (split-K partial sums),
// so a problem's result is deterministic for a given launch but may differ in
// the last bits between a grouped launch and a single one.
// M = 1 dot products on the matrix cores (gemv_m1_kernel<..., MF = true)?
// With exact (q - z) codes INT2 g64 measured 48.3% of peak with MFMA vs 46.1%
// on the VALU (v_dot2 was then its largest VALU item). With the biased codes
// the VALU form needs no accumulator registers and measured better: C4 INT2
// stack 4270 -> 4345 GB/s, C5 stack 5457 -> 5558 GB/s; INT4 and INT8 were
// within noise or slower with MFMA in both forms. So no format uses it; the
// MF form stays as the measured alternative.
constexpr bool m1_uses_mfma(int) { return false; }
constexpr int64_t kWideTiles = 6144;
constexpr int64_t kProWideTiles = 2048;  // prologue launches: see launch_gemv_prologue_t
constexpr int64_t kMinColumns = 40;

int64_t target_waves(int bits) { return bits == 8 ? 8192 : (bits == 4 ? 6144 : 4096); }

// 8-row tiles also for launches of at least kLongWideTiles of them whose
// every problem has K >= kLongK: such launches split K (8192-column rows and
// 1024-2048 eight-row tiles), and each lane's activation loads then serve 8
// rows instead of 4. Measured (graph replays, same box): INT4 C5 q|k|v
// 10.83 -> 10.33-10.65 us, o_proj 9.34 -> 8.95 us; at K = 4096 the 4-row
// rule stays (INT8 C2 9.2 against 9.46 us, C4 gate|up 12.6 against 12.8).
constexpr int64_t kLongWideTiles = 1024;
constexpr int64_t kLongK = 8192;

int rows_per_tile(const GemvOperand* ops, int count) {
  int64_t tiles8 = 0, kmin = INT64_MAX;
  for (int i = 0; i < count; ++i) {
    tiles8 += (ops[i].N + 7) / 8;
    kmin = std::min<int64_t>(kmin, ops[i].K);
  }
  return tiles8 >= kWideTiles || (tiles8 >= kLongWideTiles && kmin >= kLongK) ? 8 : 4;
}

// wk[i] for every problem of the launch (rows per tile R).
void waves_per_tile(const GemvOperand* ops, int count, int bits, int R, int* wk, int64_t target = 0) {
  if (target == 0) target = target_waves(bits);
  int w = 1;
  for (; w < 4; w *= 2) {
    int64_t waves = 0;
    for (int i = 0; i < count; ++i) {
      const int64_t chunks = ops[i].K / (128 / bits);
      int wi = 1;
      while (wi < w && chunks / (2 * wi) >= kMinColumns) wi *= 2;
      waves += (ops[i].N + R - 1) / R * wi;
    }
    if (waves >= target) break;
  }
  for (int i = 0; i < count; ++i) {
    const int64_t chunks = ops[i].K / (128 / bits);
    int wi = 1;
    while (wi < w && chunks / (2 * wi) >= kMinColumns) wi *= 2;
    wk[i] = wi;
  }
}

// wk for an M = 1 launch (gemv_m1_pipe_kernel takes those of one-wave
// tiles): one-wave tiles, in place of the K split above, for INT2 launches
// and for INT4 / INT8 launches of at most kPipeTiles four-row tiles, from
// kPipeMinTiles tiles on (smaller launches keep the split: one-wave tiles
// leave most SIMDs idle there).
// The pipelined kernel then walks whole rows with the activations staged per
// block (the INT2 kept variant: kept per wave). Measured against the K split
// (graph replays of distinct weights): INT2 8192 x 28672 (C5 down_proj)
// 24.1 -> 16.9 us, 4096 x 14336 8.57 -> 7.52, 4096 x 11008 (C3) 7.39 ->
// 6.42; INT4 4096 x 4096 (C1, C4 o_proj; 1024 tiles) 4.72 -> 4.20,
// 4096 x 14336 (C4 down_proj) 9.15 -> 8.75; but INT4 C4 q|k|v (1536 tiles)
// 5.10 -> 5.22, C5 o_proj (2048) 9.33 -> 9.7, C5 q|k|v (2560) 10.8 -> 11.8,
// INT8 11008 x 4096 (C2, 2752 tiles) 9.24 -> 10.32.
constexpr int64_t kPipeTiles = 1024;
// INT4 1024 x 4096 (k_proj; 256 tiles) 3.50 us split against 3.81 one-wave,
// 1024 x 8192 3.88 against 5.36.
constexpr int64_t kPipeMinTiles = 512;

// RMSNorm launches take one-wave tiles up to kRmsPipeTiles: on the K split
// every lane of every K share forms x * gamma and sum(x^2) again, where the
// pipelined kernel does it once per block and batch (the C4 q|k|v launch with
// RMSNorm, 1536 tiles: fused decode step 34.0 -> 33.8 us/layer).
constexpr int64_t kRmsPipeTiles = 2048;

void m1_waves_per_tile(const GemvOperand* ops, int count, int bits, int R, int* wk,
                       int64_t max_tiles = kPipeTiles) {
  waves_per_tile(ops, count, bits, R, wk);
  int64_t tiles = 0;
  for (int i = 0; i < count; ++i) tiles += (ops[i].N + R - 1) / R;
  if (tiles >= kPipeMinTiles && (bits == 2 || (R == 4 && tiles <= max_tiles)))
    for (int i = 0; i < count; ++i) wk[i] = 1;
}

int log2_exact(int64_t v) {  // log2 of a power of two, else -1
  if (v <= 0 || (v & (v - 1)) != 0) return -1;
  int s = 0;
  while ((int64_t(1) << s) < v) ++s;
  return s;
}

thread_local hipEvent_t t_start_event = nullptr, t_stop_event = nullptr;

template <typename Kernel, typename Batch>
hipError_t launch_kernel(Kernel kernel, int blocks, const Batch& kb, hipStream_t stream, int threads = kGemvThreads) {
  if (t_start_event && t_stop_event) {
    hipExtLaunchKernelGGL(kernel, dim3(blocks), dim3(threads), 0, stream, t_start_event, t_stop_event, 0, kb);
    t_start_event = t_stop_event = nullptr;
  } else {
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(threads), 0, stream, kb);
  }
  return hipGetLastError();
}

// Co-resident blocks of a kernel instance on the current device. Queried once
// per instance and device: the cache is keyed by the kernel itself (a
// template argument, because every instance of one kernel template has the
// same function type) and indexed by the device, each entry written once with
// an atomic store (concurrent first calls on one device store the same value).
constexpr int kMaxDevices = 64;

template <auto Kernel, int THREADS = kGemvThreads>
int resident_blocks() {
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 512;
  }
  const bool indexed = dev >= 0 && dev < kMaxDevices;
  if (indexed) {
    const int v = cached[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, Kernel, THREADS, 0) != hipSuccess || cus <= 0 ||
      per_cu <= 0) {
    (void)hipGetLastError();
    return 512;
  }
  if (indexed) cached[dev].store(cus * per_cu, std::memory_order_relaxed);
  return cus * per_cu;
}

// The launch description of a list of problems cut into tiles of R rows
// whose K ranges wk[i] waves share; a wave's share is a multiple of `step`
// chunks. Returns the number of block-tiles.
int fill_kernel_batch(const GemvOperand* ops, int count, int64_t M, int bits, int R, int step, const int* wks,
                      KernelBatch& kb) {
  const int cpl = 128 / bits;
  kb = KernelBatch{};
  kb.count = count;
  kb.M = static_cast<int>(M);
  int bts = 0;
  for (int i = 0; i < count; ++i) {
    const GemvOperand& o = ops[i];
    KernelProblem& k = kb.p[i];
    k.qweight = o.qweight;
    k.scales = o.scales;
    k.zeros = o.zeros;
    k.x = o.x;
    k.y = o.y;
    k.aux = o.aux;
    k.N = static_cast<int>(o.N);
    k.K = static_cast<int>(o.K);
    k.n_groups = static_cast<int>(o.K / o.group_size);
    k.chunks_per_group = static_cast<int>(o.group_size / cpl);
    k.cpg_shift = log2_exact(k.chunks_per_group);
    k.n_chunks = static_cast<int>(o.K / cpl);
    const int wk = wks[i];
    k.lwk = log2_exact(wk);
    k.per_wave = ((k.n_chunks + wk - 1) / wk + step - 1) / step * step;
    k.tiles = static_cast<int>((o.N + R - 1) / R);
    k.ldy = static_cast<int>(o.ldy ? o.ldy : o.N);
    const int tiles_per_bt = kWavesPerBlock / wk;
    kb.bt_start[i] = bts;
    bts += (k.tiles + tiles_per_bt - 1) / tiles_per_bt;
  }
  kb.bt_start[count] = bts;
  return bts;
}

// Activations kept across tiles (gemv_m1_kernel<..., kXmKeep>) for INT2
// launches of 8-row, one-batch tiles (K <= 4096, one wave per tile) of at
// least kKeepRounds rounds of block-tiles: the grid walks runs of kKeepRun
// consecutive block-tiles, and a wave's tiles within a run mostly read the
// same x. (The variant's 33 KiB of LDS per block allow four waves per SIMD:
// the 8-row tiles' register count allows no more, the 4-row tiles' six.)
// Measured on the C4 INT2 stack (2752- and 3488-block-tile launches, 2.7 and
// 3.4 rounds): with the activation loads removed altogether (a timing copy)
// 12.6% faster; runs of 3 +4-5% over the plain kernel (the 3488-block-tile
// launches 31.8 -> 29.1 us), runs of 2 on the shorter launches 0.8% less,
// runs of 4 +0.9%, one contiguous share per block +0.4% (that walk alone
// -7.7%).
constexpr bool m1_keeps_x(int bits) { return bits == 2; }
constexpr int kKeepRun = 3;
constexpr int kKeepRounds = 2;

// Which M = 1 kernel variant a launch runs (PRO = none; of the prologue
// launches, those of one-wave tiles take gemv_m1_pipe_kernel with the
// prologue, the others gemv_m1_kernel's load variant):
//   kM1Keep   INT2, 8-row one-batch tiles, activations kept across tiles,
//             needs kKeepRounds rounds of its grid;
//   kM1Pipe   gemv_m1_pipe_kernel: every other launch of one-wave tiles
//             (wk = 1 for every problem, so its walk has no barrier). On the
//             INT2 launches outside the kept variant it measured 13% faster
//             than the load variant (C4 INT2 decode 1.04 -> 0.905 ms/step),
//             and faster than a block-staged variant of gemv_m1_kernel (one
//             coalesced activation load per block and batch) that took the
//             INT2 launches of K >= 8192 before: C5 stack 54.7 -> 51.4
//             us/layer, C4 INT2 stack 14.79 -> 14.38 us/layer, C5 decode
//             5.386 -> 5.362 ms/step (that variant was then removed); on the
//             INT2 stack it ties the kept variant;
//   kM1Load   gemv_m1_kernel, activations loaded per wave (split-K launches).
// Kind 5 of dq_gemv_plan (the block-staged variant) is no longer returned.
// grid_keep: the co-resident blocks of the kept kernel.
//
// Of the split launches, INT4 / INT8 ones of four-row tiles whose K shares
// are the same 2 or 4 waves in every problem, at most kPipeSplitBlockTiles
// block-tiles (4096 waves), take gemv_m1_pipe_split_kernel (kind 8 of
// dq_gemv_plan). Measured against gemv_m1_kernel (graph replays of distinct
// weights, same box): INT4 1024 x 4096 (k_proj alone, 256 tiles x 2) 3.45 ->
// 3.20 us, 1024 x 8192 (x 4) 3.86 -> 3.63, C4 q|k|v (1536 x 2) 5.11 -> 5.03;
// larger launches lost (14336 x 4096, 3584 x 2: 8.15 -> 8.65 us; 11008 x
// 4096 7.10 -> 7.4; eight-row tiles x 4 on C5 q|k|v 10.4 -> 11.2).
constexpr int kPipeSplitBlockTiles = 1024;

bool pipe_split(int bits, int R, const int* wks, int count, int bts) {
  if (bits == 2 || R != 4 || bts > kPipeSplitBlockTiles) return false;
  for (int i = 1; i < count; ++i)
    if (wks[i] != wks[0]) return false;
  return wks[0] == 2 || wks[0] == 4;
}
enum M1Variant : int { kM1Load = 2, kM1Pipe = 4, kM1Keep = 6 };

M1Variant m1_variant(const KernelBatch& kb, int count, int bits, int R, const int* wks, int bts, int grid_keep) {
  bool one_wave = true;
  for (int i = 0; i < count; ++i) one_wave = one_wave && wks[i] == 1;
  if (!one_wave) return kM1Load;
  if (m1_keeps_x(bits) && R == 8) {
    bool keep = true;
    for (int i = 0; i < count; ++i) keep = keep && kb.p[i].n_chunks <= 64;
    if (keep && bts >= kKeepRounds * grid_keep) return kM1Keep;
  }
  return kM1Pipe;
}

template <int BITS, bool SYM, bool INTER, int R, int PRO = kProNone>
hipError_t launch_gemv_m1(const GemvOperand* ops, int count, int64_t M, hipStream_t stream, float eps = 0.f) {
  int wks[kMaxBatch];
  m1_waves_per_tile(ops, count, BITS, R, wks, PRO == kProRmsNorm ? kRmsPipeTiles : kPipeTiles);
  KernelBatch kb;
  const int bts = fill_kernel_batch(ops, count, M, BITS, R, 1, wks, kb);
  kb.eps = eps;
  if (bts == 0) return hipSuccess;
  if constexpr (PRO == kProNone && !m1_uses_mfma(BITS)) {
    constexpr auto keep_kernel = gemv_m1_kernel<BITS, SYM, INTER, R, false, PRO, kXmKeep>;
    const int grid_keep = m1_keeps_x(BITS) && R == 8 ? resident_blocks<keep_kernel>() : 0;
    switch (m1_variant(kb, count, BITS, R, wks, bts, grid_keep)) {
      case kM1Keep:
        if constexpr (m1_keeps_x(BITS) && R == 8) {
          kb.run = kKeepRun;
          return launch_kernel(keep_kernel, grid_keep, kb, stream);
        }
        break;
      case kM1Pipe: {
        constexpr auto kernel = gemv_m1_pipe_kernel<BITS, SYM, INTER, R>;
        return launch_kernel(kernel, std::min(bts, resident_blocks<kernel>()), kb, stream);
      }
      default:
        if constexpr (R == 4 && BITS != 2) {
          if (pipe_split(BITS, R, wks, count, bts)) {
            if (wks[0] == 2) {
              constexpr auto kernel = gemv_m1_pipe_split_kernel<BITS, SYM, INTER, R, 2>;
              return launch_kernel(kernel, std::min(bts, resident_blocks<kernel>()), kb, stream);
            }
            constexpr auto kernel = gemv_m1_pipe_split_kernel<BITS, SYM, INTER, R, 4>;
            return launch_kernel(kernel, std::min(bts, resident_blocks<kernel>()), kb, stream);
          }
        }
        break;
    }
  }
  if constexpr ((PRO == kProRmsNorm || PRO == kProSwiGlu) && !m1_uses_mfma(BITS)) {
    bool one_wave = true;
    for (int i = 0; i < count; ++i) one_wave = one_wave && wks[i] == 1;
    if (one_wave) {
      constexpr auto kernel = gemv_m1_pipe_kernel<BITS, SYM, INTER, R, PRO>;
      return launch_kernel(kernel, std::min(bts, resident_blocks<kernel>()), kb, stream);
    }
  }
  constexpr auto kernel = gemv_m1_kernel<BITS, SYM, INTER, R, m1_uses_mfma(BITS), PRO, kXmLoad>;
  return launch_kernel(kernel, std::min(bts, resident_blocks<kernel>()), kb, stream);
}

// Geometry of the quad kernel (2 <= M <= 8): tiles of 4 * kQuadsPerTile rows,
// MG = 1 batch-row group of 4 for M <= 4, else 2; wk as for the M = 1 kernel
// (tiles of 8 rows), the same for every problem of the launch (the smallest
// of the problems' choices; capped at 2 for INT2 with MG = 2, whose staging
// buffers would otherwise take 132 KiB of LDS), each wave's share rounded up
// to whole steps of 16 chunks. Two quads per tile measured best on the C4
// stack (M = 2 / 4 / 8: +2 / +4 / +16% over four, whose accumulators and
// operands held M = 8 to two waves per SIMD; one quad lost 4-17%).
constexpr int kQuadsPerTile = 2;

// The quad kernel's INT8 launches want fewer K-shares than the M = 1 rule
// gives them (its waves carry M rows of MFMA work per weight): a target of
// 2048 waves took C2 at M = 4 (11008 x 4096, per-channel) from 14.5 to 13.2-13.5
// us per call; the same target for the M = 1 kernel cost C2 at M = 1 10%.
int64_t quad_target_waves(int bits) { return bits == 8 ? 2048 : target_waves(bits); }

int quad_waves_per_tile(const GemvOperand* ops, int count, int bits, int mg) {
  int wks[kMaxBatch];
  waves_per_tile(ops, count, bits, 4 * kQuadsPerTile, wks, quad_target_waves(bits));
  int wk = 4;
  for (int i = 0; i < count; ++i) wk = std::min(wk, wks[i]);
  if (bits == 2 && mg == 2) wk = std::min(wk, 2);
  return wk;
}

template <int BITS, bool SYM, bool INTER, int MG, int WK>
hipError_t launch_gemv_quad_wk(const GemvOperand* ops, int count, int64_t M, hipStream_t stream) {
  constexpr int R = 4 * kQuadsPerTile;
  int wks[kMaxBatch];
  for (int i = 0; i < count; ++i) wks[i] = WK;
  KernelBatch kb;
  const int bts = fill_kernel_batch(ops, count, M, BITS, R, 16, wks, kb);
  if (bts == 0) return hipSuccess;
  constexpr auto kernel = gemv_quad_kernel<BITS, SYM, INTER, kQuadsPerTile, MG, WK>;
  return launch_kernel(kernel, std::min(bts, resident_blocks<kernel>()), kb, stream);
}

template <int BITS, bool SYM, bool INTER, int MG>
hipError_t launch_gemv_quad(const GemvOperand* ops, int count, int64_t M, hipStream_t stream) {
  const int wk = quad_waves_per_tile(ops, count, BITS, MG);
  if (wk == 1) return launch_gemv_quad_wk<BITS, SYM, INTER, MG, 1>(ops, count, M, stream);
  if (wk == 2) return launch_gemv_quad_wk<BITS, SYM, INTER, MG, 2>(ops, count, M, stream);
  if constexpr (BITS == 2 && MG == 2) return hipErrorInvalidValue;  // capped above
  else return launch_gemv_quad_wk<BITS, SYM, INTER, MG, 4>(ops, count, M, stream);
}

// Geometry of the small GEMM (8 < M <= 64, or any M <= 64 the caller sends):
// MB activation tiles of 16 rows; 16-row weight tiles; wk waves per tile
// along K, the fewest of {1, 2, 4} that give the launch kGemmWaves waves while
// leaving each wave at least 4 iterations of 4 chunks.
constexpr int64_t kGemmWaves = 4096;

int gemm_waves_per_tile(const GemvOperand* ops, int count, int bits, int max_wk, int* wk) {
  const int cpl = 128 / bits;
  int w = 1;
  for (; w < max_wk; w *= 2) {
    int64_t waves = 0;
    for (int i = 0; i < count; ++i) {
      const int64_t iters = (ops[i].K / cpl + 3) / 4;
      int wi = 1;
      while (wi < w && iters / (2 * wi) >= 4) wi *= 2;
      waves += (ops[i].N + 15) / 16 * wi;
    }
    if (waves >= kGemmWaves) break;
  }
  for (int i = 0; i < count; ++i) {
    const int64_t iters = (ops[i].K / cpl + 3) / 4;
    int wi = 1;
    while (wi < w && iters / (2 * wi) >= 4) wi *= 2;
    wk[i] = wi;
  }
  return w;
}

// Waves per block of gemm_mfma_kernel, and so the largest split along K: 8
// for M <= 32, 4 above. Measured on the Llama-3-8B shapes against 4-wave
// blocks: at M = 16 q|k|v|o_proj -8% and down_proj -11% (one tile per block
// split 8 ways: the same 256 blocks, half the iterations per wave), at
// M = 32 the small shapes -4%; at M = 64 the large ones +2% (so 4 stay).
// 16-wave blocks put two tiles in a block and halved the blocks of a q_proj
// launch: +45%.
template <int BITS, int MB>
constexpr int gemm_block_waves() {
  return MB <= 2 ? 8 : 4;
}

template <int BITS, bool SYM, bool INTER, int MB>
hipError_t launch_gemm_mb(const GemvOperand* ops, int count, int64_t M, hipStream_t stream) {
  constexpr int CPL = 128 / BITS;
  constexpr int WAVES = gemm_block_waves<BITS, MB>();
  auto fill = [&](const int* wks, int waves_per_block, GemmBatch& gb) {
    gb = GemmBatch{};
    gb.count = count;
    gb.M = static_cast<int>(M);
    int bts = 0;
    for (int i = 0; i < count; ++i) {
      const GemvOperand& o = ops[i];
      GemmProblem& k = gb.p[i];
      k.qweight = o.qweight;
      k.scales = o.scales;
      k.zeros = o.zeros;
      k.x = o.x;
      k.y = o.y;
      k.N = static_cast<int>(o.N);
      k.K = static_cast<int>(o.K);
      k.n_groups = static_cast<int>(o.K / o.group_size);
      k.cpg = static_cast<int>(o.group_size / CPL);
      k.cpg_shift = log2_exact(k.cpg);
      k.n_chunks = static_cast<int>(o.K / CPL);
      k.n_iters = (k.n_chunks + 3) / 4;
      const int wk = wks[i];
      k.lwk = log2_exact(wk);
      k.per_wave = (k.n_iters + wk - 1) / wk;
      k.tiles = static_cast<int>((o.N + 15) / 16);
      k.ldy = static_cast<int>(o.ldy ? o.ldy : o.N);
      const int tiles_per_bt = waves_per_block / wk;
      gb.bt_start[i] = bts;
      bts += (k.tiles + tiles_per_bt - 1) / tiles_per_bt;
    }
    gb.bt_start[count] = bts;
    return bts;
  };
  GemmBatch gb;
  int wks[kMaxBatch];
  if constexpr (MB <= 2 && BITS != 2) {
    // Every tile split 4 ways along K and enough tiles for kSxMinBlocks
    // blocks: the variant that shares each K-share's activations across the
    // block's tiles (4 tiles at M <= 16, 2 at M <= 32, where the registers
    // allow two waves per SIMD). Measured on the Llama-3-8B shapes: gate/up_proj
    // 29.5 -> 20.8 us at M = 16 (224 blocks), 44.0 -> 31.7 us at M = 32 (448
    // blocks); at M = 16 down_proj and q|o_proj (64 blocks: three quarters of
    // the CUs idle) ran 2x slower in it. INT2, whose lanes carry 128 bytes of
    // activations per chunk, does not take it.
    constexpr int TPB = MB == 1 ? 4 : 2;
    gemm_waves_per_tile(ops, count, BITS, 4, wks);
    bool four = true;
    int sbts = 0;
    for (int i = 0; i < count; ++i) {
      four = four && wks[i] == 4;
      sbts += static_cast<int>(((ops[i].N + 15) / 16 + TPB - 1) / TPB);
    }
    if (four && sbts >= kSxMinBlocks) {
      fill(wks, 4 * TPB, gb);
      using SX = SxStage<BITS, MB, TPB>;
      constexpr auto kernel = gemm_shared_x_kernel<BITS, SYM, INTER, MB, TPB>;
      return launch_kernel(kernel, std::min(sbts, resident_blocks<kernel, SX::kThreads>()), gb, stream,
                           SX::kThreads);
    }
  }
  gemm_waves_per_tile(ops, count, BITS, WAVES, wks);
  const int bts = fill(wks, WAVES, gb);
  if (bts == 0) return hipSuccess;
  constexpr auto kernel = gemm_mfma_kernel<BITS, SYM, INTER, MB, WAVES>;
  return launch_kernel(kernel, std::min(bts, resident_blocks<kernel, 64 * WAVES>()), gb, stream, 64 * WAVES);
}

// Splits along K for gemm_walk_kernel: the fewest (a power of two) that give
// the launch kWalkBlocks blocks, each split at least one unrolled trip of
// kWalkDepth iterations, within the scratch. Without a scratch every problem
// runs unsplit. Measured on the Llama-3-8B shapes (M = 32 and 64), per layer
// at M = 64: 142.5 us with 160 (gate/up, 224 column groups, unsplit; q/o
// and down 4 splits, k/v 8), 161 us with 320 or 640.
constexpr int kWalkBlocks = 160;

template <int BITS, bool SYM, bool INTER, int MB>
hipError_t launch_gemm_walk(const GemvOperand* ops, int count, int64_t M, void* scratch, hipStream_t stream) {
  constexpr int CPL = 128 / BITS;
  GemmBatch gb{};
  gb.count = count;
  gb.M = static_cast<int>(M);
  const int S = gemm_walk_splits(ops, count, M, BITS, scratch != nullptr);
  GemmBatch sum{};  // the second launch: one block per split column group
  sum.count = count;
  sum.M = gb.M;
  int bts = 0, tiles = 0, sbts = 0;
  for (int i = 0; i < count; ++i) {
    const GemvOperand& o = ops[i];
    GemmProblem& k = gb.p[i];
    k.qweight = o.qweight;
    k.scales = o.scales;
    k.zeros = o.zeros;
    k.x = o.x;
    k.y = o.y;
    k.N = static_cast<int>(o.N);
    k.K = static_cast<int>(o.K);
    k.n_groups = static_cast<int>(o.K / o.group_size);
    k.cpg = static_cast<int>(o.group_size / CPL);
    k.cpg_shift = log2_exact(k.cpg);
    k.n_chunks = static_cast<int>(o.K / CPL);
    k.ldy = static_cast<int>(o.ldy ? o.ldy : o.N);
    const int iters = (k.n_chunks + 3) / 4;
    const int g = static_cast<int>((o.N + kTileCols - 1) / kTileCols);
    k.ips = ((iters + S - 1) / S + kWalkDepth - 1) / kWalkDepth * kWalkDepth;
    k.splits = gemm_problem_splits(o.K, BITS, S);
    k.part_base = tiles;
    gb.bt_start[i] = bts;
    bts += g * k.splits;
    sum.p[i] = k;
    sum.bt_start[i] = sbts;
    if (k.splits > 1) {
      tiles += g * k.splits;
      sbts += g;
    }
  }
  gb.bt_start[count] = bts;
  sum.bt_start[count] = sbts;
  if (bts == 0) return hipSuccess;
  gb.part = sum.part = static_cast<float*>(scratch);
  const hipError_t e = launch_kernel(gemm_walk_kernel<BITS, SYM, INTER, MB>, bts, gb, stream, 256);
  if (e != hipSuccess || sbts == 0) return e;
  return launch_kernel(gemm_split_sum_kernel<MB>, sbts, sum, stream, 256);
}

template <int BITS, bool SYM, bool INTER>
hipError_t launch_gemm_t(const GemvOperand* ops, int count, int64_t M, void* scratch, hipStream_t stream) {
  if (M > 32) return launch_gemm_walk<BITS, SYM, INTER, 4>(ops, count, M, scratch, stream);
  if (M > 16) return launch_gemm_walk<BITS, SYM, INTER, 2>(ops, count, M, scratch, stream);
  if (M <= 16) return launch_gemm_mb<BITS, SYM, INTER, 1>(ops, count, M, stream);
  if (M <= 32) return launch_gemm_mb<BITS, SYM, INTER, 2>(ops, count, M, stream);
  return launch_gemm_mb<BITS, SYM, INTER, 4>(ops, count, M, stream);
}

// Batches of 2 rows run gemv_mx_pipe_kernel<..., MX = 2> when the M = 1 rule
// gives every problem one-wave tiles; the others run gemv_quad_kernel.
// Measured on the C4 stack: M = 2 25.29 -> 22.82 us/layer; at M = 4 the
// four-row instance (192 VGPRs, two waves per SIMD) ran 33.3 us/layer
// against the quad kernel's 26.8, so M >= 3 stays there.
constexpr bool mx_pipe_fits(int, int64_t M) { return M == 2; }

bool mx_pipe_plan(const GemvOperand* ops, int count, int64_t M, int bits, int* R, int* wks) {
  if (!mx_pipe_fits(bits, M)) return false;
  *R = rows_per_tile(ops, count);
  waves_per_tile(ops, count, bits, *R, wks);
  for (int i = 0; i < count; ++i)
    if (wks[i] != 1) return false;
  return true;
}

template <int BITS, bool SYM, bool INTER, int R, int MX>
hipError_t launch_gemv_mx(const GemvOperand* ops, int count, int64_t M, const int* wks, hipStream_t stream) {
  KernelBatch kb;
  const int bts = fill_kernel_batch(ops, count, M, BITS, R, 1, wks, kb);
  if (bts == 0) return hipSuccess;
  constexpr auto kernel = gemv_mx_pipe_kernel<BITS, SYM, INTER, R, MX>;
  return launch_kernel(kernel, std::min(bts, resident_blocks<kernel>()), kb, stream);
}

template <int BITS, bool SYM, bool INTER>
hipError_t launch_gemv_t(const GemvOperand* ops, int count, int64_t M, hipStream_t stream) {
  if (M == 1) {
    if (rows_per_tile(ops, count) == 8) return launch_gemv_m1<BITS, SYM, INTER, 8>(ops, count, M, stream);
    return launch_gemv_m1<BITS, SYM, INTER, 4>(ops, count, M, stream);
  }
  int R = 0, wks[kMaxBatch];
  if (mx_pipe_plan(ops, count, M, BITS, &R, wks)) {
    return R == 8 ? launch_gemv_mx<BITS, SYM, INTER, 8, 2>(ops, count, M, wks, stream)
                  : launch_gemv_mx<BITS, SYM, INTER, 4, 2>(ops, count, M, wks, stream);
  }
  if (M <= 4) return launch_gemv_quad<BITS, SYM, INTER, 1>(ops, count, M, stream);
  return launch_gemv_quad<BITS, SYM, INTER, 2>(ops, count, M, stream);
}

template <int BITS, bool SYM, bool INTER>
hipError_t launch_gemv_prologue_t(const GemvOperand* ops, int count, int64_t M, int prologue, float eps,
                                  hipStream_t stream) {
  if (M != 1) return hipErrorInvalidValue;
  // 8-row tiles where the plain rule would pick 4 for a prologue's sake: each
  // tile recomputes the prologue of its chunk columns (SwiGLU: two
  // transcendentals per activation), so twice the rows per tile halve that
  // work. Measured on the Llama-3-8B decode launches: down_proj with SwiGLU
  // 12.6 -> 11.3 us, gate|up with RMSNorm 16.1 -> 14.7 us; q|k|v with RMSNorm
  // (768 tiles of 8 rows) 6.6 -> 6.9 us, so RMSNorm keeps the plain rule below
  // kProWideTiles.
  int64_t tiles8 = 0;
  for (int i = 0; i < count; ++i) tiles8 += (ops[i].N + 7) / 8;
  const bool wide_tiles =
      rows_per_tile(ops, count) == 8 || prologue == kPrologueSwiGlu || tiles8 >= kProWideTiles;
  if (prologue == kPrologueRmsNorm) {
    // RMSNorm launches whose 4-row tiles are one wave wide (the decode step's
    // gate | up) keep the plain rule: launch_gemv_m1 runs them on the
    // pipelined kernel, which applies the prologue once per block and batch.
    // Measured on the Llama-3-8B decode gate | up launch: 14.1 us with 8-row
    // tiles (split-K, gemv_m1_kernel) against 12.3 us for the plain launch.
    int wks[kMaxBatch];
    waves_per_tile(ops, count, BITS, 4, wks);
    bool one_wave = rows_per_tile(ops, count) == 4;
    for (int i = 0; i < count; ++i) one_wave = one_wave && wks[i] == 1;
    return wide_tiles && !one_wave ? launch_gemv_m1<BITS, SYM, INTER, 8, kProRmsNorm>(ops, count, M, stream, eps)
                                   : launch_gemv_m1<BITS, SYM, INTER, 4, kProRmsNorm>(ops, count, M, stream, eps);
  }
  if (prologue == kPrologueSwiGlu) {
    // SwiGLU launches whose plain-rule tiles are one wave wide (down_proj at
    // decode) take the pipelined kernel, which forms the prologue once per
    // block and batch; the others keep 8-row tiles.
    int wks[kMaxBatch];
    m1_waves_per_tile(ops, count, BITS, rows_per_tile(ops, count), wks);
    bool one_wave = rows_per_tile(ops, count) == 4;
    for (int i = 0; i < count; ++i) one_wave = one_wave && wks[i] == 1;
    return wide_tiles && !one_wave ? launch_gemv_m1<BITS, SYM, INTER, 8, kProSwiGlu>(ops, count, M, stream)
                                   : launch_gemv_m1<BITS, SYM, INTER, 4, kProSwiGlu>(ops, count, M, stream);
  }
  return hipErrorInvalidValue;
}

template <int BITS, bool SYM, bool INTER>
hipError_t launch_dequantize_t(const DequantProblem& p, hipStream_t stream) {
  constexpr int PER = 32 / BITS;
  const int64_t wpr = p.K / PER;
  const int64_t wpg = p.group_size / PER;
  const int gshift = p.group_size == p.K ? 0 : log2_exact(wpg);
  // x: enough blocks to cover a row's words (up to 4 per CU's worth); y: rows,
  // walked with a stride beyond 65535
  const int gx = static_cast<int>(std::min<int64_t>((wpr + kElemThreads - 1) / kElemThreads, 64));
  const int gy = static_cast<int>(std::min<int64_t>(p.N, 65535));
  hipLaunchKernelGGL((dequantize_kernel<BITS, SYM, INTER>), dim3(gx, gy), dim3(kElemThreads), 0, stream, p.qweight,
                     p.scales, p.zeros, p.out, static_cast<int>(p.N), static_cast<int>(p.K),
                     static_cast<int>(p.group_size), gshift);
  return hipGetLastError();
}

template <int BITS, bool INTER>
hipError_t launch_unpack_t(const uint32_t* qweight, int32_t* out, int64_t N, int64_t K, hipStream_t stream) {
  const int64_t total = N * (K / (32 / BITS));
  hipLaunchKernelGGL((unpack_kernel<BITS, INTER>), dim3(elementwise_blocks(total)), dim3(kElemThreads), 0, stream,
                     qweight, out, total, static_cast<int>(K));
  return hipGetLastError();
}

}  // namespace

// bits x symmetric x interleaved -> one of 12 instantiations (the reference's
// DISPATCH_VARIANT, kernels/dequant_gemv.cu:285-306).
#define DQ_DISPATCH_12(BITS_, SYM_, INTER_, CALL)                              \
  switch ((BITS_) << 2 | ((SYM_) ? 2 : 0) | ((INTER_) ? 1 : 0)) {              \
    case (2 << 2 | 0): return CALL(2, false, false);                           \
    case (2 << 2 | 1): return CALL(2, false, true);                            \
    case (2 << 2 | 2): return CALL(2, true, false);                            \
    case (2 << 2 | 3): return CALL(2, true, true);                             \
    case (4 << 2 | 0): return CALL(4, false, false);                           \
    case (4 << 2 | 1): return CALL(4, false, true);                            \
    case (4 << 2 | 2): return CALL(4, true, false);                            \
    case (4 << 2 | 3): return CALL(4, true, true);                             \
    case (8 << 2 | 0): return CALL(8, false, false);                           \
    case (8 << 2 | 1): return CALL(8, false, true);                            \
    case (8 << 2 | 2): return CALL(8, true, false);                            \
    case (8 << 2 | 3): return CALL(8, true, true);                             \
    default: return hipErrorInvalidValue;                                      \
  }

void plan_gemv_batch(const GemvOperand* ops, int count, int64_t M, int bits, int* wk, int* rows, int* mfma) {
  if (mx_pipe_plan(ops, count, M, bits, rows, wk)) {
    *mfma = 7;
    return;
  }
  if (M >= 2) {
    *mfma = 1;
    *rows = 4 * kQuadsPerTile;
    const int w = quad_waves_per_tile(ops, count, bits, M <= 4 ? 1 : 2);
    for (int i = 0; i < count; ++i) wk[i] = w;
    return;
  }
  *mfma = M == 1 ? (m1_uses_mfma(bits) ? 3 : 2) : 0;
  *rows = rows_per_tile(ops, count);
  if (M == 1) m1_waves_per_tile(ops, count, bits, *rows, wk);
  else waves_per_tile(ops, count, bits, *rows, wk);
  if (M == 1 && !m1_uses_mfma(bits)) {
    // the INT2 kept variant holds four blocks per CU; the launch
    // itself asks the device for its kernel's co-resident blocks
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
      (void)hipGetLastError();
      cus = 256;
    }
    KernelBatch kb;
    const int bts = fill_kernel_batch(ops, count, M, bits, *rows, 1, wk, kb);
    *mfma = m1_variant(kb, count, bits, *rows, wk, bts, 4 * cus);
    if (*mfma == kM1Load && pipe_split(bits, *rows, wk, count, bts)) *mfma = 8;
  }
}

void set_launch_events(hipEvent_t start, hipEvent_t stop) {
  t_start_event = start;
  t_stop_event = stop;
}

hipError_t launch_gemv_batch(const GemvOperand* ops, int count, int64_t M, int bits, bool symmetric,
                             bool interleaved, hipStream_t stream) {
  if (count < 1 || count > kMaxBatch) return hipErrorInvalidValue;
#define DQ_CALL_GEMV(B, S, I) launch_gemv_t<B, S, I>(ops, count, M, stream)
  DQ_DISPATCH_12(bits, symmetric, interleaved, DQ_CALL_GEMV)
#undef DQ_CALL_GEMV
}

hipError_t launch_gemv_prologue_batch(const GemvOperand* ops, int count, int64_t M, int bits, bool symmetric,
                                      bool interleaved, int prologue, float eps, hipStream_t stream) {
  if (count < 1 || count > kMaxBatch) return hipErrorInvalidValue;
#define DQ_CALL_PRO(B, S, I) launch_gemv_prologue_t<B, S, I>(ops, count, M, prologue, eps, stream)
  DQ_DISPATCH_12(bits, symmetric, interleaved, DQ_CALL_PRO)
#undef DQ_CALL_PRO
}

int gemm_walk_splits(const GemvOperand* ops, int count, int64_t M, int bits, bool scratch) {
  if (M <= 16 || !scratch) return 1;
  const int64_t cpl = 128 / bits;
  const int64_t tile = 16 * (M > 32 ? 4 : 2) * kTileCols;
  int64_t groups = 0, min_iters = INT64_MAX;
  for (int i = 0; i < count; ++i) {
    groups += (ops[i].N + kTileCols - 1) / kTileCols;
    min_iters = std::min<int64_t>(min_iters, (ops[i].K / cpl + 3) / 4);
  }
  int S = 1;
  while (groups * S < kWalkBlocks && min_iters / (2 * S) >= kWalkDepth && groups * 2 * S * tile * 4 <= kGemmScratchBytes)
    S *= 2;
  return S;
}

int gemm_problem_splits(int64_t K, int bits, int S) {
  const int iters = static_cast<int>((K / (128 / bits) + 3) / 4);
  const int ips = ((iters + S - 1) / S + kWalkDepth - 1) / kWalkDepth * kWalkDepth;
  return (iters + ips - 1) / ips;
}

// Scratch of dq_gemm_small_noalloc, for callers that cannot allocate: the
// small GEMM's split partial tiles in a static device array, one per GPU,
// held until the process ends. Host code never passes the array's name to a
// kernel (on the host it stands for no device address): its address on each
// device comes from hipGetSymbolAddress, taken once per device with that
// device current, and every launch gets that pointer. Nothing in it needs
// initial contents (a launch writes each partial tile before the next launch
// reads it); launches that use it and overlap on one GPU race.
static __device__ __align__(256) unsigned char scratch[kGemmScratchBytes];

hipError_t gemm_static_scratch(void** out) {
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    addr[dev] = p;
  }
  *out = addr[dev];
  return hipSuccess;
}

hipError_t launch_gemm_batch(const GemvOperand* ops, int count, int64_t M, int bits, bool symmetric,
                             bool interleaved, void* scratch, hipStream_t stream) {
  if (count < 1 || count > kMaxBatch || M < 1 || M > kMaxGemmM) return hipErrorInvalidValue;
#define DQ_CALL_GEMM(B, S, I) launch_gemm_t<B, S, I>(ops, count, M, scratch, stream)
  DQ_DISPATCH_12(bits, symmetric, interleaved, DQ_CALL_GEMM)
#undef DQ_CALL_GEMM
}


hipError_t launch_dequantize(const DequantProblem& p, hipStream_t stream) {
#define DQ_CALL_DEQ(B, S, I) launch_dequantize_t<B, S, I>(p, stream)
  DQ_DISPATCH_12(p.bits, p.symmetric, p.interleaved, DQ_CALL_DEQ)
#undef DQ_CALL_DEQ
}

hipError_t launch_unpack(const uint32_t* qweight, int32_t* out, int64_t N, int64_t K, int bits, bool interleaved,
                         hipStream_t stream) {
  switch (bits << 1 | (interleaved ? 1 : 0)) {
    case (2 << 1 | 0): return launch_unpack_t<2, false>(qweight, out, N, K, stream);
    case (2 << 1 | 1): return launch_unpack_t<2, true>(qweight, out, N, K, stream);
    case (4 << 1 | 0): return launch_unpack_t<4, false>(qweight, out, N, K, stream);
    case (4 << 1 | 1): return launch_unpack_t<4, true>(qweight, out, N, K, stream);
    case (8 << 1 | 0): return launch_unpack_t<8, false>(qweight, out, N, K, stream);
    case (8 << 1 | 1): return launch_unpack_t<8, true>(qweight, out, N, K, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_stream_read(const void* data, int64_t bytes, uint32_t* sink, hipStream_t stream) {
  const int grid = resident_blocks<stream_read_kernel>();
  hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(256), 0, stream, static_cast<const unsigned char*>(data),
                     bytes, sink);
  return hipGetLastError();
}

hipError_t launch_empty(hipStream_t stream) {
  hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, stream);
  return hipGetLastError();
}

hipError_t launch_add_one(const float* in, float* out, int64_t n, hipStream_t stream) {
  hipLaunchKernelGGL(add_one_kernel, dim3(elementwise_blocks(n)), dim3(kElemThreads), 0, stream, in, out, n);
  return hipGetLastError();
}

}  // namespace dq

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
//   gemv_kernel        <- gemv_kernel<BITS,SYM,INTER,MT>       :144-217
//   dequantize_kernel  <- dequantize_kernel<BITS,SYM,INTER>    :113-140
//   unpack_kernel      (new: exposes the unpack step for bit-exact checks)
//   add_one_kernel     <- kernels/smoke.cu:9-13
//
// GEMV design (CDNA4, wave64):
//   * One launch takes a list of up to 16 problems of one format (a single
//     call is a list of one; q|k|v or gate|up of a decoder layer share one
//     launch). Work is cut into tiles of R rows; a 256-thread block holds
//     4/wk tiles and the wk waves of a tile split its K range, meeting in LDS.
//   * Lane l walks the 16-byte chunks cb + l + 64t of its rows, so every
//     global_load_dwordx4 of a wave reads 1 KiB of one row contiguously. A
//     chunk holds 128/BITS codes of one group (group_size % (128/BITS) == 0).
//     Every weight, scale and zero load of up to CMAX chunk columns is issued
//     before any math (R*CMAX 16-byte loads in flight per lane); with M = 1
//     the activations of those columns are gathered up front too.
//   * Unpack to exact fp16 (code - zero) pairs in two VALU ops per pair:
//       v_and_or_b32  (w & mask) | 0x64006400  -> fp16 (1024 + q * 2^p) in both
//                     halves (q sits in mantissa bits [p, p+BITS), p <= 8);
//       v_pk_fma_f16  * 2^-p - (2^(10-p) + z)  -> fp16 (q - z), exact.
//     (INT8 builds the 0x64qq halves with one v_perm_b32 instead.) Pair i holds
//     the word's slots (i, i + PER/2); the activations are gathered into the
//     same pair order, so sequential and interleaved layouts cost the same.
//   * v_dot2_f32_f16 multiplies a (q - z) pair with an activation pair and
//     accumulates in fp32; per chunk, acc * scale is added in fp32 -- the
//     reference's arithmetic (fp32 accumulation of exact (q - z) * x products,
//     factorized scale), so the reference's elementwise fp32 error bound holds.
//   * Zero points outside [-1024, 1024] (possible: the packer stores them
//     unclamped) cannot use the exact fp16 form; such chunks take q exactly and
//     subtract z * sum(x) in fp32 instead (uniform branch, rare).
//   * Rows are finished with a DPP wave64 reduction (row_shr 1/2/4/8,
//     row_bcast 15/31) instead of an LDS tree; fp16 (RNE) stores.
//
// All kernels are written for gfx950 only; no other target is built.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "dq_internal.h"

namespace dq {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

// Word -> PER/2 magic pairs: both fp16 halves of pair i are 1024 + q * 2^p,
// the low half from slot i, the high half from slot i + PER/2.
template <int BITS>
__device__ __forceinline__ void magic_pairs(uint32_t w, uint32_t* p) {
  constexpr uint32_t kMagic = 0x64006400u;
  if constexpr (BITS == 8) {
    p[0] = __builtin_amdgcn_perm(0x64646464u, w, 0x04020400u);  // {0x64, b2, 0x64, b0}
    p[1] = __builtin_amdgcn_perm(0x64646464u, w, 0x04030401u);  // {0x64, b3, 0x64, b1}
  } else if constexpr (BITS == 4) {
    p[0] = (w & 0x000F000Fu) | kMagic;
    p[1] = (w & 0x00F000F0u) | kMagic;
    const uint32_t w8 = w >> 8;
    p[2] = (w8 & 0x000F000Fu) | kMagic;
    p[3] = (w8 & 0x00F000F0u) | kMagic;
  } else {
#pragma unroll
    for (int i = 0; i < 5; ++i) p[i] = (w & (0x00030003u << (2 * i))) | kMagic;
    const uint32_t w10 = w >> 10;
#pragma unroll
    for (int i = 0; i < 3; ++i) p[5 + i] = (w10 & (0x00030003u << (2 * i))) | kMagic;
  }
}

// Per (row, chunk) constants turning magic pairs of class c into (q - z):
// (1024 + q 2^p) * 2^-p + off[c] with off[c] = -(2^(10-p) + z). When z is
// outside [-1024, 1024] the exact fp16 form is unavailable; then off[c]
// yields q alone and the caller subtracts z * sum(x) in fp32.
template <int BITS>
__device__ __forceinline__ bool class_offsets(float z, h2* off) {
  using F = Fmt<BITS>;
  const bool exact = __builtin_fabsf(z) <= 1024.0f;  // z is an integer or not finite
  const _Float16 zh = exact ? static_cast<_Float16>(z) : static_cast<_Float16>(0.0f);
#pragma unroll
  for (int c = 0; c < F::NCLS; ++c) {
    const _Float16 base = static_cast<_Float16>(static_cast<float>(1 << (10 - F::class_pow(c))));
    off[c] = splat(-(base + zh));  // exact: |base + z| <= 2048
  }
  return exact;
}

// ------------------------------------------------------------ wave reduction
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the 64 lanes of a wave; the total lands in lane 63.
__device__ __forceinline__ float wave_sum_lane63(float v) {
  v += dpp_move<0x111, 0xf>(v);  // row_shr:1
  v += dpp_move<0x112, 0xf>(v);  // row_shr:2
  v += dpp_move<0x114, 0xf>(v);  // row_shr:4
  v += dpp_move<0x118, 0xf>(v);  // row_shr:8   -> lane 16r+15 holds row r's sum
  v += dpp_move<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
  v += dpp_move<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
  return v;
}

// ---------------------------------------------------------------------- gemv
constexpr int kGemvThreads = 256;  // 4 waves
constexpr int kWavesPerBlock = kGemvThreads / 64;

// Gather the PER activations of word j of chunk c for batch row m into pair order.
template <int BITS, bool INTER>
__device__ __forceinline__ void load_x_pairs(const uint16_t* __restrict__ xw, h2* xp) {
  using F = Fmt<BITS>;
  uint16_t xv[F::PER];
  if constexpr (F::PER == 4) {
    const uint2 t = *reinterpret_cast<const uint2*>(xw);
    xv[0] = t.x & 0xFFFF; xv[1] = t.x >> 16; xv[2] = t.y & 0xFFFF; xv[3] = t.y >> 16;
  } else {
#pragma unroll
    for (int q = 0; q < F::PER / 8; ++q) {
      const uint4 t = *reinterpret_cast<const uint4*>(xw + 8 * q);
      const uint32_t u[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xv[8 * q + 2 * e] = u[e] & 0xFFFF;
        xv[8 * q + 2 * e + 1] = u[e] >> 16;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < F::PAIRS; ++i) {
    const uint32_t lo = xv[logical_of_slot<BITS, INTER>(i)];
    const uint32_t hi = xv[logical_of_slot<BITS, INTER>(i + F::PAIRS)];
    xp[i] = as_h2(lo | (hi << 16));
  }
}

// Launch-wide description of up to kMaxBatch problems (passed by value).
struct KernelProblem {
  const uint32_t* qweight;
  const uint16_t* scales;
  const uint16_t* zeros;
  const uint16_t* x;
  uint16_t* y;
  int N, K;
  int n_groups;          // K / group_size
  int chunks_per_group;  // group_size / (128/BITS)
  int n_chunks;          // K / (128/BITS)
  int wk;                // waves sharing one tile along K (1, 2 or 4)
  int tiles;             // ceil(N / R)
};

struct KernelBatch {
  KernelProblem p[kMaxBatch];
  int block_start[kMaxBatch + 1];  // blocks never mix problems
  int count;
  int M;
};

// One wave's share of a tile: rows row0 .. row0+R-1 of problem d, chunks
// [cb, ce) of each row. Lane l takes chunks cb + l + 64 t. All weight, scale
// and zero loads of a batch of CMAX columns are issued before any math, so a
// lane has R*CMAX 16-byte loads in flight; for M = 1 the activations of the
// batch are gathered up front as well.
template <int BITS, bool SYM, bool INTER, int MT, int R, int CMAX>
__device__ __forceinline__ void gemv_tile(const KernelProblem& d, int M, int row0, int cb, int ce, int lane,
                                          float (&yacc)[R][MT]) {
  using F = Fmt<BITS>;
  const int64_t words_per_row = d.K / F::PER;
  const uint32_t* wrow[R];
  int64_t moff[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(row0 + r, d.N - 1);  // rows past N re-read row N-1 and are never stored
    wrow[r] = d.qweight + row * words_per_row;
    moff[r] = static_cast<int64_t>(row) * d.n_groups;
  }

  h2 pow_scale[F::NCLS];
#pragma unroll
  for (int c = 0; c < F::NCLS; ++c)
    pow_scale[c] = splat(static_cast<_Float16>(__builtin_ldexpf(1.0f, -F::class_pow(c))));
  const h2 ones = splat(static_cast<_Float16>(1.0f));

  for (int c0 = cb + lane; c0 < ce; c0 += 64 * CMAX) {
    // ---- issue every load of the batch
    u32x4 wv[CMAX][R];
    uint16_t sraw[CMAX][R], zraw[CMAX][R];
    h2 xq[MT == 1 ? CMAX : 1][MT == 1 ? 4 : 1][F::PAIRS];
#pragma unroll
    for (int t = 0; t < CMAX; ++t) {
      const int c = c0 + 64 * t;
      if (c < ce) {
        const int g = c / d.chunks_per_group;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          // weights are read exactly once: stream them past the caches
          wv[t][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[r] + 4 * c));
          sraw[t][r] = d.scales[moff[r] + g];
          if (!SYM) zraw[t][r] = d.zeros[moff[r] + g];
        }
        if constexpr (MT == 1) {
#pragma unroll
          for (int j = 0; j < 4; ++j) load_x_pairs<BITS, INTER>(d.x + c * F::CPL + j * F::PER, xq[t][j]);
        }
      }
    }

    // ---- math, one column at a time
#pragma unroll
    for (int t = 0; t < CMAX; ++t) {
      const int c = c0 + 64 * t;
      if (c < ce) {
        float sc[R], zf[R];
        h2 off[R][F::NCLS];
        bool any_inexact = false;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          sc[r] = f16_to_f32(sraw[t][r]);
          zf[r] = SYM ? static_cast<float>(F::BIAS) : f16_to_f32(zraw[t][r]);
          const bool exact = class_offsets<BITS>(zf[r], off[r]);
          if (!SYM) {
            if (exact) zf[r] = 0.f;
            any_inexact |= !exact;
          }
        }
        // uniform over the lanes of this column: does any need sum(x)?
        const bool need_xsum = !SYM && __builtin_amdgcn_ballot_w64(any_inexact) != 0;

        float acc[R][MT], xsum[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          xsum[m] = 0.f;
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r][m] = 0.f;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          h2 xp[MT][F::PAIRS];
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            if (MT == 1 || m < M) {
              if constexpr (MT == 1) {
#pragma unroll
                for (int i = 0; i < F::PAIRS; ++i) xp[m][i] = xq[t][j][i];
              } else {
                load_x_pairs<BITS, INTER>(d.x + static_cast<int64_t>(m) * d.K + c * F::CPL + j * F::PER, xp[m]);
              }
              if (need_xsum) {
#pragma unroll
                for (int i = 0; i < F::PAIRS; ++i) xsum[m] = __builtin_amdgcn_fdot2(xp[m][i], ones, xsum[m], false);
              }
            }
          }
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const uint32_t w = wv[t][r][j];
            uint32_t mp[F::PAIRS];
            magic_pairs<BITS>(w, mp);
            h2 dq2[F::PAIRS];
#pragma unroll
            for (int i = 0; i < F::PAIRS; ++i)
              dq2[i] = __builtin_elementwise_fma(as_h2(mp[i]), pow_scale[F::cls(i)], off[r][F::cls(i)]);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
              if (MT == 1 || m < M) {
#pragma unroll
                for (int i = 0; i < F::PAIRS; ++i) acc[r][m] = __builtin_amdgcn_fdot2(dq2[i], xp[m][i], acc[r][m], false);
              }
            }
          }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            const float u = need_xsum ? __builtin_fmaf(-zf[r], xsum[m], acc[r][m]) : acc[r][m];
            yacc[r][m] = __builtin_fmaf(sc[r], u, yacc[r][m]);
          }
        }
      }
    }
  }
}

// Grouped fused dequant + GEMV. A block (4 waves) belongs to one problem and
// holds 4/wk tiles of it; a tile is R rows whose K range is split over wk
// waves meeting in LDS. wk depends only on the problem's own K, so a problem
// gives bit-identical results whether launched alone or in a group.
template <int BITS, bool SYM, bool INTER, int MT, int R, int CMAX>
__global__ void __launch_bounds__(kGemvThreads)
gemv_batched_kernel(const KernelBatch b) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int p = 0;
  while (p + 1 < b.count && static_cast<int>(blockIdx.x) >= b.block_start[p + 1]) ++p;
  const KernelProblem& d = b.p[p];
  const int wk = d.wk;
  const int slot = wave / wk;
  const int kw = wave - slot * wk;
  const int tile = (static_cast<int>(blockIdx.x) - b.block_start[p]) * (kWavesPerBlock / wk) + slot;
  const bool active = tile < d.tiles;
  const int row0 = tile * R;

  float yacc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) yacc[r][m] = 0.f;

  if (active) {
    const int per_wave = (d.n_chunks + wk - 1) / wk;
    const int cb = kw * per_wave;
    const int ce = min(d.n_chunks, cb + per_wave);
    gemv_tile<BITS, SYM, INTER, MT, R, CMAX>(d, b.M, row0, cb, ce, lane, yacc);
  }

  if (wk == 1) {
    // the wave owns the whole row: lane 63 stores
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float v = wave_sum_lane63(yacc[r][m]);
        if (active && lane == 63 && row0 + r < d.N && (MT == 1 || m < b.M))
          d.y[static_cast<int64_t>(m) * d.N + row0 + r] = f32_to_f16_rn(v);
      }
  } else {
    __shared__ float partial[kWavesPerBlock][R * MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float v = wave_sum_lane63(yacc[r][m]);
        if (lane == 63) partial[wave][r * MT + m] = v;
      }
    __syncthreads();  // every wave of the block reaches this (no early exit above)
    if (active && kw == 0 && lane < R * MT) {
      float v = 0.f;
      for (int j = 0; j < wk; ++j) v += partial[wave + j][lane];
      const int r = lane / MT, m = lane - (lane / MT) * MT;
      if (row0 + r < d.N && m < b.M) d.y[static_cast<int64_t>(m) * d.N + row0 + r] = f32_to_f16_rn(v);
    }
  }
}

// ---------------------------------------------------------------- dequantize
constexpr int kElemThreads = 256;

template <int BITS, bool SYM, bool INTER>
__global__ void __launch_bounds__(kElemThreads)
dequantize_kernel(const uint32_t* __restrict__ qweight, const uint16_t* __restrict__ scales,
                  const uint16_t* __restrict__ zeros, uint16_t* __restrict__ out,
                  int64_t total_words, int K, int group_size) {
  using F = Fmt<BITS>;
  const int64_t words_per_row = K / F::PER;
  const int ng = K / group_size;
  for (int64_t widx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; widx < total_words;
       widx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = widx / words_per_row;
    const int k0 = static_cast<int>(widx - n * words_per_row) * F::PER;
    const int64_t gidx = n * ng + k0 / group_size;  // group_size % PER == 0: one group per word
    const float s = f16_to_f32(scales[gidx]);
    const float off = SYM ? static_cast<float>(F::BIAS) : f16_to_f32(zeros[gidx]);
    const uint32_t w = qweight[widx];
    uint16_t v[F::PER];
#pragma unroll
    for (int sl = 0; sl < F::PER; ++sl) {
      const float code = static_cast<float>((w >> (BITS * sl)) & ((1u << BITS) - 1u));
      // (code - off) then a separate fp32 multiply, then fp16 RNE: packer.py:183-189
      const float d = code - off;
      v[logical_of_slot<BITS, INTER>(sl)] = f32_to_f16_rn(__fmul_rn(d, s));
    }
    uint16_t* o = out + n * K + k0;
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


// ----------------------------------------------------------------- launchers
namespace {

int64_t elementwise_blocks(int64_t items) {
  const int64_t b = (items + kElemThreads - 1) / kElemThreads;
  return b < 1 ? 1 : (b > 65536 ? 65536 : b);  // grid-stride loops cover the rest
}

// Launch geometry of a grouped GEMV:
//   wk   per problem, waves per tile along K: the fewest of {1, 2, 4} that
//        leave each lane at most CMAX 16-byte columns of its row (one batch of
//        loads); it depends on the problem's K alone;
//   R    rows per tile, shared by the launch: 4 (activations reused 4x) unless
//        that leaves fewer than two waves per SIMD on the 1024 SIMDs of an
//        MI355X, then 2 or 1. R does not change any row's arithmetic.
constexpr int kCmax = 2;

int waves_per_tile(int64_t K, int bits) {
  const int64_t chunks = K / (128 / bits);
  int wk = 1;
  while (wk < 4 && (chunks + wk - 1) / wk > 64 * kCmax) wk *= 2;
  return wk;
}

int rows_per_tile(const GemvOperand* ops, int count, int64_t M, int bits) {
  if (M > 1) return 1;
  constexpr int64_t kTargetWaves = 2048;
  int R = 4;
  for (; R > 1; R /= 2) {
    int64_t waves = 0;
    for (int i = 0; i < count; ++i) waves += (ops[i].N + R - 1) / R * waves_per_tile(ops[i].K, bits);
    if (waves >= kTargetWaves) break;
  }
  return R;
}

thread_local hipEvent_t t_start_event = nullptr, t_stop_event = nullptr;

template <int BITS, bool SYM, bool INTER, int MT, int R>
hipError_t launch_batch_t(const KernelBatch& kb, hipStream_t stream) {
  const int blocks = kb.block_start[kb.count];
  if (t_start_event && t_stop_event) {
    hipExtLaunchKernelGGL((gemv_batched_kernel<BITS, SYM, INTER, MT, R, kCmax>), dim3(blocks), dim3(kGemvThreads),
                          0, stream, t_start_event, t_stop_event, 0, kb);
    t_start_event = t_stop_event = nullptr;
  } else {
    hipLaunchKernelGGL((gemv_batched_kernel<BITS, SYM, INTER, MT, R, kCmax>), dim3(blocks), dim3(kGemvThreads), 0,
                       stream, kb);
  }
  return hipGetLastError();
}

template <int BITS, bool SYM, bool INTER, int MT, int R>
hipError_t launch_gemv_r(const GemvOperand* ops, int count, int64_t M, hipStream_t stream) {
  constexpr int CPL = 128 / BITS;
  KernelBatch kb{};
  kb.count = count;
  kb.M = static_cast<int>(M);
  int blocks = 0;
  for (int i = 0; i < count; ++i) {
    const GemvOperand& o = ops[i];
    KernelProblem& k = kb.p[i];
    k.qweight = o.qweight;
    k.scales = o.scales;
    k.zeros = o.zeros;
    k.x = o.x;
    k.y = o.y;
    k.N = static_cast<int>(o.N);
    k.K = static_cast<int>(o.K);
    k.n_groups = static_cast<int>(o.K / o.group_size);
    k.chunks_per_group = static_cast<int>(o.group_size / CPL);
    k.n_chunks = static_cast<int>(o.K / CPL);
    k.wk = waves_per_tile(o.K, BITS);
    k.tiles = static_cast<int>((o.N + R - 1) / R);
    const int tiles_per_block = kWavesPerBlock / k.wk;
    kb.block_start[i] = blocks;
    blocks += (k.tiles + tiles_per_block - 1) / tiles_per_block;
  }
  kb.block_start[count] = blocks;
  if (blocks == 0) return hipSuccess;
  return launch_batch_t<BITS, SYM, INTER, MT, R>(kb, stream);
}

template <int BITS, bool SYM, bool INTER>
hipError_t launch_gemv_t(const GemvOperand* ops, int count, int64_t M, hipStream_t stream) {
  if (M == 1) {
    const int R = rows_per_tile(ops, count, M, BITS);
    if (R == 4) return launch_gemv_r<BITS, SYM, INTER, 1, 4>(ops, count, M, stream);
    if (R == 2) return launch_gemv_r<BITS, SYM, INTER, 1, 2>(ops, count, M, stream);
    return launch_gemv_r<BITS, SYM, INTER, 1, 1>(ops, count, M, stream);
  }
  if (M == 2) return launch_gemv_r<BITS, SYM, INTER, 2, 1>(ops, count, M, stream);
  if (M <= 4) return launch_gemv_r<BITS, SYM, INTER, 4, 1>(ops, count, M, stream);
  return launch_gemv_r<BITS, SYM, INTER, 8, 1>(ops, count, M, stream);
}

template <int BITS, bool SYM, bool INTER>
hipError_t launch_dequantize_t(const DequantProblem& p, hipStream_t stream) {
  const int64_t total = p.N * (p.K / (32 / BITS));
  hipLaunchKernelGGL((dequantize_kernel<BITS, SYM, INTER>), dim3(elementwise_blocks(total)), dim3(kElemThreads),
                     0, stream, p.qweight, p.scales, p.zeros, p.out, total, static_cast<int>(p.K),
                     static_cast<int>(p.group_size));
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

void plan_gemv_batch(const GemvOperand* ops, int count, int64_t M, int bits, int* wk, int* rows) {
  for (int i = 0; i < count; ++i) wk[i] = waves_per_tile(ops[i].K, bits);
  *rows = rows_per_tile(ops, count, M, bits);
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

hipError_t launch_add_one(const float* in, float* out, int64_t n, hipStream_t stream) {
  hipLaunchKernelGGL(add_one_kernel, dim3(elementwise_blocks(n)), dim3(kElemThreads), 0, stream, in, out, n);
  return hipGetLastError();
}

}  // namespace dq

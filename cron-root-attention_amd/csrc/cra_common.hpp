// Shared building blocks for the gfx950 kernels: element types, MFMA
// fragments, LDS tile staging and the sqrt(N) index geometry.
//
// MFMA shape used everywhere: v_mfma_f32_16x16x32_{f16,bf16} (fp32 inputs:
// eight v_mfma_f32_16x16x4_f32). Register layout of one wave (64 lanes),
// l16 = lane % 16, g = lane / 16:
//   A operand (16 x 32):  lane holds A[row = l16][k = kappa(g, s)], s = 0..7
//   B operand (32 x 16):  lane holds B[k = kappa(g, s)][col = l16]
//   C result  (16 x 16):  lane holds C[row = 4g + r][col = l16], r = 0..3
// Any bijection kappa works as long as A and B use the same one; a fragment
// loaded from a row-major tile uses kappa(g, s) = 8g + s, a fragment built
// from two C results (rows 16kb0.. and 16kb1..) uses
// kappa(g, s) = 16kb0 + 4g + s (s < 4), 16kb1 + 4g + s - 4 (s >= 4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cra {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

static constexpr float kLog2e = 1.4426950408889634f;
static constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------
// Eight-element operand fragment, stored as raw 16-byte words.
// ---------------------------------------------------------------------------
template <typename T>
struct Frag {
  static constexpr int kWords = sizeof(T) / 2;  // 16-byte words: 1 (f16/bf16) or 2 (f32)
  uint4 w[kWords];
};

__device__ __forceinline__ f32x4 mma(f32x4 c, const Frag<f16>& a, const Frag<f16>& b) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a.w[0]),
                                                __builtin_bit_cast(f16x8, b.w[0]), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma(f32x4 c, const Frag<bf16>& a, const Frag<bf16>& b) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a.w[0]),
                                                 __builtin_bit_cast(bf16x8, b.w[0]), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma(f32x4 c, const Frag<float>& a, const Frag<float>& b) {
  const float* pa = reinterpret_cast<const float*>(a.w);
  const float* pb = reinterpret_cast<const float*>(b.w);
#pragma unroll
  for (int s = 0; s < 8; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[s], pb[s], c, 0, 0, 0);
  return c;
}

// Element conversions (round to nearest even, as torch's .to(dtype)).
template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ f16 from_f32<f16>(float x) { return (f16)x; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }

template <typename T>
__device__ __forceinline__ float to_f32(T x) { return (float)x; }

// Packs eight fp32 values into a fragment of T.
template <typename T>
__device__ __forceinline__ Frag<T> pack8(const float (&v)[8]) {
  Frag<T> f;
  T* e = reinterpret_cast<T*>(f.w);
#pragma unroll
  for (int s = 0; s < 8; ++s) e[s] = from_f32<T>(v[s]);
  return f;
}

// ---------------------------------------------------------------------------
// LDS operand reads.
// ---------------------------------------------------------------------------
// Eight consecutive elements of a row-major tile (16-byte aligned).
template <typename T>
__device__ __forceinline__ Frag<T> lds_frag_row(const T* p) {
  Frag<T> f;
#pragma unroll
  for (int i = 0; i < Frag<T>::kWords; ++i) f.w[i] = reinterpret_cast<const uint4*>(p)[i];
  return f;
}

// Two runs of four consecutive elements (kappa of a C-built fragment).
template <typename T>
__device__ __forceinline__ Frag<T> lds_frag_2x4(const T* p0, const T* p1) {
  Frag<T> f;
  if constexpr (sizeof(T) == 2) {
    uint2 a = *reinterpret_cast<const uint2*>(p0);
    uint2 b = *reinterpret_cast<const uint2*>(p1);
    f.w[0] = make_uint4(a.x, a.y, b.x, b.y);
  } else {
    f.w[0] = *reinterpret_cast<const uint4*>(p0);
    f.w[1] = *reinterpret_cast<const uint4*>(p1);
  }
  return f;
}

// ---------------------------------------------------------------------------
// Cooperative staging of ROWS x D tiles from HBM into LDS.
// Each thread owns RPT consecutive rows of one 8-element column group; the
// global reads are 16-byte vectors, consecutive threads read consecutive
// 16-byte pieces of a row. Rows outside [row_lo, row_hi) read as zero.
// ---------------------------------------------------------------------------
template <typename T, int D, int ROWS, int NT>
struct TileStage {
  static constexpr int kColGroups = D / 8;
  static constexpr int kRowGroups = (NT / kColGroups) < ROWS ? NT / kColGroups : ROWS;
  static constexpr int kRPT = ROWS / kRowGroups;  // rows per thread
  static_assert(kRPT >= 1 && kRowGroups * kRPT == ROWS, "tile/thread mismatch");
  static constexpr int kWords = Frag<T>::kWords;
  uint4 r[kRPT][kWords];

  // Threads beyond kRowGroups * kColGroups hold no rows.
  __device__ __forceinline__ static bool owner(int tid) { return tid < kRowGroups * kColGroups; }

  __device__ __forceinline__ void load(const T* base, int64_t row_stride, int row0, int row_lo,
                                       int row_hi, int tid) {
    const int cg = tid % kColGroups;
    const int rg = tid / kColGroups;
#pragma unroll
    for (int i = 0; i < kRPT; ++i) {
      const int row = row0 + rg * kRPT + i;
      if (owner(tid) && row >= row_lo && row < row_hi) {
        const uint4* src = reinterpret_cast<const uint4*>(base + (int64_t)row * row_stride + cg * 8);
#pragma unroll
        for (int w = 0; w < kWords; ++w) r[i][w] = src[w];
      } else {
#pragma unroll
        for (int w = 0; w < kWords; ++w) r[i][w] = make_uint4(0, 0, 0, 0);
      }
    }
  }

  // Row-major copy: tile[row][d], row stride LD elements.
  template <int LD>
  __device__ __forceinline__ void store_rows(T* tile, int tid) const {
    if (!owner(tid)) return;
    const int cg = tid % kColGroups;
    const int rg = tid / kColGroups;
#pragma unroll
    for (int i = 0; i < kRPT; ++i) {
      uint4* dst = reinterpret_cast<uint4*>(tile + (rg * kRPT + i) * LD + cg * 8);
#pragma unroll
      for (int w = 0; w < kWords; ++w) dst[w] = r[i][w];
    }
  }

  // Transposed copy: tile_t[d][row], row stride LDT elements.
  template <int LDT>
  __device__ __forceinline__ void store_cols(T* tile_t, int tid) const {
    if (!owner(tid)) return;
    const int cg = tid % kColGroups;
    const int rg = tid / kColGroups;
    const T* e = reinterpret_cast<const T*>(r);  // e[i*8 + j]: row i, column j
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      T* dst = tile_t + (cg * 8 + j) * LDT + rg * kRPT;
#pragma unroll
      for (int i = 0; i < kRPT; ++i) dst[i] = e[i * 8 + j];
    }
  }
};

// ---------------------------------------------------------------------------
// sqrt(N) geometry (reference core.py:957, 1038-1061, 1112-1117).
// ---------------------------------------------------------------------------
// Length of the global-row prefix query i attends to. With relay each W-block
// contributes rpb = 1 + top_k rows (strided row first); without, rpb = 1.
__device__ __forceinline__ int glob_prefix(int i, int W, int rpb) {
  const int a = max(i - W + 1, 0);
  const int f = a / W;
  return rpb * f + ((a - f * W) != 0 ? 1 : 0);
}

// Cross-lane helpers on the 4 lane groups of a wave (lanes l, l^16, l^32, l^48).
__device__ __forceinline__ float group_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}
__device__ __forceinline__ float group_sum(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

}  // namespace cra

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

// Packs eight fp32 values into a fragment of T (pairwise conversions, round
// to nearest even).
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef bf16 bf16x2 __attribute__((ext_vector_type(2)));
template <typename T>
__device__ __forceinline__ Frag<T> pack8(const float (&v)[8]) {
  Frag<T> f;
  if constexpr (sizeof(T) == 2) {
    typedef T t2 __attribute__((ext_vector_type(2)));
    uint32_t* w = reinterpret_cast<uint32_t*>(f.w);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      w[s] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{v[2 * s], v[2 * s + 1]}, t2));
  } else {
    T* e = reinterpret_cast<T*>(f.w);
#pragma unroll
    for (int s = 0; s < 8; ++s) e[s] = from_f32<T>(v[s]);
  }
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

// ---------------------------------------------------------------------------
// gfx950 LDS tiles for 2-byte elements: ROWS x D, row-major, no padding,
// 16-byte chunks XOR-swizzled per row so that 16 lanes reading the same
// chunk of 16 consecutive rows hit 16 different bank groups.
//
// Filled straight from HBM with global_load_lds (16 B per lane; lane i of an
// instruction lands at LDS base + 16 i, so each lane fetches the global chunk
// that belongs at its LDS position). Read either as 16-byte row fragments or
// transposed with ds_read_b64_tr_b16: in each 16-lane group, result lane L,
// slot j receives element L%4 of what source lane 4j + L/4 addressed, so if
// source lane 4j+m addresses row r_j, columns c0+4m .. c0+4m+3, result lane L
// holds column c0+L of rows r_0..r_3 -- a transposed MFMA operand.
// ---------------------------------------------------------------------------
typedef short i16x4 __attribute__((ext_vector_type(4)));
#define CRA_LDS(p) ((__attribute__((address_space(3))) void*)(p))

template <int D, int ROWS>
struct SwzTile {
  static_assert(D == 32 || D == 64 || D == 128, "head dim");
  static constexpr int kCPR = D / 8;      // 16-byte chunks per row
  static constexpr int kRPL = 128 / D;    // rows sharing one 256-byte line
  static constexpr int kBytes = ROWS * D * 2;
  static constexpr int kInstr = ROWS * kCPR / 64;  // 1 KB global_load_lds per instruction

  __device__ __forceinline__ static int swz(int row) { return (row / kRPL) % kCPR; }
  // byte offset of logical 16-byte chunk `chunk` of `row`
  __device__ __forceinline__ static int off(int row, int chunk) {
    return row * (D * 2) + ((chunk ^ swz(row)) << 4);
  }

  // Cooperative fill by NWAVES waves: instruction t = t0 * NWAVES + wave
  // moves tile rows [4t, 4t + 4) (D = 128; 64 / kCPR rows in general), so a
  // wave's successive instructions are kRowStep rows apart. kRowStep is a
  // multiple of the swizzle period, so a lane's in-row chunk is the same for
  // all of its instructions and its offset is one precomputed VGPR plus a
  // wave-uniform row offset.
  template <int NWAVES>
  struct Fill {
    static constexpr int kPer = (kInstr + NWAVES - 1) / NWAVES;
    static constexpr int kRowsPerInstr = 64 / kCPR;
    static constexpr int kRowStep = NWAVES * kRowsPerInstr;
    static_assert(kPer == 1 || (kRowStep % kRPL == 0 && (kRowStep / kRPL) % kCPR == 0),
                  "swizzle must repeat every instruction step");

    // Lane's byte offset for its first instruction, relative to tile row 0 of
    // a source whose rows are row_bytes apart.
    __device__ __forceinline__ static int lane_off(int wave, int lane, int row_bytes) {
      const int row = wave * kRowsPerInstr + lane / kCPR;
      return row * row_bytes + (((lane % kCPR) ^ swz(row)) << 4);
    }

    // Tile row i <- source row row0 + i. The buffer resource's record count
    // bounds the rows that may be read: lanes past it load zeros.
    __device__ __forceinline__ static void load(char* lds, __amdgpu_buffer_rsrc_t rsrc,
                                                int lane_off, int row_bytes, int row0,
                                                int wave) {
      // The LDS destination goes to M0: make the wave index visibly uniform,
      // and keep its range visible, or the compiler cannot tell this fill
      // from reads of the other buffer and waits for it before them.
      static_assert((NWAVES & (NWAVES - 1)) == 0, "power-of-two wave count");
      const int w = __builtin_amdgcn_readfirstlane(wave) & (NWAVES - 1);
#pragma unroll
      for (int t0 = 0; t0 < kPer; ++t0) {
        const int t = t0 * NWAVES + w;
        if (kInstr % NWAVES != 0 && t >= kInstr) break;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, CRA_LDS(lds + t * 1024), 16,
                                                 lane_off + (row0 + t0 * kRowStep) * row_bytes,
                                                 0, 0, 0);
      }
    }
  };

  // 8 consecutive elements (16 B) of `row` starting at column 8*chunk.
  template <typename T>
  __device__ __forceinline__ static Frag<T> row_frag(const char* lds, int row, int chunk) {
    Frag<T> f;
    f.w[0] = *reinterpret_cast<const uint4*>(lds + off(row, chunk));
    return f;
  }

  // The swizzle repeats every 16 rows (16 / kRPL is a multiple of kCPR), so
  // for rows 16*blk + r the offset is blk * 16 * row_bytes + lane_off(r, ..):
  // lane-constant parts are computed once and the block term folds into the
  // instruction's immediate offset.
  static constexpr int kBlk16 = 16 * D * 2;
  // row fragment of row 16*blk + (lane%16), chunk `chunk`
  __device__ __forceinline__ static int row_lane_off(int lane, int chunk) {
    return off(lane & 15, chunk);
  }
  // transposed fragment at column c0: rows 16*blk + 4g + j, this lane's part
  __device__ __forceinline__ static int tr_lane_off(int lane, int c0) {
    const int L = lane & 15, g = lane >> 4;
    const int col = c0 + 4 * (L & 3);
    return off(4 * g + (L >> 2), col >> 3) + ((col & 7) << 1);
  }
  template <typename T>
  __device__ __forceinline__ static Frag<T> row_frag_at(const char* p) {
    Frag<T> f;
    f.w[0] = *reinterpret_cast<const uint4*>(p);
    return f;
  }
  // pa: rows 16*blk_a + ..; pb: rows 16*blk_b + .. (both already offset)
  template <typename T>
  __device__ __forceinline__ static Frag<T> tr_frag_at(const char* pa, const char* pb) {
    i16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)pa);
    i16x4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)pb);
    Frag<T> f;
    const uint2 ux = __builtin_bit_cast(uint2, x);
    const uint2 uy = __builtin_bit_cast(uint2, y);
    f.w[0] = make_uint4(ux.x, ux.y, uy.x, uy.y);
    return f;
  }

  // Transposed operand: lane (L = lane%16, g = lane/16) gets column c0 + L of
  // rows ra + 4g + j (slots 0..3) and rb + 4g + j (slots 4..7).
  template <typename T>
  __device__ __forceinline__ static Frag<T> tr_frag(const char* lds, int ra, int rb, int c0,
                                                    int lane) {
    const int L = lane & 15, g = lane >> 4;
    const int j = L >> 2, m = L & 3;
    const int col = c0 + 4 * m;
    const int ca = ra + 4 * g + j, cb = rb + 4 * g + j;
    const int oa = off(ca, col >> 3) + ((col & 7) << 1);
    const int ob = off(cb, col >> 3) + ((col & 7) << 1);
    i16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4*)(lds + oa));
    i16x4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4*)(lds + ob));
    Frag<T> f;
    const uint2 ux = __builtin_bit_cast(uint2, x);
    const uint2 uy = __builtin_bit_cast(uint2, y);
    f.w[0] = make_uint4(ux.x, ux.y, uy.x, uy.y);
    return f;
  }
};

// Wait until this wave's outstanding global loads (incl. loads to LDS) landed.
// Mask of one tile for one query block: key row `ts + ko` is visible to the
// lane's query iff (unsigned)(hi - ko) <= span. Local window: hi = qi - ts,
// span = W - 1 (qi - W + 1 <= ts + ko <= qi); global prefix: hi = glen - 1 - ts,
// span = 2^31 - 1 (ts + ko < glen).
template <int NQB = 2>  // query blocks of the wave
struct TileMask {
  int hi[NQB];
  unsigned span[NQB];
  __device__ __forceinline__ bool ok(int ko, int qb) const {
    return (unsigned)(hi[qb] - ko) <= span[qb];
  }
};

__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0); }

// Raw buffer resource over `bytes` bytes at `base` (gfx9 descriptor word 3).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

}  // namespace cra

// Packed global rows: per W-block, its strided row and its top_k relay rows.
//
// Follows the reference relay pre-computation `_relay_precompute_topk`
// (core.py:2630-2748): per block, rank the valid rows by fp32 ||k||^2,
// descending, the earlier row winning ties (strict '>' insertion,
// core.py:2688-2703); a slot with no valid row left points at the block's
// first row (core.py:2668-2669). Unlike the reference, which walks the W rows
// of a block one at a time in a single program, one 256-thread workgroup scans
// a block with D/8 lanes per row; every row group keeps its own sorted top-4
// and one wave merges the lists with the same (norm desc, row asc) order (a
// wave-wide maximum per pick), which yields the same selection as the
// sequential scan.
//
// The squared norm of a row is summed in one fixed order so a CPU check can
// reproduce it bit for bit: each lane sums the squares of its 8 consecutive
// elements left to right (no fused multiply-add), then the D/8 lane partials
// are combined by a butterfly p += p[lane ^ off], off = D/16 .. 1.
#include "cra_common.hpp"
#include "cra_internal.hpp"

namespace cra {

namespace {

constexpr float kSentinel = -1e38f;  // below any squared norm

// 64-bit rank of a candidate: larger key = larger norm, then smaller row.
// The float's bits are mapped to an unsigned order-preserving form (sign bit
// set for x >= 0, all bits flipped for x < 0); every key is above 0.
__device__ __forceinline__ uint64_t rank_key(float norm, int row) {
  const uint32_t b = __float_as_uint(norm);
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(~(uint32_t)row);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t x, int off) {
  const uint32_t lo = __shfl_xor((uint32_t)x, off), hi = __shfl_xor((uint32_t)(x >> 32), off);
  return ((uint64_t)hi << 32) | lo;
}

template <typename T, int D>
__global__ __launch_bounds__(256) void build_global_kernel(GlobalArgs a) {
  constexpr int kLPR = D / 8;        // lanes per row
  constexpr int kNRG = 256 / kLPR;   // row groups per workgroup
  constexpr int kW16 = Frag<T>::kWords;
  const Doc dc = find_doc(a.docs, blockIdx.x);
  const int r = dc.item;  // block of the document
  const int W = dc.W, rpb = dc.rpb;
  const bool relay = rpb > 1;
  const int bh = blockIdx.y;
  const int b = bh / a.Hkv, h = bh % a.Hkv;
  const T* kb = static_cast<const T*>(a.k) + b * a.ksb + h * a.ksh + (int64_t)dc.off * a.kss;
  const T* vb = static_cast<const T*>(a.v) + b * a.vsb + h * a.vsh + (int64_t)dc.off * a.vss;
  const int tid = threadIdx.x;
  const int row0 = r * W;  // rows of the document

  __shared__ float s_norm[kNRG * 4];
  __shared__ int s_idx[kNRG * 4];
  __shared__ int s_sel[4];

  if (relay) {
    const int li = tid % kLPR;
    const int rg = tid / kLPR;
    const int nrows = min(W, dc.len - row0);
    float bn[4] = {kSentinel, kSentinel, kSentinel, kSentinel};
    int bi[4] = {0, 0, 0, 0};
    // kU row groups per pass: their loads are issued together (rows past the
    // block are clamped to its last row and left out of the ranking), then
    // the norms are ranked in row order
    constexpr int kU = 8;
    for (int base = 0; base < nrows; base += kU * kNRG) {  // uniform trip count
      uint4 w[kU][kW16];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int rr = min(base + u * kNRG + rg, nrows - 1);
        const uint4* p = reinterpret_cast<const uint4*>(kb + (int64_t)(row0 + rr) * a.kss + li * 8);
#pragma unroll
        for (int i = 0; i < kW16; ++i) w[u][i] = p[i];
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int rr = base + u * kNRG + rg;
        const bool valid = rr < nrows;
        const T* e = reinterpret_cast<const T*>(w[u]);
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float x = to_f32(e[i]);
          acc = __fadd_rn(acc, __fmul_rn(x, x));
        }
#pragma unroll
        for (int off = kLPR / 2; off >= 1; off >>= 1) acc = __fadd_rn(acc, __shfl_xor(acc, off));
        if (valid) {
          // strict '>' cascade, rows arrive in increasing order within a group
          const bool b0 = acc > bn[0], b1 = acc > bn[1], b2 = acc > bn[2], b3 = acc > bn[3];
          const float n3 = b2 ? bn[2] : (b3 ? acc : bn[3]);
          const int i3 = b2 ? bi[2] : (b3 ? rr : bi[3]);
          const float n2 = b1 ? bn[1] : (b2 ? acc : bn[2]);
          const int i2 = b1 ? bi[1] : (b2 ? rr : bi[2]);
          const float n1 = b0 ? bn[0] : (b1 ? acc : bn[1]);
          const int i1 = b0 ? bi[0] : (b1 ? rr : bi[1]);
          bn[0] = b0 ? acc : bn[0];
          bi[0] = b0 ? rr : bi[0];
          bn[1] = n1; bi[1] = i1;
          bn[2] = n2; bi[2] = i2;
          bn[3] = n3; bi[3] = i3;
        }
      }
    }
    if (li == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s_norm[rg * 4 + j] = bn[j];
        s_idx[rg * 4 + j] = bi[j];
      }
    }
    __syncthreads();
    if (tid < 64) {
      // Wave 0 merges the row groups' lists: each candidate becomes a 64-bit
      // key ordered as (norm desc, row asc) -- the float's order-preserving
      // bits above the complemented row -- and every pick is a wave-wide
      // maximum. A picked candidate's key becomes 0, below every candidate
      // (the sentinel of an unset slot included); of equal keys (unset slots
      // of one group list) only one is taken per pick.
      constexpr int kNC = kNRG * 4, kPer = (kNC + 63) / 64;
      uint64_t key[kPer];
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        const int c = tid + 64 * q;
        key[q] = c < kNC ? rank_key(s_norm[c], s_idx[c]) : 0ull;
      }
      int mine = 0;  // lane j keeps pick j
      for (int j = 0; j < a.top_k; ++j) {
        uint64_t m = key[0];
#pragma unroll
        for (int q = 1; q < kPer; ++q) m = key[q] > m ? key[q] : m;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
          const uint64_t o = shfl_xor_u64(m, off);
          m = o > m ? o : m;
        }
        // the lowest lane holding the maximum takes one copy of it
        int hit = -1;
#pragma unroll
        for (int q = kPer - 1; q >= 0; --q) hit = key[q] == m ? q : hit;
        const uint64_t holders = __ballot(hit >= 0);
        if (tid == __builtin_ctzll(holders)) key[hit] = 0ull;
        if (tid == j) mine = row0 + (int)~(uint32_t)m;
      }
      if (tid < a.top_k) {
        s_sel[tid] = mine;
        a.src[((int64_t)bh * a.NB + dc.bofs + r) * a.top_k + tid] = mine;
      }
    }
    __syncthreads();
  }

  // Emit rows: slot 0 = strided row r*W, slots 1..top_k = relay rows.
  T* gk = static_cast<T*>(a.gk) + ((int64_t)bh * a.G + dc.gofs + (int64_t)r * rpb) * D;
  T* gv = static_cast<T*>(a.gv) + ((int64_t)bh * a.G + dc.gofs + (int64_t)r * rpb) * D;
  const int cg = tid % (D / 8);
  const float sc = (relay && a.scale) ? a.scale[h] : 1.f;
  for (int slot = tid / (D / 8); slot < rpb; slot += 256 / (D / 8)) {
    const int row = slot == 0 ? row0 : s_sel[slot - 1];
    const uint4* pk = reinterpret_cast<const uint4*>(kb + (int64_t)row * a.kss + cg * 8);
    const uint4* pv = reinterpret_cast<const uint4*>(vb + (int64_t)row * a.vss + cg * 8);
    uint4 wk[kW16], wv[kW16];
#pragma unroll
    for (int i = 0; i < kW16; ++i) {
      wk[i] = pk[i];
      wv[i] = pv[i];
    }
    if (slot > 0 && a.scale) {
      T* ek = reinterpret_cast<T*>(wk);
      T* ev = reinterpret_cast<T*>(wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ek[i] = from_f32<T>(to_f32(ek[i]) * sc);
        ev[i] = from_f32<T>(to_f32(ev[i]) * sc);
      }
    }
    uint4* dk = reinterpret_cast<uint4*>(gk + (int64_t)slot * D + cg * 8);
    uint4* dv = reinterpret_cast<uint4*>(gv + (int64_t)slot * D + cg * 8);
#pragma unroll
    for (int i = 0; i < kW16; ++i) {
      dk[i] = wk[i];
      dv[i] = wv[i];
    }
  }
}

template <typename T>
hipError_t launch_T(int D, const GlobalArgs& args, int B, hipStream_t st) {
  GlobalArgs a = args;  // work items: the W-blocks of each document
  set_items(a.docs, [&](int d) { return (a.docs.len[d] + a.docs.W[d] - 1) / a.docs.W[d]; });
  dim3 grid(a.docs.item0[a.docs.n], B * a.Hkv);
  switch (D) {
    case 32: hipLaunchKernelGGL((build_global_kernel<T, 32>), grid, dim3(256), 0, st, a); break;
    case 64: hipLaunchKernelGGL((build_global_kernel<T, 64>), grid, dim3(256), 0, st, a); break;
    case 128: hipLaunchKernelGGL((build_global_kernel<T, 128>), grid, dim3(256), 0, st, a); break;
    case 256: hipLaunchKernelGGL((build_global_kernel<T, 256>), grid, dim3(256), 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_build_global(int dtype, int D, const GlobalArgs& a, int B, hipStream_t st) {
  switch (dtype) {
    case 0: return launch_T<f16>(D, a, B, st);
    case 1: return launch_T<bf16>(D, a, B, st);
    case 2: return launch_T<float>(D, a, B, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace cra

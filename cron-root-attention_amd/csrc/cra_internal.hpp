// Kernel argument blocks and launcher declarations shared by the kernel
// translation units and the C-ABI front end (cra_api.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cra {

// Documents of one launch: sequences packed along S (varlen), or the single
// sequence of a plain call. Each document has its own window, relay switch
// and packed global rows; nothing is attended across documents. A kernel's
// work items are numbered document by document: item0[d] is the first item
// of document d and item0[n] the total.
constexpr int kMaxDocs = 64;
struct Docs {
  int n;
  int off[kMaxDocs];   // first row along S
  int len[kMaxDocs];   // rows
  int W[kMaxDocs];     // window = block size
  int rpb[kMaxDocs];   // packed global rows per block: 1 + top_k with relay, else 1
  int gofs[kMaxDocs];  // first packed global row
  int bofs[kMaxDocs];  // first block (relay_src rows)
  int item0[kMaxDocs + 1];
};

// One document, resolved for a work item.
struct Doc {
  int off, len, W, rpb, gofs, bofs;
  int item;  // work item index within the document
};

__device__ __forceinline__ Doc find_doc(const Docs& t, int item) {
  int d = 0;
  for (int i = 1; i < t.n; ++i) d += item >= t.item0[i];  // item0 is non-decreasing
  return Doc{t.off[d], t.len[d], t.W[d], t.rpb[d], t.gofs[d], t.bofs[d], item - t.item0[d]};
}

// XCD-aware work order for launches of nbh heads x nt tiles (one document)
// when nbh is not a multiple of 8. The dispatcher sends block i to XCD i % 8;
// the plain order (item = rank * nbh + head, rank 0 the heaviest tile) then
// spreads a head's neighbouring tiles over several XCDs, whose L2s do not
// share the K/V (or Q/dO) rows those tiles overlap on. Here a head's tiles
// pair up as units {rank p, rank nt - 1 - p} (a heavy and a light tile: every
// unit costs about the same), units are numbered head by head (u = head * P +
// p), and XCD x takes a contiguous eighth of them, so it holds about nbh / 8
// heads with an equal share of the work. Its blocks take its tiles in the
// plain order's sequence (by rank, then head): heaviest first, as there.
// xcd_item returns the plain order's item index, or -1 for a padding block.
struct XcdChunk {
  int P, Pl;    // units per head; units with a light tile (the middle tile of
                // an odd nt is its unit's only tile)
  int q0, r0;   // first unit of this XCD: head q0, p = r0
  int q1, r1;   // one past its last unit
};

__host__ __device__ inline XcdChunk xcd_chunk(int x, int nbh, int nt) {
  const int P = (nt + 1) >> 1, U = nbh * P;
  const int base = U >> 3, extra = U & 7;
  const int u0 = x * base + (x < extra ? x : extra);
  const int u1 = u0 + base + (x < extra ? 1 : 0);
  return XcdChunk{P, nt >> 1, u0 / P, u0 % P, u1 / P, u1 % P};
}

// units of the chunk with p in [a, b)
__host__ __device__ inline int xcd_units(const XcdChunk& c, int a, int b) {
  if (a >= b) return 0;
  const int e1 = c.r1 < a ? a : c.r1 > b ? b : c.r1;
  const int e0 = c.r0 < a ? a : c.r0 > b ? b : c.r0;
  return (c.q1 - c.q0) * (b - a) + e1 - e0;
}

// tiles of the chunk with rank < r
__host__ __device__ inline int xcd_before(const XcdChunk& c, int nt, int r) {
  const int heavy = xcd_units(c, 0, r < c.P ? r : c.P);
  const int a = nt - r > 0 ? nt - r : 0;
  return heavy + xcd_units(c, a < c.Pl ? a : c.Pl, c.Pl);
}

__host__ __device__ inline int xcd_grid(int nbh, int nt) {
  int most = 0;
  for (int x = 0; x < 8; ++x) {
    const XcdChunk c = xcd_chunk(x, nbh, nt);
    const int n = xcd_before(c, nt, nt);
    most = n > most ? n : most;
  }
  return 8 * most;
}

__host__ __device__ inline int xcd_item(int block, int nbh, int nt) {
  const XcdChunk c = xcd_chunk(block & 7, nbh, nt);
  const int k = block >> 3;
  if (k >= xcd_before(c, nt, nt)) return -1;  // padding block
  // the rank r with xcd_before(r) <= k < xcd_before(r + 1)
  int lo = 0, hi = nt - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (xcd_before(c, nt, mid) <= k) lo = mid; else hi = mid - 1;
  }
  const int r = lo;
  const int p = r < c.P ? r : nt - 1 - r;
  // heads whose unit p lies in the chunk form a run from head q0 (q0 + 1
  // when unit (q0, p) precedes the chunk); take the j-th
  return r * nbh + c.q0 + (p < c.r0 ? 1 : 0) + (k - xcd_before(c, nt, r));
}

struct GlobalArgs {
  const void* k;
  const void* v;
  int64_t ksb, ksh, kss, vsb, vsh, vss;
  void* gk;
  void* gv;
  int32_t* src;        // [B, H_kv, NB, top_k], doc-relative rows
  const float* scale;
  int Hkv, top_k;
  int NB;              // blocks of all documents (rows of relay_src per head)
  int64_t G;           // packed global rows of all documents, per head
  Docs docs;           // items: W-blocks
};

struct FwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* gk;
  const void* gv;
  void* o;
  float* lse;
  int64_t qsb, qsh, qss, ksb, ksh, kss, vsb, vsh, vss, osb, osh, oss;
  int B, Hq, Hkv;
  int S;       // rows along S of all documents (row stride of lse)
  int64_t G;   // packed global rows of all documents, per head
  float scale;
  int phases;  // bit 0: local window, bit 1: global rows
  int* work_counter;  // persistent launch: zeroed item counter, else null
  int xcd_nt;  // > 0: XCD-aware order (xcd_item) over this many tiles per head
  Docs docs;   // items: query tiles (set by the launcher for its tile size)
};

struct BwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse;
  const void* gk;
  const void* gv;
  const int32_t* src;
  const float* rscale;
  void* dq;
  void* dk;
  void* dv;
  float* delta;    // [B, Hq, S] rowsum(o * do); 2-byte path: stored negated
  float* nlse2;    // [B, Hq, S] 2-byte path: -lse * log2(e)
  float* gpart;    // [nchunk, B, Hkv, G, 2, D] fp32 partial dK/dV of the global rows
  float* dalpha;   // [Hkv] or null
  int64_t qsb, qsh, qss, ksb, ksh, kss, vsb, vsh, vss, osb, osh, oss;
  int64_t dosb, dosh, doss, dqsb, dqsh, dqss, dksb, dksh, dkss, dvsb, dvsh, dvss;
  int B, Hq, Hkv, top_k;
  int S;           // rows along S of all documents (row stride of lse, delta)
  int NB;          // blocks of all documents (rows of relay_src per head)
  int64_t G;       // packed global rows of all documents, per head
  float scale;
  int nchunk;      // query chunks per document of the global-row kernel
  int group;       // 0: first launch of a call (fp32: computes Delta; writes dalpha);
                   // later document groups of the call add to dalpha
  int xcd_nt;      // > 0: XCD-aware order (xcd_item) over this many tiles per head
  Docs docs;       // items: set by the launcher per kernel
};

// Number the work items document by document: count(d) items for document d.
template <typename F>
inline void set_items(Docs& t, F count) {
  int s = 0;
  for (int d = 0; d < t.n; ++d) {
    t.item0[d] = s;
    s += count(d);
  }
  t.item0[t.n] = s;
}

// Queries per chunk of document length len split nchunk ways (multiple of 64).
__host__ __device__ inline int chunk_len_for(int len, int nchunk) {
  const int c = (len + nchunk - 1) / nchunk;
  return (c + 63) / 64 * 64;
}

// Compiled tile geometry (dtype 0 f16, 1 bf16, 2 f32; D 32/64/128): the forward's
// {waves, queries, key rows per tile} and the backward's {waves, rows, tile} of
// dQ, global-row dK/dV and local dK/dV. Returns false for an unbuilt (dtype, D).
bool fwd_tile_config(int dtype, int D, int out[3]);
bool bwd_tile_config(int dtype, int D, int out[9]);

// dtype: 0 f16, 1 bf16, 2 f32. Each returns hipError_t of the launch.
hipError_t launch_build_global(int dtype, int D, const GlobalArgs& a, int B, hipStream_t st);
hipError_t launch_fwd(int dtype, int D, const FwdArgs& a, hipStream_t st);
hipError_t launch_bwd(int dtype, int D, const BwdArgs& a, hipStream_t st);
// Workspace of the backward for n documents of lengths len[], windows W[]
// and packed rows per block rpb[] (G packed rows per head in total) on a
// device with `cus` compute units; *nchunk receives the query chunks per
// document of the global-row kernel.
size_t bwd_workspace_bytes(int D, int B, int Hq, int Hkv, int S, int n, const int* len,
                           const int* W, const int* rpb, int64_t G, int cus, int* nchunk);
// Workspace of the backward with nchunk query chunks: Delta and -lse*log2(e),
// [B*Hq*S] fp32 each (rounded up to 256 bytes), then the partials
// [nchunk, B, Hkv, G, 2, D] fp32.
size_t bwd_workspace_layout(int D, int B, int Hq, int Hkv, int S, int64_t G, int nchunk);

}  // namespace cra

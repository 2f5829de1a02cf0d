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

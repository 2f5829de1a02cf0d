// Kernel argument blocks and launcher declarations shared by the kernel
// translation units and the C-ABI front end (cra_api.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cra {

struct GlobalArgs {
  const void* k;
  const void* v;
  int64_t ksb, ksh, kss, vsb, vsh, vss;
  void* gk;
  void* gv;
  int32_t* src;
  const float* scale;
  int Hkv, S, W, NB, rpb, top_k, relay;
  int64_t G;
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
  int B, Hq, Hkv, S, W, rpb;
  int64_t G;
  float scale;
  int ntiles;
  int phases;  // bit 0: local window, bit 1: global rows
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
  float* delta;    // [B, Hq, S] rowsum(o * do)
  float* gpart;    // [nchunk, B, Hq, G, 2, D] fp32 partial dK/dV of the global rows
  float* dalpha;   // [Hkv] or null
  int64_t qsb, qsh, qss, ksb, ksh, kss, vsb, vsh, vss, osb, osh, oss;
  int64_t dosb, dosh, doss, dqsb, dqsh, dqss, dksb, dksh, dkss, dvsb, dvsh, dvss;
  int B, Hq, Hkv, S, W, rpb, top_k, relay;
  int64_t G;
  float scale;
  int nchunk;      // query chunks of the global-row kernel
  int chunk_len;   // queries per chunk
};

// dtype: 0 f16, 1 bf16, 2 f32. Each returns hipError_t of the launch.
hipError_t launch_build_global(int dtype, int D, const GlobalArgs& a, int B, hipStream_t st);
hipError_t launch_fwd(int dtype, int D, const FwdArgs& a, hipStream_t st);
hipError_t launch_bwd(int dtype, int D, const BwdArgs& a, hipStream_t st);
size_t bwd_workspace_bytes(int D, int B, int Hq, int Hkv, int S, int W, int64_t G, int* nchunk,
                           int* chunk_len);

}  // namespace cra

// C-ABI front end of libcra_hip.so: argument validation, planning of the
// launch geometry and error reporting. Declarations and the contract live in
// include/cra.h.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "../../include/cra.h"
#include "cra_common.hpp"
#include "cra_internal.hpp"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* where) {
  return fail(CRA_E_HIP, "%s: %s", where, hipGetErrorString(e));
}

// Compute units of the current device, looked up once per device. The
// backward's query-chunk rule sizes its work to the resident workgroup slots
// of the device it runs on. With no device to ask (a host without a GPU
// planning a workspace) the MI355X's 256 stands in: planning only, nothing
// is launched then.
constexpr int kMaxCuDevices = 64;
std::mutex g_cu_mu;
int g_cu_count[kMaxCuDevices] = {};

int device_cus() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxCuDevices) {
    (void)hipGetLastError();
    return 256;
  }
  std::lock_guard<std::mutex> lock(g_cu_mu);
  if (!g_cu_count[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus < 1) {
      (void)hipGetLastError();
      return 256;
    }
    g_cu_count[dev] = cus;
  }
  return g_cu_count[dev];
}

}  // namespace

namespace cra {
// Error text for the host-only translation units (the CPU-tensor path).
int set_error(int code, const char* msg) { return fail(code, "%s", msg); }
}  // namespace cra

namespace {

int elem_size(int dtype) { return dtype == CRA_F32 ? 4 : 2; }

// Fields every entry point needs; W and relay are checked by the plain
// entry points only (a varlen call gives them per document).
int check_problem_common(const cra_problem* p) {
  if (!p) return fail(CRA_E_INVALID, "problem is NULL");
  if (p->dtype != CRA_F16 && p->dtype != CRA_BF16 && p->dtype != CRA_F32)
    return fail(CRA_E_DTYPE, "unknown dtype code %d", p->dtype);
  if (p->B < 1 || p->H_q < 1 || p->H_kv < 1 || p->S < 1)
    return fail(CRA_E_INVALID, "B, H_q, H_kv, S must be >= 1 (got %d, %d, %d, %d)", p->B, p->H_q,
                p->H_kv, p->S);
  if (p->H_q % p->H_kv)
    return fail(CRA_E_INVALID, "H_q (%d) must be a multiple of H_kv (%d)", p->H_q, p->H_kv);
  if (!cra_supported_head_dim(p->D))
    return fail(CRA_E_UNSUPPORTED, "head dim %d not built (32, 64, 128, 256)", p->D);
  if (!(p->scale > 0.f)) return fail(CRA_E_INVALID, "scale must be > 0");
  // 32-bit row indices inside the kernels
  if ((int64_t)p->B * p->H_q * (int64_t)p->S > (int64_t)1 << 31)
    return fail(CRA_E_INVALID, "B*H*S exceeds 2^31");
  return CRA_OK;
}

int check_top_k(const cra_problem* p) {
  if (p->top_k < 1 || p->top_k > 4) return fail(CRA_E_INVALID, "top_k=%d outside [1, 4]", p->top_k);
  return CRA_OK;
}

int check_problem(const cra_problem* p) {
  if (int e = check_problem_common(p)) return e;
  if (p->W < 1 || p->W > p->S)
    return fail(CRA_E_INVALID, "window W=%d outside [1, S=%d]", p->W, p->S);
  if (p->relay != 0 && p->relay != 1) return fail(CRA_E_INVALID, "relay must be 0 or 1");
  if (p->relay)
    if (int e = check_top_k(p)) return e;
  return CRA_OK;
}

int check_tensor(const char* name, const cra_tensor& t, int esz) {
  if (!t.ptr) return fail(CRA_E_INVALID, "%s: NULL pointer", name);
  if (reinterpret_cast<uintptr_t>(t.ptr) % 16)
    return fail(CRA_E_LAYOUT, "%s: pointer not 16-byte aligned", name);
  const int64_t vec = 16 / esz;
  if (t.sb % vec || t.sh % vec || t.ss % vec)
    return fail(CRA_E_LAYOUT, "%s: strides (%lld, %lld, %lld) must be multiples of %lld elements",
                name, (long long)t.sb, (long long)t.sh, (long long)t.ss, (long long)vec);
  return CRA_OK;
}

// Kernels address one (b, h) slice with 32-bit byte offsets.
int check_span(const char* name, const cra_tensor& t, const cra_problem* p, int esz) {
  const int64_t span = ((int64_t)(p->S - 1) * t.ss + p->D) * esz;
  if (span >= ((int64_t)1 << 31))
    return fail(CRA_E_LAYOUT, "%s: one head spans %lld bytes (limit 2^31); pass a contiguous tensor",
                name, (long long)span);
  return CRA_OK;
}

int check_buf(const char* name, const void* p) {
  if (!p) return fail(CRA_E_INVALID, "%s: NULL pointer", name);
  if (reinterpret_cast<uintptr_t>(p) % 16)
    return fail(CRA_E_LAYOUT, "%s: pointer not 16-byte aligned", name);
  return CRA_OK;
}

int64_t num_blocks(const cra_problem* p) { return (p->S + p->W - 1) / p->W; }
int rows_per_block(const cra_problem* p) { return p->relay ? 1 + p->top_k : 1; }

// The documents of one call in layout order (a plain call is one document),
// their packed global rows (gofs) and W-blocks (bofs) per (b, kv head), and
// the order the kernels take them in: longest first, so that the heaviest
// work items start first and short documents fill the tail.
struct Plan {
  int n = 0;
  std::vector<int> off, len, W, rpb, gofs, bofs, order;
  int64_t G = 0;   // packed global rows per (b, kv head)
  int64_t NB = 0;  // W-blocks per (b, kv head)
  bool any_relay = false;
  int top_k = 0;   // relay rows per block of the documents with relay
};

void plan_add(Plan& pl, int off, int len, int W, bool relay, int top_k) {
  const int nb = (len + W - 1) / W;
  const int rpb = relay ? 1 + top_k : 1;
  pl.off.push_back(off);
  pl.len.push_back(len);
  pl.W.push_back(W);
  pl.rpb.push_back(rpb);
  pl.gofs.push_back((int)pl.G);
  pl.bofs.push_back((int)pl.NB);
  pl.G += (int64_t)nb * rpb;
  pl.NB += nb;
  pl.any_relay = pl.any_relay || relay;
  ++pl.n;
}

void plan_order(Plan& pl) {
  pl.order.resize(pl.n);
  for (int d = 0; d < pl.n; ++d) pl.order[d] = d;
  std::stable_sort(pl.order.begin(), pl.order.end(),
                   [&](int x, int y) { return pl.len[x] > pl.len[y]; });
}

int plan_plain(const cra_problem* p, Plan* pl) {
  if (int e = check_problem(p)) return e;
  *pl = Plan{};
  pl->top_k = p->relay ? p->top_k : 0;
  plan_add(*pl, 0, p->S, p->W, p->relay != 0, pl->top_k);
  plan_order(*pl);
  return CRA_OK;
}

int plan_varlen(const cra_problem* p, const cra_docs* d, Plan* pl) {
  if (int e = check_problem_common(p)) return e;
  if (!d) return fail(CRA_E_INVALID, "docs is NULL");
  if (d->n_docs < 1) return fail(CRA_E_INVALID, "n_docs=%d must be >= 1", d->n_docs);
  if (!d->cu_seqlens || !d->window || !d->relay)
    return fail(CRA_E_INVALID, "docs: cu_seqlens, window and relay must not be NULL");
  if (d->cu_seqlens[0] != 0 || d->cu_seqlens[d->n_docs] != p->S)
    return fail(CRA_E_INVALID, "cu_seqlens must run from 0 to S=%d (got %d .. %d)", p->S,
                d->cu_seqlens[0], d->cu_seqlens[d->n_docs]);
  bool relay = false;
  for (int i = 0; i < d->n_docs; ++i) {
    const int len = d->cu_seqlens[i + 1] - d->cu_seqlens[i];
    if (len < 1) return fail(CRA_E_INVALID, "cu_seqlens must rise strictly (document %d)", i);
    if (d->window[i] < 1 || d->window[i] > len)
      return fail(CRA_E_INVALID, "document %d: window %d outside [1, %d]", i, d->window[i], len);
    if (d->relay[i] != 0 && d->relay[i] != 1)
      return fail(CRA_E_INVALID, "document %d: relay must be 0 or 1", i);
    relay = relay || d->relay[i];
  }
  if (relay)
    if (int e = check_top_k(p)) return e;
  *pl = Plan{};
  pl->top_k = relay ? p->top_k : 0;
  for (int i = 0; i < d->n_docs; ++i)
    plan_add(*pl, d->cu_seqlens[i], d->cu_seqlens[i + 1] - d->cu_seqlens[i], d->window[i],
             d->relay[i] != 0, pl->top_k);
  if (pl->G * p->D >= ((int64_t)1 << 31))
    return fail(CRA_E_INVALID, "%lld packed global rows per head exceed the 32-bit offsets",
                (long long)pl->G);
  plan_order(*pl);
  return CRA_OK;
}

int num_groups(const Plan& pl) { return (pl.n + cra::kMaxDocs - 1) / cra::kMaxDocs; }

// Kernel-argument table of document group g (up to kMaxDocs documents, in
// launch order); the launchers number the work items.
cra::Docs group_table(const Plan& pl, int g) {
  cra::Docs t{};
  const int lo = g * cra::kMaxDocs;
  t.n = std::min(pl.n - lo, cra::kMaxDocs);
  for (int i = 0; i < t.n; ++i) {
    const int d = pl.order[lo + i];
    t.off[i] = pl.off[d];
    t.len[i] = pl.len[d];
    t.W[i] = pl.W[d];
    t.rpb[i] = pl.rpb[d];
    t.gofs[i] = pl.gofs[d];
    t.bofs[i] = pl.bofs[d];
  }
  return t;
}

size_t workspace_bytes(const cra_problem* p, const Plan& pl, int* nchunk) {
  return cra::bwd_workspace_bytes(p->D, p->B, p->H_q, p->H_kv, p->S, pl.n, pl.len.data(),
                                  pl.W.data(), pl.rpb.data(), pl.G, device_cus(), nchunk);
}

int build_global_impl(const cra_problem* p, const Plan& pl, cra_tensor k, cra_tensor v,
                      void* glob_k, void* glob_v, int32_t* relay_src, const float* relay_scale,
                      void* stream) {
  const int esz = elem_size(p->dtype);
  if (int e = check_tensor("k", k, esz)) return e;
  if (int e = check_tensor("v", v, esz)) return e;
  if (int e = check_buf("glob_k", glob_k)) return e;
  if (int e = check_buf("glob_v", glob_v)) return e;
  if (pl.any_relay && !relay_src) return fail(CRA_E_INVALID, "relay_src is NULL with relay on");
  if ((int64_t)p->B * p->H_kv > 65535) return fail(CRA_E_INVALID, "B*H_kv exceeds 65535");
  cra::GlobalArgs a{};
  a.k = k.ptr;
  a.v = v.ptr;
  a.ksb = k.sb; a.ksh = k.sh; a.kss = k.ss;
  a.vsb = v.sb; a.vsh = v.sh; a.vss = v.ss;
  a.gk = glob_k;
  a.gv = glob_v;
  a.src = relay_src;
  a.scale = relay_scale;
  a.Hkv = p->H_kv;
  a.top_k = pl.top_k;
  a.NB = (int)pl.NB;
  a.G = pl.G;
  for (int g = 0; g < num_groups(pl); ++g) {
    a.docs = group_table(pl, g);
    hipError_t e = cra::launch_build_global(p->dtype, p->D, a, p->B, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "cra_build_global launch");
  }
  return CRA_OK;
}

int fwd_impl(const cra_problem* p, const Plan& pl, cra_tensor q, cra_tensor k, cra_tensor v,
             const void* glob_k, const void* glob_v, cra_tensor o, float* lse,
             int32_t phase_mask, void* stream, int32_t* work_counter = nullptr) {
  if (phase_mask < 1 || phase_mask > (CRA_PHASE_LOCAL | CRA_PHASE_GLOBAL))
    return fail(CRA_E_INVALID, "phase_mask must be a non-empty subset of CRA_PHASE_LOCAL | CRA_PHASE_GLOBAL");
  const int esz = elem_size(p->dtype);
  if (int e = check_tensor("q", q, esz)) return e;
  if (int e = check_tensor("k", k, esz)) return e;
  if (int e = check_tensor("v", v, esz)) return e;
  if (int e = check_tensor("o", o, esz)) return e;
  if (int e = check_span("k", k, p, esz)) return e;
  if (int e = check_span("v", v, p, esz)) return e;
  if (int e = check_buf("glob_k", glob_k)) return e;
  if (int e = check_buf("glob_v", glob_v)) return e;
  if (int e = check_buf("lse", lse)) return e;
  cra::FwdArgs a{};
  a.q = q.ptr; a.k = k.ptr; a.v = v.ptr; a.gk = glob_k; a.gv = glob_v; a.o = o.ptr; a.lse = lse;
  a.qsb = q.sb; a.qsh = q.sh; a.qss = q.ss;
  a.ksb = k.sb; a.ksh = k.sh; a.kss = k.ss;
  a.vsb = v.sb; a.vsh = v.sh; a.vss = v.ss;
  a.osb = o.sb; a.osh = o.sh; a.oss = o.ss;
  a.B = p->B; a.Hq = p->H_q; a.Hkv = p->H_kv; a.S = p->S;
  a.G = pl.G;
  a.scale = p->scale;
  a.phases = phase_mask;
  a.work_counter = work_counter;
  for (int g = 0; g < num_groups(pl); ++g) {
    a.docs = group_table(pl, g);
    hipError_t e = cra::launch_fwd(p->dtype, p->D, a, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "cra_fwd launch");
  }
  return CRA_OK;
}

// nchunk_cap > 0 limits the query chunks of the global-row partials (the
// allocation-free entry point fits them into its fixed scratch); 0 keeps
// the planned count.
int bwd_impl(const cra_problem* p, const Plan& pl, cra_tensor q, cra_tensor k, cra_tensor v,
             cra_tensor o, cra_tensor dout, const float* lse, const void* glob_k,
             const void* glob_v, const int32_t* relay_src, const float* relay_scale,
             cra_tensor dq, cra_tensor dk, cra_tensor dv, float* dalpha, void* workspace,
             size_t workspace_bytes_given, void* stream, int nchunk_cap = 0) {
  const int esz = elem_size(p->dtype);
  if (int e = check_tensor("q", q, esz)) return e;
  if (int e = check_tensor("k", k, esz)) return e;
  if (int e = check_tensor("v", v, esz)) return e;
  if (int e = check_tensor("o", o, esz)) return e;
  if (int e = check_tensor("dout", dout, esz)) return e;
  if (int e = check_tensor("dq", dq, esz)) return e;
  if (int e = check_tensor("dk", dk, esz)) return e;
  if (int e = check_tensor("dv", dv, esz)) return e;
  // the backward reads these through buffer resources with 32-bit offsets
  if (int e = check_span("q", q, p, esz)) return e;
  if (int e = check_span("k", k, p, esz)) return e;
  if (int e = check_span("v", v, p, esz)) return e;
  if (int e = check_span("dout", dout, p, esz)) return e;
  if (int e = check_buf("lse", lse)) return e;
  if (int e = check_buf("glob_k", glob_k)) return e;
  if (int e = check_buf("glob_v", glob_v)) return e;
  if (pl.any_relay && !relay_src) return fail(CRA_E_INVALID, "relay_src is NULL with relay on");
  int nchunk = 0;
  size_t need = workspace_bytes(p, pl, &nchunk);
  if (nchunk_cap > 0 && nchunk > nchunk_cap) {
    nchunk = nchunk_cap;
    need = cra::bwd_workspace_layout(p->D, p->B, p->H_q, p->H_kv, p->S, pl.G, nchunk);
  }
  if (need > 0 && (!workspace || workspace_bytes_given < need))
    return fail(CRA_E_WORKSPACE, "workspace of %zu bytes needed, %zu given", need,
                workspace ? workspace_bytes_given : (size_t)0);
  if (workspace && reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(CRA_E_LAYOUT, "workspace not 256-byte aligned");
  cra::BwdArgs a{};
  a.q = q.ptr; a.k = k.ptr; a.v = v.ptr; a.o = o.ptr; a.dout = dout.ptr; a.lse = lse;
  a.gk = glob_k; a.gv = glob_v; a.src = relay_src; a.rscale = relay_scale;
  a.dq = dq.ptr; a.dk = dk.ptr; a.dv = dv.ptr;
  a.qsb = q.sb; a.qsh = q.sh; a.qss = q.ss;
  a.ksb = k.sb; a.ksh = k.sh; a.kss = k.ss;
  a.vsb = v.sb; a.vsh = v.sh; a.vss = v.ss;
  a.osb = o.sb; a.osh = o.sh; a.oss = o.ss;
  a.dosb = dout.sb; a.dosh = dout.sh; a.doss = dout.ss;
  a.dqsb = dq.sb; a.dqsh = dq.sh; a.dqss = dq.ss;
  a.dksb = dk.sb; a.dksh = dk.sh; a.dkss = dk.ss;
  a.dvsb = dv.sb; a.dvsh = dv.sh; a.dvss = dv.ss;
  a.B = p->B; a.Hq = p->H_q; a.Hkv = p->H_kv; a.S = p->S;
  a.top_k = pl.top_k;
  a.NB = (int)pl.NB;
  a.G = pl.G;
  a.scale = p->scale;
  a.nchunk = nchunk;
  // workspace carve-up: delta and nlse2 [B*Hq*S] fp32 each, then the
  // global-row partials
  char* ws = static_cast<char*>(workspace);
  const size_t delta_bytes = (((size_t)p->B * p->H_q * p->S * 4) + 255) / 256 * 256;
  a.delta = reinterpret_cast<float*>(ws);
  a.nlse2 = reinterpret_cast<float*>(ws + delta_bytes);
  a.gpart = reinterpret_cast<float*>(ws + 2 * delta_bytes);
  a.dalpha = dalpha;
  for (int g = 0; g < num_groups(pl); ++g) {
    a.group = g;
    a.docs = group_table(pl, g);
    hipError_t e = cra::launch_bwd(p->dtype, p->D, a, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "cra_bwd launch");
  }
  return CRA_OK;
}

// ---- allocation-free backward ----------------------------------------------
// The workspace of cra_bwd_noalloc: one file-scope array per device, held
// until the process ends. In host code `scratch` is only a handle; its
// device address (different on every device) comes from
// hipGetSymbolAddress, looked up once per device with that device current.
static __device__ __align__(256) char scratch[CRA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device, which must also be the
// stream's device (the kernels run on the stream's device).
int scratch_address(void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) return hip_fail(e, "hipStreamGetDevice");
    if (sdev != dev)
      return fail(CRA_E_INVALID,
                  "stream belongs to device %d but device %d is current; make the stream's "
                  "device current", (int)sdev, dev);
  }
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(CRA_E_UNSUPPORTED, "device %d: at most %d devices", dev, kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!ptr) return fail(CRA_E_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return CRA_OK;
}

}  // namespace

extern "C" {

int cra_supported_head_dim(int32_t D) { return D == 32 || D == 64 || D == 128 || D == 256; }

int32_t cra_abi_version(void) { return CRA_ABI_VERSION; }

int64_t cra_global_rows(const cra_problem* p) {
  if (check_problem(p)) return -1;
  return num_blocks(p) * rows_per_block(p);
}

int cra_build_global(const cra_problem* p, cra_tensor k, cra_tensor v, void* glob_k, void* glob_v,
                     int32_t* relay_src, const float* relay_scale, void* stream) {
  Plan pl;
  if (int e = plan_plain(p, &pl)) return e;
  return build_global_impl(p, pl, k, v, glob_k, glob_v, relay_src, relay_scale, stream);
}

int cra_fwd(const cra_problem* p, cra_tensor q, cra_tensor k, cra_tensor v, const void* glob_k,
            const void* glob_v, cra_tensor o, float* lse, void* stream) {
  return cra_fwd_phases(p, q, k, v, glob_k, glob_v, o, lse, CRA_PHASE_LOCAL | CRA_PHASE_GLOBAL,
                        stream);
}

int cra_fwd_phases(const cra_problem* p, cra_tensor q, cra_tensor k, cra_tensor v,
                   const void* glob_k, const void* glob_v, cra_tensor o, float* lse,
                   int32_t phase_mask, void* stream) {
  Plan pl;
  if (int e = plan_plain(p, &pl)) return e;
  return fwd_impl(p, pl, q, k, v, glob_k, glob_v, o, lse, phase_mask, stream);
}

int cra_fwd_persistent(const cra_problem* p, cra_tensor q, cra_tensor k, cra_tensor v,
                       const void* glob_k, const void* glob_v, cra_tensor o, float* lse,
                       int32_t* work_counter, void* stream) {
  Plan pl;
  if (int e = plan_plain(p, &pl)) return e;
  if (int e = check_buf("work_counter", work_counter)) return e;
  return fwd_impl(p, pl, q, k, v, glob_k, glob_v, o, lse, CRA_PHASE_LOCAL | CRA_PHASE_GLOBAL,
                  stream, work_counter);
}

size_t cra_bwd_workspace_bytes(const cra_problem* p) {
  Plan pl;
  if (plan_plain(p, &pl)) return 0;
  int nchunk = 0;
  return workspace_bytes(p, pl, &nchunk);
}

int cra_bwd(const cra_problem* p, cra_tensor q, cra_tensor k, cra_tensor v, cra_tensor o,
            cra_tensor dout, const float* lse, const void* glob_k, const void* glob_v,
            const int32_t* relay_src, const float* relay_scale, cra_tensor dq, cra_tensor dk,
            cra_tensor dv, float* dalpha, void* workspace, size_t workspace_bytes, void* stream) {
  Plan pl;
  if (int e = plan_plain(p, &pl)) return e;
  return bwd_impl(p, pl, q, k, v, o, dout, lse, glob_k, glob_v, relay_src, relay_scale, dq, dk,
                  dv, dalpha, workspace, workspace_bytes, stream);
}

int cra_bwd_noalloc(const cra_problem* p, cra_tensor q, cra_tensor k, cra_tensor v, cra_tensor o,
                    cra_tensor dout, const float* lse, const void* glob_k, const void* glob_v,
                    const int32_t* relay_src, const float* relay_scale, cra_tensor dq,
                    cra_tensor dk, cra_tensor dv, float* dalpha, void* stream) {
  Plan pl;
  if (int e = plan_plain(p, &pl)) return e;
  int nchunk = 0;
  const size_t planned = workspace_bytes(p, pl, &nchunk);
  int cap = 0;  // keep the planned chunks if they fit: then results equal cra_bwd's bit for bit
  if (planned > (size_t)CRA_NOALLOC_SCRATCH_BYTES) {
    const size_t one = cra::bwd_workspace_layout(p->D, p->B, p->H_q, p->H_kv, p->S, pl.G, 1);
    const size_t per_chunk = one - cra::bwd_workspace_layout(p->D, p->B, p->H_q, p->H_kv, p->S,
                                                             pl.G, 0);
    if (one > (size_t)CRA_NOALLOC_SCRATCH_BYTES)
      return fail(CRA_E_WORKSPACE,
                  "cra_bwd_noalloc: this problem needs %zu bytes of workspace even with one "
                  "query chunk; the fixed scratch holds %u bytes (use cra_bwd with a "
                  "caller-allocated workspace)", one, (unsigned)CRA_NOALLOC_SCRATCH_BYTES);
    cap = (int)(((size_t)CRA_NOALLOC_SCRATCH_BYTES - (one - per_chunk)) / per_chunk);
  }
  void* ws = nullptr;
  if (int e = scratch_address(stream, &ws)) return e;
  return bwd_impl(p, pl, q, k, v, o, dout, lse, glob_k, glob_v, relay_src, relay_scale, dq, dk,
                  dv, dalpha, ws, (size_t)CRA_NOALLOC_SCRATCH_BYTES, stream, cap);
}

int cra_varlen_sizes(const cra_problem* p, const cra_docs* docs, int64_t* global_rows,
                     int64_t* relay_src_len) {
  Plan pl;
  if (int e = plan_varlen(p, docs, &pl)) return e;
  if (global_rows) *global_rows = pl.G;
  if (relay_src_len) *relay_src_len = pl.NB * pl.top_k;
  return CRA_OK;
}

int cra_build_global_varlen(const cra_problem* p, const cra_docs* docs, cra_tensor k,
                            cra_tensor v, void* glob_k, void* glob_v, int32_t* relay_src,
                            const float* relay_scale, void* stream) {
  Plan pl;
  if (int e = plan_varlen(p, docs, &pl)) return e;
  return build_global_impl(p, pl, k, v, glob_k, glob_v, relay_src, relay_scale, stream);
}

int cra_fwd_varlen(const cra_problem* p, const cra_docs* docs, cra_tensor q, cra_tensor k,
                   cra_tensor v, const void* glob_k, const void* glob_v, cra_tensor o, float* lse,
                   void* stream) {
  Plan pl;
  if (int e = plan_varlen(p, docs, &pl)) return e;
  return fwd_impl(p, pl, q, k, v, glob_k, glob_v, o, lse, CRA_PHASE_LOCAL | CRA_PHASE_GLOBAL,
                  stream);
}

size_t cra_bwd_workspace_bytes_varlen(const cra_problem* p, const cra_docs* docs) {
  Plan pl;
  if (plan_varlen(p, docs, &pl)) return 0;
  int nchunk = 0;
  return workspace_bytes(p, pl, &nchunk);
}

int cra_bwd_varlen(const cra_problem* p, const cra_docs* docs, cra_tensor q, cra_tensor k,
                   cra_tensor v, cra_tensor o, cra_tensor dout, const float* lse,
                   const void* glob_k, const void* glob_v, const int32_t* relay_src,
                   const float* relay_scale, cra_tensor dq, cra_tensor dk, cra_tensor dv,
                   float* dalpha, void* workspace, size_t workspace_bytes, void* stream) {
  Plan pl;
  if (int e = plan_varlen(p, docs, &pl)) return e;
  return bwd_impl(p, pl, q, k, v, o, dout, lse, glob_k, glob_v, relay_src, relay_scale, dq, dk,
                  dv, dalpha, workspace, workspace_bytes, stream);
}

int cra_device_info(int32_t device, cra_device_info_t* out) {
  if (!out) return fail(CRA_E_INVALID, "out is NULL");
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  memset(out, 0, sizeof(*out));
  out->cu_count = prop.multiProcessorCount;
  out->lds_bytes_per_cu = (int32_t)prop.maxSharedMemoryPerMultiProcessor;
  out->arch_major = prop.major;
  out->arch_minor = prop.minor;
  snprintf(out->arch_name, sizeof(out->arch_name), "%s", prop.gcnArchName);
  snprintf(out->device_name, sizeof(out->device_name), "%s", prop.name);
  return CRA_OK;
}

int cra_tile_config(int32_t dtype, int32_t D, cra_tile_config_t* out) {
  if (!out) return fail(CRA_E_INVALID, "out is NULL");
  if (dtype != CRA_F16 && dtype != CRA_BF16 && dtype != CRA_F32)
    return fail(CRA_E_DTYPE, "unknown dtype code %d", dtype);
  int f[3], b[9];
  if (!cra::fwd_tile_config(dtype, D, f) || !cra::bwd_tile_config(dtype, D, b))
    return fail(CRA_E_UNSUPPORTED, "head dim %d not built (32, 64, 128, 256)", D);
  out->fwd_waves = f[0];
  out->fwd_queries = f[1];
  out->fwd_key_tile = f[2];
  out->dq_waves = b[0];
  out->dq_queries = b[1];
  out->dq_key_tile = b[2];
  out->dkdv_global_waves = b[3];
  out->dkdv_global_rows = b[4];
  out->dkdv_global_query_tile = b[5];
  out->dkdv_local_waves = b[6];
  out->dkdv_local_keys = b[7];
  out->dkdv_local_query_tile = b[8];
  return CRA_OK;
}

const char* cra_strerror(int32_t code) {
  switch (code) {
    case CRA_OK: return "ok";
    case CRA_E_INVALID: return "invalid argument";
    case CRA_E_LAYOUT: return "unsupported layout";
    case CRA_E_DTYPE: return "unknown dtype";
    case CRA_E_UNSUPPORTED: return "unsupported configuration";
    case CRA_E_HIP: return "HIP runtime error";
    case CRA_E_WORKSPACE: return "workspace too small";
  }
  return "unknown error";
}

const char* cra_last_error(void) { return g_err; }

}  // extern "C"

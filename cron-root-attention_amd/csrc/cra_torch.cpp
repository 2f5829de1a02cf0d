// Torch operator binding of libcra_hip.so (include/cra.h) with its autograd
// in C++: torch.ops.cra.attention(q, k, v, window, relay, top_k, scale).
//
// It serves the common call of cron_root_attention_v14 (reference
// core.py:3767-3797) -- GPU tensors, head dim 32/64/128/256, no
// relay_log_scale, the tiled forward -- with the
// same launches as the Python autograd Function (cra_build_global + cra_fwd,
// then cra_bwd) but without the Python autograd and ctypes layers, which at
// small S cost more host time than the kernels take on the GPU. Layouts the
// kernels cannot take are copied to contiguous ones here, as the Python path
// does. Everything else (padded head dims, relay scale, the persistent kernel,
// varlen, CPU tensors) stays on the Python path; both reach the same C ABI.
//
// The library is bound at run time (cra::bind(path)) so that the op uses the
// very library the Python binding loaded.
#include <dlfcn.h>

#include <atomic>
#include <mutex>
#include <string>

#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <torch/autograd.h>
#include <torch/library.h>

#include "cra.h"

namespace {

struct Api {
  decltype(&cra_global_rows) global_rows = nullptr;
  decltype(&cra_build_global) build_global = nullptr;
  decltype(&cra_fwd) fwd = nullptr;
  decltype(&cra_bwd_workspace_bytes) ws_bytes = nullptr;
  decltype(&cra_bwd) bwd = nullptr;
  decltype(&cra_strerror) strerror_ = nullptr;
  decltype(&cra_last_error) last_error = nullptr;
  decltype(&cra_abi_version) abi_version = nullptr;
};

// Written once under g_mu by bind(); g_bound is published last (release) and
// read with acquire, so a reader that sees it set sees the whole table.
std::mutex g_mu;
Api g_api;
std::atomic<bool> g_bound{false};

template <typename F>
void resolve(void* h, const std::string& path, const char* name, F& out) {
  void* f = dlsym(h, name);
  TORCH_CHECK(f != nullptr, path, " does not export ", name);
  out = reinterpret_cast<F>(f);
}

void bind(std::string path) {
  std::lock_guard<std::mutex> lk(g_mu);
  void* h = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
  TORCH_CHECK(h != nullptr, "cannot load ", path, ": ", dlerror());
  Api api;
  resolve(h, path, "cra_global_rows", api.global_rows);
  resolve(h, path, "cra_build_global", api.build_global);
  resolve(h, path, "cra_fwd", api.fwd);
  resolve(h, path, "cra_bwd_workspace_bytes", api.ws_bytes);
  resolve(h, path, "cra_bwd", api.bwd);
  resolve(h, path, "cra_strerror", api.strerror_);
  resolve(h, path, "cra_last_error", api.last_error);
  resolve(h, path, "cra_abi_version", api.abi_version);
  TORCH_CHECK(api.abi_version() == CRA_ABI_VERSION, path, ": ABI ", api.abi_version(),
              " != ", CRA_ABI_VERSION);
  if (g_bound.load(std::memory_order_acquire)) {
    // already bound (a second bind is a no-op unless it names another library)
    TORCH_CHECK(api.fwd == g_api.fwd, "cra::bind: already bound to another library");
    return;
  }
  g_api = api;
  g_bound.store(true, std::memory_order_release);
}

const Api& api() {
  TORCH_CHECK(g_bound.load(std::memory_order_acquire),
              "cra::attention: library not bound (call torch.ops.cra.bind first)");
  return g_api;
}

void check(int code, const char* func) {
  if (code == CRA_OK) return;
  const char* msg = api().last_error();
  TORCH_CHECK(false, func, ": ", (msg && *msg) ? msg : api().strerror_(code), " (code ", code,
              ")");
}

int32_t dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kHalf: return CRA_F16;
    case at::kBFloat16: return CRA_BF16;
    case at::kFloat: return CRA_F32;
    default: TORCH_CHECK(false, "cra::attention: unsupported dtype ", t);
  }
  return -1;
}

cra_tensor targ(const at::Tensor& t) {
  return cra_tensor{t.data_ptr(), t.stride(0), t.stride(1), t.stride(2)};
}

// D contiguous, 16-byte aligned rows, one head within 2 GiB: what the kernels
// address.
bool kernel_ready(const at::Tensor& t) {
  const int64_t es = t.element_size(), vec = 16 / es;
  const int64_t span = ((t.size(2) - 1) * t.stride(2) + t.size(3)) * es;
  return t.stride(3) == 1 && reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0 &&
         span < (int64_t(1) << 31) && t.stride(0) % vec == 0 && t.stride(1) % vec == 0 &&
         t.stride(2) % vec == 0;
}

cra_problem make_problem(const at::Tensor& q, const at::Tensor& k, int64_t window, bool relay,
                         int64_t top_k, double scale) {
  cra_problem p;
  p.B = (int32_t)q.size(0);
  p.H_q = (int32_t)q.size(1);
  p.H_kv = (int32_t)k.size(1);
  p.S = (int32_t)q.size(2);
  p.D = (int32_t)q.size(3);
  p.W = (int32_t)window;
  p.relay = relay ? 1 : 0;
  p.top_k = relay ? (int32_t)top_k : 0;
  p.dtype = dtype_code(q.scalar_type());
  p.scale = (float)scale;
  return p;
}

void* stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// Forward launches: packed global rows (one allocation for K and V rows),
// relay source rows, then the three-phase forward. Returns o, lse, the packed
// rows and the relay source rows (undefined without relay).
std::array<at::Tensor, 4> run_forward(const cra_problem& p, const at::Tensor& q,
                                      const at::Tensor& k, const at::Tensor& v) {
  const Api& a = api();
  void* st = stream_of(q);
  const int64_t G = a.global_rows(&p);
  TORCH_CHECK(G >= 0, "cra_global_rows: invalid problem");
  at::Tensor gkv = at::empty({2, p.B, p.H_kv, G, p.D}, k.options());
  char* gk = static_cast<char*>(gkv.data_ptr());
  char* gv = gk + (int64_t)p.B * p.H_kv * G * p.D * k.element_size();
  at::Tensor src;
  if (p.relay) {
    const int64_t nb = (p.S + p.W - 1) / p.W;
    src = at::empty({p.B, p.H_kv, nb * p.top_k}, k.options().dtype(at::kInt));
  }
  check(a.build_global(&p, targ(k), targ(v), gk, gv,
                       p.relay ? src.data_ptr<int32_t>() : nullptr, nullptr, st),
        "cra_build_global");
  at::Tensor o = at::empty(q.sizes(), q.options());
  at::Tensor lse = at::empty({p.B, p.H_q, p.S}, q.options().dtype(at::kFloat));
  check(a.fwd(&p, targ(q), targ(k), targ(v), gk, gv, targ(o), lse.data_ptr<float>(), st),
        "cra_fwd");
  return {o, lse, gkv, src};
}

void check_inputs(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v) {
  TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "q, k, v must be [B, H, S, D]");
  TORCH_CHECK(q.is_cuda() && k.device() == q.device() && v.device() == q.device(),
              "cra::attention: q, k, v must be on one GPU");
  TORCH_CHECK(k.sizes() == v.sizes() && k.size(0) == q.size(0) && k.size(2) == q.size(2) &&
                  k.size(3) == q.size(3) && q.size(1) % k.size(1) == 0,
              "cra::attention: shapes do not match");
  TORCH_CHECK(q.scalar_type() == k.scalar_type() && q.scalar_type() == v.scalar_type(),
              "cra::attention: q, k, v dtypes differ");
  const int64_t D = q.size(3);
  TORCH_CHECK(D == 32 || D == 64 || D == 128 || D == 256,
              "cra::attention: head dim must be 32, 64, 128 or 256");
}

// The tensor itself when the kernels take its layout, else a contiguous copy
// (what the Python path does).
at::Tensor ready(const at::Tensor& t) { return kernel_ready(t) ? t : t.contiguous(); }

class CraAttention : public torch::autograd::Function<CraAttention> {
 public:
  static at::Tensor forward(torch::autograd::AutogradContext* ctx, const at::Tensor& q_in,
                            const at::Tensor& k_in, const at::Tensor& v_in, int64_t window,
                            bool relay, int64_t top_k, double scale) {
    check_inputs(q_in, k_in, v_in);
    const at::Tensor q = ready(q_in), k = ready(k_in), v = ready(v_in);
    const cra_problem p = make_problem(q, k, window, relay, top_k, scale);
    auto r = run_forward(p, q, k, v);
    ctx->save_for_backward({q, k, v, r[0], r[1], r[2], r[3]});
    ctx->saved_data["window"] = window;
    ctx->saved_data["relay"] = relay;
    ctx->saved_data["top_k"] = top_k;
    ctx->saved_data["scale"] = scale;
    return r[0];
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const auto s = ctx->get_saved_variables();
    const at::Tensor &q = s[0], &k = s[1], &v = s[2], &o = s[3], &lse = s[4], &gkv = s[5],
                     &src = s[6];
    const cra_problem p =
        make_problem(q, k, ctx->saved_data["window"].toInt(), ctx->saved_data["relay"].toBool(),
                     ctx->saved_data["top_k"].toInt(), ctx->saved_data["scale"].toDouble());
    at::Tensor dout = grads[0].to(q.scalar_type());
    if (!kernel_ready(dout)) dout = dout.contiguous();
    const Api& a = api();
    void* st = stream_of(q);
    at::Tensor dq = at::empty(q.sizes(), q.options());
    at::Tensor dk = at::empty(k.sizes(), k.options());
    at::Tensor dv = at::empty(v.sizes(), v.options());
    const size_t nws = a.ws_bytes(&p);
    at::Tensor ws = at::empty({(int64_t)std::max<size_t>(nws, 256)}, q.options().dtype(at::kByte));
    const char* gk = static_cast<const char*>(gkv.data_ptr());
    const char* gv = gk + gkv.numel() / 2 * gkv.element_size();
    check(a.bwd(&p, targ(q), targ(k), targ(v), targ(o), targ(dout), lse.data_ptr<float>(), gk,
                gv, p.relay ? src.data_ptr<int32_t>() : nullptr, nullptr, targ(dq), targ(dk),
                targ(dv), nullptr, ws.data_ptr(), (size_t)ws.numel(), st),
          "cra_bwd");
    return {dq, dk, dv, at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor()};
  }
};

at::Tensor attention_autograd(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                              int64_t window, bool relay, int64_t top_k, double scale) {
  return CraAttention::apply(q, k, v, window, relay, top_k, scale);
}

// Below autograd (inference mode, or tensors without autograd keys): the
// forward launches alone.
at::Tensor attention_forward(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                             int64_t window, bool relay, int64_t top_k, double scale) {
  check_inputs(q, k, v);
  const at::Tensor qr = ready(q), kr = ready(k), vr = ready(v);
  return run_forward(make_problem(qr, kr, window, relay, top_k, scale), qr, kr, vr)[0];
}

}  // namespace

TORCH_LIBRARY(cra, m) {
  m.def("bind(str path) -> ()", &bind);
  m.def(
      "attention(Tensor q, Tensor k, Tensor v, int window, bool relay, int top_k, float scale)"
      " -> Tensor");
}

TORCH_LIBRARY_IMPL(cra, Autograd, m) { m.impl("attention", &attention_autograd); }

TORCH_LIBRARY_IMPL(cra, CUDA, m) { m.impl("attention", &attention_forward); }

// Host (CPU) forward of the sqrt(N) attention: what the reference computes
// for CPU tensors, `cra_cpu_fast` (cpu_reference.py:198-339, dispatched at
// core.py:3794-3796). Its plan differs from the GPU path's: window
// W = isqrt(S) (cpu_reference.py:233), relay always on with the top 2 rows
// per block by ||k||^2 (cpu_reference.py:251-268), over a last block padded
// with zero rows. For query i with ls = i - W + 1 the keys are the local
// window [max(ls, 0), i], the strided rows s*W < ls and the relay rows of
// blocks r with (r+1)*W - 1 < ls; one softmax over all of them
// (cpu_reference.py:287-337).
//
// Layout: q [B, H_q, S, D], k/v [B, H_kv, S, D] in fp32/fp16/bf16 host
// memory (D contiguous), query head h reading kv head h / (H_q / H_kv) (the
// reference repeats kv heads, cpu_reference.py:221-223). Arithmetic is fp32
// (inputs converted per row); the output is rounded once to the input type.
// Work is split over std::threads by (b, h, block of 256 queries).
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <new>
#include <thread>
#include <vector>

#include "../../include/cra.h"

namespace cra {
// Sets the calling thread's cra_last_error() text (defined beside the C ABI).
int set_error(int code, const char* msg);
}  // namespace cra

namespace {

// --- element conversions (round to nearest even) ---------------------------
inline float half_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {  // subnormal: normalise
      int e = -1;
      uint32_t m = man;
      do { m <<= 1; ++e; } while (!(m & 0x400u));
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

inline uint16_t f32_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to inf
  if (ax < 0x38800000u) {                         // below 2^-14: subnormal or zero in fp16
    if (ax < 0x33000000u) return (uint16_t)sign;  // at most half the smallest subnormal
    // value = m * 2^(e - 150); in units of 2^-24 (the fp16 subnormal step)
    // that is m * 2^(e - 126), a right shift by 126 - e (14..24)
    const uint32_t e = ax >> 23;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t sh = 126 - e;
    uint32_t r = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (r & 1))) ++r;  // 1024 becomes the smallest normal
    return (uint16_t)(sign | r);
  }
  uint32_t r = ((ax >> 13) - (112u << 10));                  // rebias exponent
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) ++r;
  return (uint16_t)(sign | r);
}

inline float bf16_to_f32(uint16_t b) {
  const uint32_t bits = (uint32_t)b << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

inline uint16_t f32_to_bf16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);  // NaN
  const uint32_t lsb = (x >> 16) & 1u;
  x += 0x7fffu + lsb;
  return (uint16_t)(x >> 16);
}

inline float load(const void* base, int64_t idx, int dtype) {
  switch (dtype) {
    case CRA_F32: return static_cast<const float*>(base)[idx];
    case CRA_F16: return half_to_f32(static_cast<const uint16_t*>(base)[idx]);
    default: return bf16_to_f32(static_cast<const uint16_t*>(base)[idx]);
  }
}

inline void store(void* base, int64_t idx, float x, int dtype) {
  switch (dtype) {
    case CRA_F32: static_cast<float*>(base)[idx] = x; break;
    case CRA_F16: static_cast<uint16_t*>(base)[idx] = f32_to_half(x); break;
    default: static_cast<uint16_t*>(base)[idx] = f32_to_bf16(x); break;
  }
}

// a value rounded to the input type (the reference computes the relay
// norms in the input dtype)
inline float round_to(float x, int dtype) {
  switch (dtype) {
    case CRA_F32: return x;
    case CRA_F16: return half_to_f32(f32_to_half(x));
    default: return bf16_to_f32(f32_to_bf16(x));
  }
}

inline float dot(const float* a, const float* b, int n) {
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  int d = 0;
  for (; d + 4 <= n; d += 4) {
    s0 += a[d] * b[d];
    s1 += a[d + 1] * b[d + 1];
    s2 += a[d + 2] * b[d + 2];
    s3 += a[d + 3] * b[d + 3];
  }
  for (; d < n; ++d) s0 += a[d] * b[d];
  return (s0 + s1) + (s2 + s3);
}

inline void axpy(float* y, float a, const float* x, int n) {
  for (int d = 0; d < n; ++d) y[d] += a * x[d];
}

// One (b, kv head): the rows as fp32 and the "global" rows every query may
// see besides its window -- strided rows s*W, then 2 relay rows per block
// (zero rows where the padded last block runs past S) -- with the query
// threshold each needs (visible to query i iff thr < i - W + 1).
struct KvHead {
  std::vector<float> k, v;          // [S, D]
  std::vector<float> gk, gv;        // [G, D]
  std::vector<int64_t> thr;         // [G]
};

void build_kv_head(const cra_problem* p, cra_tensor k, cra_tensor v, int b, int hk,
                   KvHead* out) {
  const int S = p->S, D = p->D, W = p->W, dt = p->dtype;
  const int top_k = p->relay ? p->top_k : 0;
  out->k.resize((size_t)S * D);
  out->v.resize((size_t)S * D);
  const int64_t kb = b * k.sb + hk * k.sh, vb = b * v.sb + hk * v.sh;
  for (int i = 0; i < S; ++i)
    for (int d = 0; d < D; ++d) {
      out->k[(size_t)i * D + d] = load(k.ptr, kb + i * k.ss + d, dt);
      out->v[(size_t)i * D + d] = load(v.ptr, vb + i * v.ss + d, dt);
    }
  const int NB = (S + W - 1) / W;
  const int G = NB * (1 + top_k);
  out->gk.assign((size_t)G * D, 0.f);
  out->gv.assign((size_t)G * D, 0.f);
  out->thr.resize(G);
  int g = 0;
  for (int s = 0; s < NB; ++s, ++g) {  // strided rows first (cpu_reference.py:244-247)
    memcpy(&out->gk[(size_t)g * D], &out->k[(size_t)s * W * D], D * sizeof(float));
    memcpy(&out->gv[(size_t)g * D], &out->v[(size_t)s * W * D], D * sizeof(float));
    out->thr[g] = (int64_t)s * W;
  }
  std::vector<float> norm(W);
  std::vector<int> order(W);
  for (int r = 0; r < NB && top_k > 0; ++r) {
    // ||k||^2 of the block's W rows (zero for padding rows) as the reference
    // computes it in the input type, (k * k).sum(-1): each square rounded to
    // the type, an fp32 sum, one final rounding; the top_k largest, the
    // earlier row first on equal norms
    for (int j = 0; j < W; ++j) {
      const int row = r * W + j;
      float n2 = 0.f;
      if (row < S) {
        const float* kr = &out->k[(size_t)row * D];
        for (int d = 0; d < D; ++d) n2 += round_to(kr[d] * kr[d], dt);
        n2 = round_to(n2, dt);
      }
      norm[j] = n2;
      order[j] = j;
    }
    std::stable_sort(order.begin(), order.end(), [&](int a, int c) { return norm[a] > norm[c]; });
    for (int t = 0; t < std::min(top_k, W); ++t, ++g) {
      const int row = r * W + order[t];
      if (row < S) {
        memcpy(&out->gk[(size_t)g * D], &out->k[(size_t)row * D], D * sizeof(float));
        memcpy(&out->gv[(size_t)g * D], &out->v[(size_t)row * D], D * sizeof(float));
      }
      out->thr[g] = (int64_t)(r + 1) * W - 1;  // block end (cpu_reference.py:276-278)
    }
  }
  out->gk.resize((size_t)g * D);
  out->gv.resize((size_t)g * D);
  out->thr.resize(g);
}

// Queries [q0, q1) of head (b, h) against their kv head.
void attend_rows(const cra_problem* p, cra_tensor q, cra_tensor o, int b, int h,
                 const KvHead& kv, int q0, int q1, std::vector<float>& qrow,
                 std::vector<float>& sc, std::vector<float>& acc) {
  const int D = p->D, W = p->W, dt = p->dtype;
  const int G = (int)kv.thr.size();
  const int64_t qb = b * q.sb + h * q.sh, ob = b * o.sb + h * o.sh;
  qrow.resize(D);
  acc.resize(D);
  sc.resize((size_t)W + G);
  for (int i = q0; i < q1; ++i) {
    for (int d = 0; d < D; ++d) qrow[d] = load(q.ptr, qb + i * q.ss + d, dt);
    const int64_t ls = (int64_t)i - W + 1;
    const int j0 = (int)std::max<int64_t>(ls, 0);
    int n = 0;
    float mx = -INFINITY;
    for (int j = j0; j <= i; ++j, ++n) {
      sc[n] = dot(qrow.data(), &kv.k[(size_t)j * D], D) * p->scale;
      mx = std::max(mx, sc[n]);
    }
    for (int g = 0; g < G; ++g) {
      if (!(kv.thr[g] < ls)) continue;
      sc[n] = dot(qrow.data(), &kv.gk[(size_t)g * D], D) * p->scale;
      mx = std::max(mx, sc[n]);
      ++n;
    }
    std::fill(acc.begin(), acc.end(), 0.f);
    float sum = 0.f;
    n = 0;
    for (int j = j0; j <= i; ++j, ++n) {
      const float e = expf(sc[n] - mx);
      sum += e;
      axpy(acc.data(), e, &kv.v[(size_t)j * D], D);
    }
    for (int g = 0; g < G; ++g) {
      if (!(kv.thr[g] < ls)) continue;
      const float e = expf(sc[n++] - mx);
      sum += e;
      axpy(acc.data(), e, &kv.gv[(size_t)g * D], D);
    }
    const float inv = 1.f / std::max(sum, 1e-12f);  // clamp of cpu_reference.py:334
    for (int d = 0; d < D; ++d) store(o.ptr, ob + i * o.ss + d, acc[d] * inv, dt);
  }
}

}  // namespace

namespace {

int fwd_cpu_impl(const cra_problem* p, cra_tensor q, cra_tensor k, cra_tensor v, cra_tensor o,
                 int32_t threads) {
  if (!p) return cra::set_error(CRA_E_INVALID, "cra_fwd_cpu: problem is NULL");
  if (!q.ptr || !k.ptr || !v.ptr || !o.ptr)
    return cra::set_error(CRA_E_INVALID, "cra_fwd_cpu: q, k, v and o must not be NULL");
  if (p->dtype != CRA_F16 && p->dtype != CRA_BF16 && p->dtype != CRA_F32)
    return cra::set_error(CRA_E_DTYPE, "cra_fwd_cpu: unknown dtype code");
  if (p->B < 1 || p->H_q < 1 || p->H_kv < 1 || p->S < 1 || p->D < 1)
    return cra::set_error(CRA_E_INVALID, "cra_fwd_cpu: B, H_q, H_kv, S and D must be >= 1");
  if (p->H_q % p->H_kv)
    return cra::set_error(CRA_E_INVALID, "cra_fwd_cpu: H_q must be a multiple of H_kv");
  if (p->W < 1 || p->W > p->S)
    return cra::set_error(CRA_E_INVALID, "cra_fwd_cpu: window W outside [1, S]");
  if (p->relay && (p->top_k < 1 || p->top_k > 4))
    return cra::set_error(CRA_E_INVALID, "cra_fwd_cpu: top_k outside [1, 4]");
  if (!(p->scale > 0.f)) return cra::set_error(CRA_E_INVALID, "cra_fwd_cpu: scale must be > 0");
  const int groups = p->H_q / p->H_kv;
  const int nthr = std::max(1, threads);
  // kv heads first (each shared by its query heads), then query blocks
  std::vector<KvHead> heads((size_t)p->B * p->H_kv);
  std::atomic<int> next{0};
  std::atomic<bool> failed{false};
  auto run = [&](auto&& body, int n) {
    next = 0;
    std::vector<std::thread> pool;
    const int nt = std::min(nthr, n);
    // an exception may not leave a thread's function: the item fails the call
    auto work = [&] {
      try {
        for (int i = next++; i < n; i = next++) body(i);
      } catch (...) {
        failed = true;
        next = n;
      }
    };
    try {
      for (int t = 1; t < nt; ++t) pool.emplace_back(work);
    } catch (...) {
      // fewer workers than asked (thread creation failed): the ones started
      // and this thread still take every item
    }
    work();
    for (auto& th : pool) th.join();
  };
  run([&](int i) { build_kv_head(p, k, v, i / p->H_kv, i % p->H_kv, &heads[i]); },
      p->B * p->H_kv);
  if (failed) return cra::set_error(CRA_E_INVALID, "cra_fwd_cpu: out of host memory");
  constexpr int kChunk = 256;
  const int nch = (p->S + kChunk - 1) / kChunk;
  run(
      [&](int i) {
        thread_local std::vector<float> qrow, sc, acc;
        const int c = i % nch, bh = i / nch;
        const int b = bh / p->H_q, h = bh % p->H_q;
        attend_rows(p, q, o, b, h, heads[(size_t)b * p->H_kv + h / groups], c * kChunk,
                    std::min(p->S, (c + 1) * kChunk), qrow, sc, acc);
      },
      p->B * p->H_q * nch);
  if (failed) return cra::set_error(CRA_E_INVALID, "cra_fwd_cpu: out of host memory");
  return CRA_OK;
}

}  // namespace

// No exception crosses the C ABI: an allocation failure becomes an error code.
extern "C" int cra_fwd_cpu(const cra_problem* p, cra_tensor q, cra_tensor k, cra_tensor v,
                           cra_tensor o, int32_t threads) {
  try {
    return fwd_cpu_impl(p, q, k, v, o, threads);
  } catch (const std::bad_alloc&) {
    return cra::set_error(CRA_E_INVALID, "cra_fwd_cpu: out of host memory");
  } catch (...) {
    return cra::set_error(CRA_E_INVALID, "cra_fwd_cpu: host error");
  }
}

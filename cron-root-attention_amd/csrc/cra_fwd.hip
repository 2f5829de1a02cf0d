// Forward: three-phase sqrt(N) attention with one online softmax.
//
// Reference semantics: `_cron_root_attn_fwd_v14_tiled` (core.py:907-1158).
// Per query i (ls = max(0, i-W+1)) the keys are the local window [ls, i]
// (core.py:976-1028) and the global rows -- strided rows s*W < ls
// (core.py:1042-1087) and the relay rows of blocks ending before ls
// (core.py:1097-1142). The global rows arrive packed per block
// (cra_global.hip), so the global set of query i is a prefix of one array and
// both phases are dense MFMA contractions with a mask only on edge tiles
// (the reference streams every relay row for every tile).
// Scores are fp32 dot(q, k) * scale; P is rounded to the input dtype before
// P.V (core.py:1027, 1086, 1141); O = acc / l and LSE = m + ln(l)
// (core.py:1147-1158). Unlike the reference, whose l sums the unrounded P
// (core.py:1028), l sums the rounded P of the 2-byte types.
//
// Mapping: one workgroup = 4 waves = 128 consecutive queries of one (b, h);
// each wave owns 32 queries. K/V tiles of 64 rows (32 for fp32) are staged in
// LDS, K row-major and V transposed. S^T = K . Q^T puts a query on lane%16 so
// the per-query softmax state is lane-local; O^T = V^T . P^T consumes P^T
// straight from the S^T registers. Tiles are launched heaviest first (work
// per query grows with i) and consecutive workgroups are different heads of
// the same tile, so each XCD keeps a fixed pair of heads.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "cra_common.hpp"
#include "cra_internal.hpp"

namespace cra {

namespace {

// Geometry of the generic forward (fwd_kernel: the fp32 path, and every
// dtype at head dim 256). NB = 16-query blocks per wave: two below D = 256,
// one at D = 256 (two would hold 256 VGPRs of accumulators and Q operands).
template <typename T, int D, int NB = 2>
struct FwdTraits {
  static constexpr int kWaves = 4;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kQW = 16 * NB;                // queries per wave
  static constexpr int kBM = kWaves * kQW;           // queries per workgroup
  static constexpr int kBN = (sizeof(T) == 4 || D > 128) ? 32 : 64;  // key rows per LDS tile
  static constexpr int kKB = kBN / 16;               // 16-row key blocks
  static constexpr int kKC = kBN / 32;               // 32-row key chunks
  static constexpr int kDC = D / 32;                 // 32-wide head-dim chunks
  static constexpr int kDB = D / 16;                 // 16-wide head-dim blocks
  static constexpr int kLD = D + 16 / (int)sizeof(T);  // row-major tile stride
  static constexpr int kLDT = kBN + 4;               // transposed tile stride
};

// One key tile against the wave's 16 * NB queries: S^T, masked online
// softmax, O^T += V^T P^T. `valid(key_offset, qb)` says whether tile row
// key_offset is in the set of query block qb's lane query.
template <typename T, int D, int NB, bool MASK, typename Valid>
__device__ __forceinline__ void attend_tile(const T* sK, const T* sVt,
                                            const Frag<T> (&qf)[NB][FwdTraits<T, D, NB>::kDC],
                                            f32x4 (&acc)[FwdTraits<T, D, NB>::kDB][NB],
                                            float (&m_run)[NB], float (&l_run)[NB], float c2,
                                            int l16, int g, Valid valid) {
  using Tr = FwdTraits<T, D, NB>;
  f32x4 s[Tr::kKB][NB];
#pragma unroll
  for (int kb = 0; kb < Tr::kKB; ++kb) {
#pragma unroll
    for (int qb = 0; qb < NB; ++qb) s[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < Tr::kDC; ++c) {
      const Frag<T> kf = lds_frag_row<T>(sK + (16 * kb + l16) * Tr::kLD + 32 * c + 8 * g);
#pragma unroll
      for (int qb = 0; qb < NB; ++qb) s[kb][qb] = mma(s[kb][qb], kf, qf[qb][c]);
    }
  }
  Frag<T> pf[Tr::kKC][NB];
#pragma unroll
  for (int qb = 0; qb < NB; ++qb) {
    float t[Tr::kKB][4];
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int kb = 0; kb < Tr::kKB; ++kb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = s[kb][qb][r] * c2;
        if (MASK && !valid(16 * kb + 4 * g + r, qb)) x = -__builtin_huge_valf();
        t[kb][r] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = group_max(mx);
    const float m_new = fmaxf(m_run[qb], mx);
    const float m_use = m_new == -__builtin_huge_valf() ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - m_use);
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < Tr::kKB; ++kb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = __builtin_amdgcn_exp2f(t[kb][r] - m_use);
        t[kb][r] = p;
        psum += p;
      }
    }
    l_run[qb] = l_run[qb] * alpha + psum;
    m_run[qb] = m_new;
#pragma unroll
    for (int db = 0; db < Tr::kDB; ++db) acc[db][qb] *= alpha;
#pragma unroll
    for (int kc = 0; kc < Tr::kKC; ++kc) {
      const float v8[8] = {t[2 * kc][0],     t[2 * kc][1],     t[2 * kc][2],     t[2 * kc][3],
                           t[2 * kc + 1][0], t[2 * kc + 1][1], t[2 * kc + 1][2], t[2 * kc + 1][3]};
      pf[kc][qb] = pack8<T>(v8);
    }
  }
#pragma unroll
  for (int db = 0; db < Tr::kDB; ++db) {
    const T* row = sVt + (16 * db + l16) * Tr::kLDT;
#pragma unroll
    for (int kc = 0; kc < Tr::kKC; ++kc) {
      const Frag<T> vf = lds_frag_2x4<T>(row + 32 * kc + 4 * g, row + 32 * kc + 16 + 4 * g);
#pragma unroll
      for (int qb = 0; qb < NB; ++qb) acc[db][qb] = mma(acc[db][qb], vf, pf[kc][qb]);
    }
  }
}

// At D = 256 the 2-byte forward fits 2 waves per SIMD (at most 256 VGPRs).
template <typename T, int D, int NB>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(D > 128 && sizeof(T) == 2 ? 2 : 1)))
void fwd_kernel(FwdArgs a) {
  using Tr = FwdTraits<T, D, NB>;
  __shared__ __attribute__((aligned(16))) T sK[Tr::kBN * Tr::kLD];
  __shared__ __attribute__((aligned(16))) T sVt[D * Tr::kLDT];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int nbh = a.B * a.Hq;
  const int bh = blockIdx.x % nbh;
  const Doc dc = find_doc(a.docs, (int)(blockIdx.x / nbh));
  const int tile = (dc.len + Tr::kBM - 1) / Tr::kBM - 1 - dc.item;  // heaviest first
  const int b = bh / a.Hq, h = bh % a.Hq;
  const int hk = h / (a.Hq / a.Hkv);
  const int m0 = tile * Tr::kBM;
  const int q0 = m0 + wave * Tr::kQW;
  const int S = dc.len, W = dc.W, rpb = dc.rpb;

  const T* qp = static_cast<const T*>(a.q) + b * a.qsb + h * a.qsh + (int64_t)dc.off * a.qss;
  const T* kp = static_cast<const T*>(a.k) + b * a.ksb + hk * a.ksh + (int64_t)dc.off * a.kss;
  const T* vp = static_cast<const T*>(a.v) + b * a.vsb + hk * a.vsh + (int64_t)dc.off * a.vss;
  float* lse = a.lse + (int64_t)bh * a.S + dc.off;
  const int64_t gbase = ((int64_t)(b * a.Hkv + hk) * a.G + dc.gofs) * D;
  const T* gkp = static_cast<const T*>(a.gk) + gbase;
  const T* gvp = static_cast<const T*>(a.gv) + gbase;

  // Q as the B operand of S^T = K . Q^T: lane holds q[qi][32c + 8g .. +8].
  Frag<T> qf[NB][Tr::kDC];
  int qi[NB];
#pragma unroll
  for (int qb = 0; qb < NB; ++qb) {
    qi[qb] = q0 + 16 * qb + l16;
#pragma unroll
    for (int c = 0; c < Tr::kDC; ++c) {
      if (qi[qb] < S) {
        qf[qb][c] = lds_frag_row<T>(qp + (int64_t)qi[qb] * a.qss + 32 * c + 8 * g);
      } else {
#pragma unroll
        for (int w = 0; w < Frag<T>::kWords; ++w) qf[qb][c].w[w] = make_uint4(0, 0, 0, 0);
      }
    }
  }

  const float c2 = a.scale * kLog2e;
  float m_run[NB], l_run[NB];
  f32x4 acc[Tr::kDB][NB];
#pragma unroll
  for (int qb = 0; qb < NB; ++qb) {
    m_run[qb] = -__builtin_huge_valf();
    l_run[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < Tr::kDB; ++db) acc[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const bool active = q0 < S;
  const int q_last = min(q0 + Tr::kQW, S) - 1;
  TileStage<T, D, Tr::kBN, Tr::kThreads> stk, stv;

  // ---- phase 1: local window -------------------------------------------
  const int lo = max(0, m0 - W + 1);
  const int hi = min(S, m0 + Tr::kBM);
  const int w_lo = max(0, q0 - W + 1);
  const int hi_loc = (a.phases & 1) ? hi : lo;
  for (int ts = lo; ts < hi_loc; ts += Tr::kBN) {
    stk.load(kp, a.kss, ts, 0, hi, tid);
    stv.load(vp, a.vss, ts, 0, hi, tid);
    __syncthreads();
    stk.template store_rows<Tr::kLD>(sK, tid);
    stv.template store_cols<Tr::kLDT>(sVt, tid);
    __syncthreads();
    if (active && ts <= q_last && ts + Tr::kBN - 1 >= w_lo) {
      const bool full = ts >= q_last - W + 1 && ts + Tr::kBN - 1 <= q0;
      auto valid = [&](int ko, int qb) {
        const int j = ts + ko;
        return j <= qi[qb] && j >= qi[qb] - W + 1;
      };
      if (full)
        attend_tile<T, D, NB, false>(sK, sVt, qf, acc, m_run, l_run, c2, l16, g, valid);
      else
        attend_tile<T, D, NB, true>(sK, sVt, qf, acc, m_run, l_run, c2, l16, g, valid);
    }
  }

  // ---- phase 2+3: prefix of the packed strided/relay rows ---------------
  const int gmax = glob_prefix(hi - 1, W, rpb);
  const int wg_lo = active ? glob_prefix(q0, W, rpb) : 0;
  const int wg_hi = active ? glob_prefix(q_last, W, rpb) : 0;
  int glen[NB];
#pragma unroll
  for (int qb = 0; qb < NB; ++qb) glen[qb] = glob_prefix(qi[qb], W, rpb);
  const int g_end = (a.phases & 2) ? gmax : 0;
  for (int ts = 0; ts < g_end; ts += Tr::kBN) {
    stk.load(gkp, D, ts, 0, gmax, tid);
    stv.load(gvp, D, ts, 0, gmax, tid);
    __syncthreads();
    stk.template store_rows<Tr::kLD>(sK, tid);
    stv.template store_cols<Tr::kLDT>(sVt, tid);
    __syncthreads();
    if (active && ts < wg_hi) {
      auto valid = [&](int ko, int qb) { return ts + ko < glen[qb]; };
      if (ts + Tr::kBN <= wg_lo)
        attend_tile<T, D, NB, false>(sK, sVt, qf, acc, m_run, l_run, c2, l16, g, valid);
      else
        attend_tile<T, D, NB, true>(sK, sVt, qf, acc, m_run, l_run, c2, l16, g, valid);
    }
  }

  // ---- epilogue: O = acc / l, LSE = (m + log2 l) ln 2 ---------------------
  T* op = static_cast<T*>(a.o) + b * a.osb + h * a.osh + (int64_t)dc.off * a.oss;
#pragma unroll
  for (int qb = 0; qb < NB; ++qb) {
    const float l = group_sum(l_run[qb]);
    if (!active || qi[qb] >= S) continue;
    const float inv = 1.f / fmaxf(l, 1e-6f);
    T* orow = op + (int64_t)qi[qb] * a.oss;
#pragma unroll
    for (int db = 0; db < Tr::kDB; ++db) {
      T e[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) e[r] = from_f32<T>(acc[db][qb][r] * inv);
      if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<uint2*>(orow + 16 * db + 4 * g) = *reinterpret_cast<const uint2*>(e);
      } else {
        *reinterpret_cast<uint4*>(orow + 16 * db + 4 * g) = *reinterpret_cast<const uint4*>(e);
      }
    }
    if (g == 0)
      lse[qi[qb]] = (m_run[qb] + __builtin_amdgcn_logf(fmaxf(l, 1e-6f))) * kLn2;
  }
}

// ---------------------------------------------------------------------------
// fp16/bf16 forward. Same mapping as fwd_kernel (4 waves x 32 queries), but
// K/V tiles (64 rows) are double-buffered in swizzled LDS, filled with
// global_load_lds while the previous tile is computed, V^T operands come from
// ds_read_b64_tr_b16 on the row-major V tile, each tile is processed in two
// 32-key halves, and the running max is raised only when the rounded
// exponentials of a half against it sum past 2^15 (each P stays <= 2^15;
// O and LSE are exact for any reference max). The normaliser l sums the
// rounded P that the P.V MFMAs use.
// ---------------------------------------------------------------------------
// MFMA steps by which the forward's LDS operand reads run ahead of their use
// (K row fragments and transposed V fragments). Three measured 0.6% faster
// than two and four no better than two (D = 128: 242, 238 and 246 VGPRs, 2
// waves per SIMD either way; D = 64 stays at 168, 3 waves per SIMD).
#ifndef CRA_FWD_PF
#define CRA_FWD_PF 3
#endif

template <int D>
struct Fwd2Lane {
  int k[D / 32];   // K row fragment, chunk 4c + g, row lane%16
  int v[D / 16];   // V^T fragment, columns 16 db ..
};

template <typename T, int D, int BN>
__device__ __forceinline__ void tile_scores(const char* tK, const Fwd2Lane<D>& lo,
                                            const Frag<T> (&qf)[2][D / 32], int kc,
                                            f32x4 (&s)[2][2]) {
  using Tile = SwzTile<D, BN>;
  constexpr int NC = D / 32, NK = 2 * NC;
  // K fragments are read CRA_FWD_PF steps ahead of the MFMAs that use them; fences
  // keep the compiler from moving the reads next to their uses. Step t takes
  // key block t % 2 and D-chunk t / 2, so the four accumulators alternate and
  // each MFMA's accumulator was last written four MFMAs earlier (key block
  // major, two apart, measured 0.5% slower).
  auto k_frag = [&](int t) {
    return Tile::template row_frag_at<T>(tK + (2 * kc + t % 2) * Tile::kBlk16 + lo.k[t / 2]);
  };
  constexpr int PF = CRA_FWD_PF < NK ? CRA_FWD_PF : NK;
  Frag<T> kf[PF + 1];
#pragma unroll
  for (int t = 0; t < PF; ++t) kf[t] = k_frag(t);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < NK; ++t) {
    if (t + PF < NK) kf[(t + PF) % (PF + 1)] = k_frag(t + PF);
    const int h = t % 2, c = t / 2;
    if (c == 0) s[h][0] = s[h][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    s[h][0] = mma(s[h][0], kf[t % (PF + 1)], qf[0][c]);
    s[h][1] = mma(s[h][1], kf[t % (PF + 1)], qf[1][c]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// O^T += V^T . P^T for 32-key half kh: transposed V fragments read
// CRA_FWD_PF steps ahead of the MFMAs that use them.
template <typename T, int D, int BN>
__device__ __forceinline__ void pv_half(const char* tV, int kh, const Fwd2Lane<D>& lo,
                                        const Frag<T> (&pf)[2], f32x4 (&acc)[D / 16][2]) {
  using Tile = SwzTile<D, BN>;
  constexpr int NDB = D / 16;
  auto tr_v = [&](int db) {
    const char* pa = tV + (2 * kh) * Tile::kBlk16 + lo.v[db];
    return Tile::template tr_frag_at<T>(pa, pa + Tile::kBlk16);
  };
  constexpr int PF = CRA_FWD_PF < NDB ? CRA_FWD_PF : NDB;
  Frag<T> vt[PF + 1];
#pragma unroll
  for (int db = 0; db < PF; ++db) vt[db] = tr_v(db);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    if (db + PF < NDB) vt[(db + PF) % (PF + 1)] = tr_v(db + PF);
    acc[db][0] = mma(acc[db][0], vt[db % (PF + 1)], pf[0]);
    acc[db][1] = mma(acc[db][1], vt[db % (PF + 1)], pf[1]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Largest sum of a half's 32 rounded exponentials accepted against the
// running maximum: each term is then at most 2^15 and finite in fp16.
constexpr float kSumMax = 32768.f;

// All-ones A operand: ones . P^T puts the sum over the 32 keys of each query
// (column of P^T) in all four of that query's lanes' result rows.
template <typename T>
__device__ __forceinline__ Frag<T> ones_frag() {
  Frag<T> f;
  const uint32_t w = sizeof(T) == 2 ? (std::is_same<T, bf16>::value ? 0x3f803f80u : 0x3c003c00u)
                                    : 0u;
  f.w[0] = make_uint4(w, w, w, w);
  return f;
}

// Sum of the rounded P of a 32-key half for each query, on the matrix core
// (one MFMA in place of four v_dot2 per lane plus a cross-lane sum).
template <typename T>
__device__ __forceinline__ float half_sum(const Frag<T>& pk, const Frag<T>& one) {
  return mma(f32x4{0.f, 0.f, 0.f, 0.f}, one, pk)[0];
}

// Exponentials of one 32-key half (8 per lane and query block) against the
// running maximum, rounded to the input type, and the sum of the rounded
// values over the half's 32 keys (the P.V operand and its normaliser).
template <typename T, bool MASK>
__device__ __forceinline__ void half_exp(f32x4 (&s)[2][2], int kc, int qb, float c2, float m,
                                         int g, const TileMask<2>& mk, const Frag<T>& one,
                                         Frag<T>& pk, float& ps) {
  float pv[8];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (MASK && !mk.ok(32 * kc + 16 * h + 4 * g + r, qb)) s[h][qb][r] = -__builtin_huge_valf();
      pv[4 * h + r] = __builtin_amdgcn_exp2f(fmaf(s[h][qb][r], c2, -m));
    }
  pk = pack8<T>(pv);
  ps = half_sum(pk, one);
}

// Raise the running maximum of query block qb to this half's maximum,
// rescale its accumulators and redo the half's exponentials. Taken for the
// first visible keys and whenever a score exceeds the running maximum by
// enough to push a sum of 8 rounded terms past kSumMax (inf and NaN sums
// included).
template <typename T, int D>
__device__ __forceinline__ void half_rescale(f32x4 (&s)[2][2], int qb, float c2,
                                             f32x4 (&acc)[D / 16][2], float (&m_run)[2],
                                             float (&l_run)[2], const Frag<T>& one, Frag<T>& pk,
                                             float& ps) {
  float mx = -__builtin_huge_valf();
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[h][qb][r]);
  const float m_new = fmaxf(m_run[qb], group_max(mx * c2));
  // Until a query's first visible key its accumulators and l are zero; the
  // whole wave's first rescale (its first tile) has nothing to scale.
  if (!__all(m_run[qb] == -__builtin_huge_valf())) {
    const float alpha =
        m_run[qb] == -__builtin_huge_valf() ? 0.f : __builtin_amdgcn_exp2f(m_run[qb] - m_new);
    l_run[qb] *= alpha;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) acc[db][qb] *= alpha;
  }
  m_run[qb] = m_new;
  const float mu = m_new == -__builtin_huge_valf() ? 0.f : m_new;
  float pv[8];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int r = 0; r < 4; ++r) pv[4 * h + r] = __builtin_amdgcn_exp2f(fmaf(s[h][qb][r], c2, -mu));
  pk = pack8<T>(pv);
  ps = half_sum(pk, one);
}

// One BN-key tile for the wave's 32 queries, in 32-key halves. The online
// softmax keeps a lazily raised running maximum: exponentials are taken
// against it first and the maximum is recomputed only when their sum says a
// term got too large. Program order puts the next half's score MFMAs and the
// previous half's PV MFMAs beside each half's exponentials, in one basic
// block, so matrix and vector work can overlap.
template <typename T, int D, int BN, bool MASK>
__device__ __forceinline__ void attend_tile2(const char* tK, const char* tV, const Fwd2Lane<D>& lo,
                                             const Frag<T> (&qf)[2][D / 32],
                                             f32x4 (&acc)[D / 16][2], float (&m_run)[2],
                                             float (&l_run)[2], float c2, int g,
                                             const TileMask<2>& mk, const Frag<T>& one) {
  using Tile = SwzTile<D, BN>;
  constexpr int kHalves = BN / 32;
  f32x4 s[kHalves][2][2];
  tile_scores<T, D, BN>(tK, lo, qf, 0, s[0]);
  Frag<T> pf[2];
#pragma unroll
  for (int kc = 0; kc < kHalves; ++kc) {
    Frag<T> pn[2];
    float ps[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
      half_exp<T, MASK>(s[kc], kc, qb, c2, m_run[qb], g, mk, one, pn[qb], ps[qb]);
    if (kc > 0) pv_half<T, D, BN>(tV, kc - 1, lo, pf, acc);  // beside this half's exponentials
    if (kc + 1 < kHalves) tile_scores<T, D, BN>(tK, lo, qf, kc + 1, s[kc + 1]);
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      if (__any(!(ps[qb] <= kSumMax)))
        half_rescale<T, D>(s[kc], qb, c2, acc, m_run, l_run, one, pn[qb], ps[qb]);
      l_run[qb] += ps[qb];
      pf[qb] = pn[qb];
    }
  }
  pv_half<T, D, BN>(tV, kHalves - 1, lo, pf, acc);
}

// One 32-key half kc of a masked tile, for tiles whose other half has no
// key visible to any of the wave's queries (window and prefix edges).
template <typename T, int D, int BN>
__device__ __forceinline__ void attend_half(const char* tK, const char* tV, int kc,
                                            const Fwd2Lane<D>& lo, const Frag<T> (&qf)[2][D / 32],
                                            f32x4 (&acc)[D / 16][2], float (&m_run)[2],
                                            float (&l_run)[2], float c2, int g,
                                            const TileMask<2>& mk, const Frag<T>& one) {
  using Tile = SwzTile<D, BN>;
  f32x4 s[2][2];
  tile_scores<T, D, BN>(tK, lo, qf, kc, s);
  float ps[2];
  Frag<T> pf[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
    half_exp<T, true>(s, kc, qb, c2, m_run[qb], g, mk, one, pf[qb], ps[qb]);
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    if (__any(!(ps[qb] <= kSumMax)))
      half_rescale<T, D>(s, qb, c2, acc, m_run, l_run, one, pf[qb], ps[qb]);
    l_run[qb] += ps[qb];
  }
  pv_half<T, D, BN>(tV, kc, lo, pf, acc);
}

// NW waves of 32 queries share each K/V tile of BN = 64 rows (2 x 32 KB
// double buffer at D = 128); at least 2 waves per SIMD at D = 128 (240
// VGPRs), 3 below it (168 VGPRs at D = 64, where the compiler's own choice
// of 174 allowed only 2: the D = 64 forward is 8% faster at 3). PH selects the key
// phases (bit 0 local window, bit 1 global rows) at compile time, so the
// phase-restricted launches are kernels of their own in a trace.
template <int D>
using FwdStage = char[2][SwzTile<D, 64>::kBytes];  // K and V tiles of one pipeline stage

// One work item (a 128-query tile of one (b, h); items numbered heaviest
// first, consecutive items on different heads) with its LDS stages.
template <typename T, int D, int NW, int PH>
__device__ __forceinline__ void fwd2_item(const FwdArgs& a, const int item, FwdStage<D>& stage0,
                                          FwdStage<D>& stage1) {
  constexpr int BN = 64;
  using Tile = SwzTile<D, BN>;
  constexpr int kQW = 32, kBM = NW * kQW, kBN = BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int nbh = a.B * a.Hq;
  const int bh = item % nbh;
  const Doc dc = find_doc(a.docs, item / nbh);
  const int tile = (dc.len + kBM - 1) / kBM - 1 - dc.item;  // heaviest first
  const int b = bh / a.Hq, h = bh % a.Hq;
  const int hk = h / (a.Hq / a.Hkv);
  const int m0 = tile * kBM;
  const int q0 = m0 + wave * kQW;
  const int S = dc.len, W = dc.W, rpb = dc.rpb;

  const T* qp = static_cast<const T*>(a.q) + b * a.qsb + h * a.qsh + (int64_t)dc.off * a.qss;
  const T* kp = static_cast<const T*>(a.k) + b * a.ksb + hk * a.ksh + (int64_t)dc.off * a.kss;
  const T* vp = static_cast<const T*>(a.v) + b * a.vsb + hk * a.vsh + (int64_t)dc.off * a.vss;
  float* lse = a.lse + (int64_t)bh * a.S + dc.off;
  const int64_t gbase = ((int64_t)(b * a.Hkv + hk) * a.G + dc.gofs) * D;
  const T* gkp = static_cast<const T*>(a.gk) + gbase;
  const T* gvp = static_cast<const T*>(a.gv) + gbase;

  const int lo_k = max(0, m0 - W + 1);
  const int hi = min(S, m0 + kBM);
  const int gmax = glob_prefix(hi - 1, W, rpb);
  const int nloc = (PH & 1) ? (hi - lo_k + kBN - 1) / kBN : 0;
  // Global tiles come first: every workgroup of the head reads them, so the
  // first fill (issued before anything can hide it) is an L2 hit, and the
  // cold local rows are fetched while global tiles are computed. The local
  // window is then walked from its highest key tile down: the workgroup of
  // the next lower query tile (launched next for this head) walks down the
  // same keys one or two tiles behind and finds them in L2 (the forward's HBM
  // reads drop from 1.32 to 1.14 times the compulsory bytes).
  const int nglob = (PH & 2) ? (gmax + kBN - 1) / kBN : 0;
  const int ntot = nloc + nglob;

  // Buffer resources over the rows this workgroup may read (local rows below
  // hi, global rows below gmax): loads past them return zeros. 32-bit
  // offsets, uniform bases.
  using Fill = typename Tile::template Fill<NW>;
  const int kbytes = (int)(a.kss * 2), vbytes = (int)(a.vss * 2);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kp, (uint32_t)((hi - 1) * kbytes + D * 2));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vp, (uint32_t)((hi - 1) * vbytes + D * 2));
  const __amdgpu_buffer_rsrc_t rgk = make_rsrc(gkp, (uint32_t)(gmax * D * 2));
  const __amdgpu_buffer_rsrc_t rgv = make_rsrc(gvp, (uint32_t)(gmax * D * 2));
  const int fk = Fill::lane_off(wave, lane, kbytes);
  const int fv = Fill::lane_off(wave, lane, vbytes);
  const int fg = Fill::lane_off(wave, lane, D * 2);
  auto issue = [&](int it, char* dst) {
    if (it >= nglob) {
      const int ts = lo_k + (nloc - 1 - (it - nglob)) * kBN;
      Fill::load(dst, rk, fk, kbytes, ts, wave);
      Fill::load(dst + Tile::kBytes, rv, fv, vbytes, ts, wave);
    } else {
      const int ts = it * kBN;
      Fill::load(dst, rgk, fg, D * 2, ts, wave);
      Fill::load(dst + Tile::kBytes, rgv, fg, D * 2, ts, wave);
    }
  };
  issue(0, stage0[0]);

  Fwd2Lane<D> lo;
#pragma unroll
  for (int c = 0; c < D / 32; ++c) lo.k[c] = Tile::row_lane_off(lane, 4 * c + g);
#pragma unroll
  for (int db = 0; db < D / 16; ++db) lo.v[db] = Tile::tr_lane_off(lane, 16 * db);

  Frag<T> qf[2][D / 32];
  int qi[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    qi[qb] = q0 + 16 * qb + l16;
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
      if (qi[qb] < S)
        qf[qb][c] = lds_frag_row<T>(qp + (int64_t)qi[qb] * a.qss + 32 * c + 8 * g);
      else
        qf[qb][c].w[0] = make_uint4(0, 0, 0, 0);
    }
  }
  const float c2 = a.scale * kLog2e;
  float m_run[2] = {-__builtin_huge_valf(), -__builtin_huge_valf()};
  float l_run[2] = {0.f, 0.f};
  f32x4 acc[D / 16][2];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) acc[db][0] = acc[db][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bool active = q0 < S;
  const int q_last = min(q0 + kQW, S) - 1;
  const int w_lo = max(0, q0 - W + 1);
  const int wg_lo = active ? glob_prefix(q0, W, rpb) : 0;
  const int wg_hi = active ? glob_prefix(q_last, W, rpb) : 0;
  const int glen[2] = {glob_prefix(qi[0], W, rpb), glob_prefix(qi[1], W, rpb)};

  const Frag<T> one = ones_frag<T>();
  // Local and global tiles share one body (parameters chosen per tile); the
  // loop is unrolled over the two stages.
  auto step = [&](auto stage_c, int it) {
    constexpr int kStage = decltype(stage_c)::value;
    char(&cur)[2][Tile::kBytes] = kStage ? stage1 : stage0;
    char(&nxt)[2][Tile::kBytes] = kStage ? stage0 : stage1;
    wait_vmem();
    __syncthreads();
    if (it + 1 < ntot) issue(it + 1, nxt[0]);
    const char* tK = cur[0];
    const char* tV = cur[1];
    const bool loc = it >= nglob;
    const int ts = loc ? lo_k + (nloc - 1 - (it - nglob)) * kBN : it * kBN;
    const bool work = active && (loc ? (ts <= q_last && ts + kBN - 1 >= w_lo) : ts < wg_hi);
    const bool full = loc ? (ts >= q_last - W + 1 && ts + kBN - 1 <= q0) : ts + kBN <= wg_lo;
    TileMask<2> mk;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      mk.hi[qb] = loc ? qi[qb] - ts : glen[qb] - 1 - ts;
      mk.span[qb] = loc ? (unsigned)(W - 1) : 0x7fffffffu;
    }
    if (work) {
      // keys of the tile visible to some query of the wave: [vis_lo, vis_hi]
      const int vis_lo = loc ? w_lo - ts : 0;
      const int vis_hi = loc ? q_last - ts : wg_hi - 1 - ts;
      const bool half0 = vis_lo <= 31, half1 = vis_hi >= 32;
      if (full)
        attend_tile2<T, D, BN, false>(tK, tV, lo, qf, acc, m_run, l_run, c2, g, mk, one);
      else if (half0 && half1)
        attend_tile2<T, D, BN, true>(tK, tV, lo, qf, acc, m_run, l_run, c2, g, mk, one);
      else
        attend_half<T, D, BN>(tK, tV, half0 ? 0 : 1, lo, qf, acc, m_run, l_run, c2, g, mk, one);
    }
  };
  for (int it = 0; it < ntot; it += 2) {
    step(std::integral_constant<int, 0>{}, it);
    if (it + 1 < ntot) step(std::integral_constant<int, 1>{}, it + 1);
  }

  T* op = static_cast<T*>(a.o) + b * a.osb + h * a.osh + (int64_t)dc.off * a.oss;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float l = l_run[qb];  // each lane holds its query's whole sum
    if (!active || qi[qb] >= S) continue;
    // O is rounded to the 2-byte type: the reciprocal's 1-ulp error is invisible
    const float inv = __builtin_amdgcn_rcpf(fmaxf(l, 1e-6f));
    T* orow = op + (int64_t)qi[qb] * a.oss;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      T e[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) e[r] = from_f32<T>(acc[db][qb][r] * inv);
      *reinterpret_cast<uint2*>(orow + 16 * db + 4 * g) = *reinterpret_cast<const uint2*>(e);
    }
    if (g == 0)
      lse[qi[qb]] = (m_run[qb] + __builtin_amdgcn_logf(fmaxf(l, 1e-6f))) * kLn2;
  }
}

// Two pipeline stages as separate LDS objects, each selected at compile
// time: the compiler can then tell the fill of one stage from reads of the
// other and does not wait for the fill before those reads.
template <typename T, int D, int NW, int PH>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(D == 128 ? 2 : 3)))
void fwd2_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(1024))) FwdStage<D> stage0;
  __shared__ __attribute__((aligned(1024))) FwdStage<D> stage1;
  int item = (int)blockIdx.x;
  if (a.xcd_nt > 0) {
    item = xcd_item(item, a.B * a.Hq, a.xcd_nt);
    if (item < 0) return;  // padding block
  }
  fwd2_item<T, D, NW, PH>(a, item, stage0, stage1);
}

// Persistent form (use_persistent; the reference's work-queue kernel,
// core.py:711-900): a grid of at most one round of resident workgroups, each
// taking items in order (heaviest first) from a counter in device memory
// that the caller zeroes, until none is left. Every workgroup ends once the
// counter passes the item count.
template <typename T, int D, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(D == 128 ? 2 : 3)))
void fwd2_persistent_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(1024))) FwdStage<D> stage0;
  __shared__ __attribute__((aligned(1024))) FwdStage<D> stage1;
  __shared__ int next_item;
  const int n_items = a.docs.item0[a.docs.n] * a.B * a.Hq;
  for (;;) {
    if (threadIdx.x == 0) next_item = atomicAdd(a.work_counter, 1);
    __syncthreads();  // also: every wave is done with the previous item's LDS tiles
    const int item = next_item;
    __syncthreads();  // read before the next overwrite
    if (item >= n_items) break;
    fwd2_item<T, D, NW, 3>(a, item, stage0, stage1);
  }
}

// Resident workgroups of `kern` on the current device (CUs x workgroups per
// CU), looked up once per device and instantiation: the persistent launch
// serves small problems, where per-call host queries would cost more than
// the kernel.
template <typename T, int D, typename K>
hipError_t resident_slots(K kern, int threads, int* out) {
  constexpr int kMaxDev = 64;
  static std::mutex mu;
  static int cache[kMaxDev] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDev) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!cache[dev]) {
    int per_cu = 0, cus = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, 0);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    cache[dev] = std::max(1, per_cu) * std::max(1, cus);
  }
  *out = cache[dev];
  return hipSuccess;
}

// Waves per forward workgroup (32 queries each) for 2-byte types. 8 waves
// (256 queries sharing each K/V tile) halve the tile loads per query but
// measured 4% slower at D = 128: the wider local window adds key tiles.
constexpr int kFwdWaves = 4;

// Head dim 256, every dtype: the generic forward with 16 queries per wave
// (64 per workgroup). A persistent request runs the same tiled kernel (the
// work-queue form is built for the gfx950-tiled kernel only; the results
// are the same function of the inputs).
template <typename T>
hipError_t launch_wide(const FwdArgs& a, hipStream_t st) {
  using Tr = FwdTraits<T, 256, 1>;
  FwdArgs b = a;
  set_items(b.docs, [&](int d) { return (b.docs.len[d] + Tr::kBM - 1) / Tr::kBM; });
  const dim3 grid(b.docs.item0[b.docs.n] * b.B * b.Hq);
  hipLaunchKernelGGL((fwd_kernel<T, 256, 1>), grid, dim3(Tr::kThreads), 0, st, b);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_T(int D, const FwdArgs& a, hipStream_t st) {
  if (D == 256) return launch_wide<T>(a, st);
  if constexpr (sizeof(T) == 2) {
    FwdArgs b = a;
    constexpr int kBM = 32 * kFwdWaves;
    set_items(b.docs, [&](int d) { return (b.docs.len[d] + kBM - 1) / kBM; });
    const dim3 grid(b.docs.item0[b.docs.n] * b.B * b.Hq), block(64 * kFwdWaves);
    // one document, D = 128 and a head count that is not a multiple of 8:
    // XCD-aware order (measured 2.5-5% faster at D = 128; at D = 64, with
    // 45% less HBM traffic, 0.5% faster to 3.6% slower)
    const bool xcd = b.docs.n == 1 && (b.B * b.Hq) % 8 != 0 && D == 128;
    FwdArgs bx = b;
    bx.xcd_nt = xcd ? b.docs.item0[1] : 0;
    const dim3 xgrid(xcd ? xcd_grid(b.B * b.Hq, b.docs.item0[1]) : grid.x);
    hipError_t qerr = hipSuccess;
    auto go = [&](auto dc) {
      constexpr int Dc = decltype(dc)::value;
      if (a.work_counter && a.phases == 3) {
        // one round of resident workgroups: CUs x workgroups per CU
        auto kern = fwd2_persistent_kernel<T, Dc, kFwdWaves>;
        int slots = 0;
        qerr = resident_slots<T, Dc>(kern, 64 * kFwdWaves, &slots);
        if (qerr != hipSuccess) return;
        const int items = (int)grid.x;
        const dim3 pgrid(std::max(1, std::min(items, slots)));
        hipLaunchKernelGGL(kern, pgrid, block, 0, st, b);
        return;
      }
      switch (a.phases) {
        case 1: hipLaunchKernelGGL((fwd2_kernel<T, Dc, kFwdWaves, 1>), xgrid, block, 0, st, bx); break;
        case 2: hipLaunchKernelGGL((fwd2_kernel<T, Dc, kFwdWaves, 2>), xgrid, block, 0, st, bx); break;
        default: hipLaunchKernelGGL((fwd2_kernel<T, Dc, kFwdWaves, 3>), xgrid, block, 0, st, bx);
      }
    };
    switch (D) {
      case 32: go(std::integral_constant<int, 32>{}); break;
      case 64: go(std::integral_constant<int, 64>{}); break;
      case 128: go(std::integral_constant<int, 128>{}); break;
      default: return hipErrorInvalidValue;
    }
    if (qerr != hipSuccess) return qerr;
  } else {
    FwdArgs b = a;
    constexpr int kBM = FwdTraits<T, 128, 2>::kBM;
    set_items(b.docs, [&](int d) { return (b.docs.len[d] + kBM - 1) / kBM; });
    const dim3 grid(b.docs.item0[b.docs.n] * b.B * b.Hq);
    switch (D) {
      case 32: hipLaunchKernelGGL((fwd_kernel<T, 32, 2>), grid, dim3(256), 0, st, b); break;
      case 64: hipLaunchKernelGGL((fwd_kernel<T, 64, 2>), grid, dim3(256), 0, st, b); break;
      case 128: hipLaunchKernelGGL((fwd_kernel<T, 128, 2>), grid, dim3(256), 0, st, b); break;
      default: return hipErrorInvalidValue;
    }
  }
  return hipGetLastError();
}

}  // namespace


bool fwd_tile_config(int dtype, int D, int out[3]) {
  if (dtype < 0 || dtype > 2 || (D != 32 && D != 64 && D != 128 && D != 256)) return false;
  if (D == 256) {
    using Tr = FwdTraits<f16, 256, 1>;  // the same geometry for every dtype
    out[0] = Tr::kWaves; out[1] = Tr::kBM; out[2] = Tr::kBN;
  } else if (dtype == 2) {
    using Tr = FwdTraits<float, 128>;
    out[0] = Tr::kWaves; out[1] = Tr::kBM; out[2] = Tr::kBN;
  } else {
    out[0] = kFwdWaves; out[1] = 32 * kFwdWaves; out[2] = 64;
  }
  return true;
}

hipError_t launch_fwd(int dtype, int D, const FwdArgs& a, hipStream_t st) {
  switch (dtype) {
    case 0: return launch_T<f16>(D, a, st);
    case 1: return launch_T<bf16>(D, a, st);
    case 2: return launch_T<float>(D, a, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace cra

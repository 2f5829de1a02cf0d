// Backward of the three-phase sqrt(N) attention.
//
// Reference: `CronRootAttentionV14Function.backward` (core.py:3626-3759) runs
// dQ (core.py:1165-1316), local dK/dV (core.py:1650-1745), strided dK/dV with
// fp16 atomics (core.py:1755-1889), relay dK/dV (core.py:2381-2492) and a
// read-add-store scatter of the relay gradients onto their source rows
// (core.py:2767-2815). Math per pair (i, j): P = exp(s - LSE_i),
// dP = dO_i . v_j, dS = P (dP - Delta_i), Delta_i = O_i . dO_i;
// dQ_i += scale dS k_j, dK_j += scale dS q_i, dV_j += P dO_i.
//
// This build keeps every accumulation in fp32 and rounds once:
//   1. delta_kernel      Delta = rowsum(O * dO)  (fp32 inputs; for fp16/bf16
//                        dq2_kernel computes Delta of its queries and stores
//                        -Delta and -lse * log2(e) for the dK/dV kernels)
//   2. dq_kernel         query-centric: local band + global prefix -> dQ
//   3. dkdv_kernel<GLOB> packed global rows (strided + relay), query range
//                        split in chunks -> fp32 partials in the workspace
//   3b. gsum_kernel      sums the chunk partials of each global row
//   4. dalpha_kernel     (optional) gradient of the relay log-scale
//   5. dkdv_kernel<LOC>  key-centric local band; its epilogue adds the
//                        summed partials of the global rows whose source is
//                        the key row (strided row r*W, relay source rows) and
//                        writes dK/dV once.
// No atomics: every output row has exactly one writer and the partial sums
// are reduced in a fixed order, so two runs give identical bits.
#include <type_traits>

#include "cra_common.hpp"
#include "cra_internal.hpp"

namespace cra {

namespace {

// Geometry of the generic (non-gfx950-tiled) kernels: the fp32 path, and
// every dtype at head dim 256. NB = 16-row blocks per wave (queries for dQ,
// keys for dK/dV): two below D = 256; one at D = 256, where two would hold
// 256 VGPRs of accumulators and operands per wave.
template <typename T, int D, int NB = 2>
struct BwdTraits {
  static constexpr int kThreads = 256;
  static constexpr bool kSmallTiles = sizeof(T) == 4 || D > 128;
  static constexpr int kQW = 16 * NB;                   // dq: queries per wave
  static constexpr int kBM = 4 * kQW;                   // dq: queries per workgroup
  static constexpr int kBN = kSmallTiles ? 32 : 64;     // dq: key rows per tile
  static constexpr int kKW = 16 * NB;                   // dkdv: key rows per wave
  static constexpr int kBK = 4 * kKW;                   // dkdv: key rows per workgroup
  static constexpr int kBQ = kSmallTiles ? 32 : 64;     // dkdv: queries per tile
  static constexpr int kDC = D / 32;
  static constexpr int kDB = D / 16;
  static constexpr int kLD = D + 16 / (int)sizeof(T);
  static constexpr int kLDTN = kBN + 4;
  static constexpr int kLDTQ = kBQ + 4;
};

template <typename T>
__device__ __forceinline__ void zero_frag(Frag<T>& f) {
#pragma unroll
  for (int w = 0; w < Frag<T>::kWords; ++w) f.w[w] = make_uint4(0, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const f32x4& v, float mul) {
  T e[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) e[r] = from_f32<T>(v[r] * mul);
  if constexpr (sizeof(T) == 2)
    *reinterpret_cast<uint2*>(p) = *reinterpret_cast<const uint2*>(e);
  else
    *reinterpret_cast<uint4*>(p) = *reinterpret_cast<const uint4*>(e);
}

// First query that sees packed global row gr (inverse of glob_prefix).
__device__ __forceinline__ int glob_row_first_query(int gr, int W, int rpb) {
  const int r = gr / rpb;
  return (gr - r * rpb) == 0 ? r * W + W : (r + 1) * W + W - 1;
}

// ---------------------------------------------------------------------------
// 1. Delta = rowsum(O * dO)
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void delta_kernel(BwdArgs a) {
  constexpr int kLPR = D / 8;
  constexpr int kRows = 256 / kLPR;
  const int bh = blockIdx.y;
  const int b = bh / a.Hq, h = bh % a.Hq;
  const int tid = threadIdx.x;
  const int li = tid % kLPR;
  const int row = blockIdx.x * kRows + tid / kLPR;
  float acc = 0.f;
  if (row < a.S) {
    const Frag<T> o = lds_frag_row<T>(static_cast<const T*>(a.o) + b * a.osb + h * a.osh +
                                      (int64_t)row * a.oss + li * 8);
    const Frag<T> d = lds_frag_row<T>(static_cast<const T*>(a.dout) + b * a.dosb + h * a.dosh +
                                      (int64_t)row * a.doss + li * 8);
    const T* eo = reinterpret_cast<const T*>(o.w);
    const T* ed = reinterpret_cast<const T*>(d.w);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += to_f32(eo[i]) * to_f32(ed[i]);
  }
#pragma unroll
  for (int off = kLPR / 2; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
  if (row < a.S && li == 0) a.delta[(int64_t)bh * a.S + row] = acc;
}

// ---------------------------------------------------------------------------
// 2. dQ, query-centric (mirror of the forward's tiling)
// ---------------------------------------------------------------------------
template <typename T, int D, int NB, bool MASK, typename Valid>
__device__ __forceinline__ void dq_tile(const T* sK, const T* sV, const T* sKt,
                                        const Frag<T> (&qf)[NB][BwdTraits<T, D, NB>::kDC],
                                        const Frag<T> (&df)[NB][BwdTraits<T, D, NB>::kDC],
                                        f32x4 (&dqa)[BwdTraits<T, D, NB>::kDB][NB],
                                        const float (&lse2)[NB], const float (&dl)[NB], float c2,
                                        int l16, int g, Valid valid) {
  using Tr = BwdTraits<T, D, NB>;
  constexpr int kKB = Tr::kBN / 16, kKC = Tr::kBN / 32;
  Frag<T> dsf[kKC][NB];
  float ds[kKB][NB][4];
#pragma unroll
  for (int kb = 0; kb < kKB; ++kb) {
    f32x4 sc[NB], dp[NB];
#pragma unroll
    for (int qb = 0; qb < NB; ++qb) sc[qb] = dp[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < Tr::kDC; ++c) {
      const Frag<T> kf = lds_frag_row<T>(sK + (16 * kb + l16) * Tr::kLD + 32 * c + 8 * g);
      const Frag<T> vf = lds_frag_row<T>(sV + (16 * kb + l16) * Tr::kLD + 32 * c + 8 * g);
#pragma unroll
      for (int qb = 0; qb < NB; ++qb) sc[qb] = mma(sc[qb], kf, qf[qb][c]);
#pragma unroll
      for (int qb = 0; qb < NB; ++qb) dp[qb] = mma(dp[qb], vf, df[qb][c]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ko = 16 * kb + 4 * g + r;
#pragma unroll
      for (int qb = 0; qb < NB; ++qb) {
        float x = sc[qb][r] * c2 - lse2[qb];
        if (MASK && !valid(ko, qb)) x = -__builtin_huge_valf();
        ds[kb][qb][r] = __builtin_amdgcn_exp2f(x) * (dp[qb][r] - dl[qb]);
      }
    }
  }
#pragma unroll
  for (int kc = 0; kc < kKC; ++kc) {
#pragma unroll
    for (int qb = 0; qb < NB; ++qb) {
      const float v8[8] = {ds[2 * kc][qb][0],     ds[2 * kc][qb][1],     ds[2 * kc][qb][2],
                           ds[2 * kc][qb][3],     ds[2 * kc + 1][qb][0], ds[2 * kc + 1][qb][1],
                           ds[2 * kc + 1][qb][2], ds[2 * kc + 1][qb][3]};
      dsf[kc][qb] = pack8<T>(v8);
    }
  }
#pragma unroll
  for (int db = 0; db < Tr::kDB; ++db) {
    const T* row = sKt + (16 * db + l16) * Tr::kLDTN;
#pragma unroll
    for (int kc = 0; kc < kKC; ++kc) {
      const Frag<T> kt = lds_frag_2x4<T>(row + 32 * kc + 4 * g, row + 32 * kc + 16 + 4 * g);
#pragma unroll
      for (int qb = 0; qb < NB; ++qb) dqa[db][qb] = mma(dqa[db][qb], kt, dsf[kc][qb]);
    }
  }
}

template <typename T, int D, int NB>
__global__ __launch_bounds__(256) void dq_kernel(BwdArgs a) {
  using Tr = BwdTraits<T, D, NB>;
  __shared__ __attribute__((aligned(16))) T sK[Tr::kBN * Tr::kLD];
  __shared__ __attribute__((aligned(16))) T sV[Tr::kBN * Tr::kLD];
  __shared__ __attribute__((aligned(16))) T sKt[D * Tr::kLDTN];

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
  const T* dop =
      static_cast<const T*>(a.dout) + b * a.dosb + h * a.dosh + (int64_t)dc.off * a.doss;
  const T* kp = static_cast<const T*>(a.k) + b * a.ksb + hk * a.ksh + (int64_t)dc.off * a.kss;
  const T* vp = static_cast<const T*>(a.v) + b * a.vsb + hk * a.vsh + (int64_t)dc.off * a.vss;
  const float* lse = a.lse + (int64_t)bh * a.S + dc.off;
  const float* delta = a.delta + (int64_t)bh * a.S + dc.off;
  const int64_t gbase = ((int64_t)(b * a.Hkv + hk) * a.G + dc.gofs) * D;
  const T* gkp = static_cast<const T*>(a.gk) + gbase;
  const T* gvp = static_cast<const T*>(a.gv) + gbase;

  Frag<T> qf[NB][Tr::kDC], df[NB][Tr::kDC];
  int qi[NB];
  float lse2[NB], dl[NB];
#pragma unroll
  for (int qb = 0; qb < NB; ++qb) {
    qi[qb] = q0 + 16 * qb + l16;
    const bool ok = qi[qb] < S;
    lse2[qb] = ok ? lse[qi[qb]] * kLog2e : 0.f;
    dl[qb] = ok ? delta[qi[qb]] : 0.f;
#pragma unroll
    for (int c = 0; c < Tr::kDC; ++c) {
      if (ok) {
        qf[qb][c] = lds_frag_row<T>(qp + (int64_t)qi[qb] * a.qss + 32 * c + 8 * g);
        df[qb][c] = lds_frag_row<T>(dop + (int64_t)qi[qb] * a.doss + 32 * c + 8 * g);
      } else {
        zero_frag(qf[qb][c]);
        zero_frag(df[qb][c]);
      }
    }
  }
  const float c2 = a.scale * kLog2e;
  f32x4 dqa[Tr::kDB][NB];
#pragma unroll
  for (int db = 0; db < Tr::kDB; ++db)
#pragma unroll
    for (int qb = 0; qb < NB; ++qb) dqa[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bool active = q0 < S;
  const int q_last = min(q0 + Tr::kQW, S) - 1;
  TileStage<T, D, Tr::kBN, Tr::kThreads> stk, stv;

  const int lo = max(0, m0 - W + 1);
  const int hi = min(S, m0 + Tr::kBM);
  const int w_lo = max(0, q0 - W + 1);
  for (int ts = lo; ts < hi; ts += Tr::kBN) {
    stk.load(kp, a.kss, ts, 0, hi, tid);
    stv.load(vp, a.vss, ts, 0, hi, tid);
    __syncthreads();
    stk.template store_rows<Tr::kLD>(sK, tid);
    stk.template store_cols<Tr::kLDTN>(sKt, tid);
    stv.template store_rows<Tr::kLD>(sV, tid);
    __syncthreads();
    if (active && ts <= q_last && ts + Tr::kBN - 1 >= w_lo) {
      const bool full = ts >= q_last - W + 1 && ts + Tr::kBN - 1 <= q0;
      auto valid = [&](int ko, int qb) {
        const int j = ts + ko;
        return j <= qi[qb] && j >= qi[qb] - W + 1;
      };
      if (full)
        dq_tile<T, D, NB, false>(sK, sV, sKt, qf, df, dqa, lse2, dl, c2, l16, g, valid);
      else
        dq_tile<T, D, NB, true>(sK, sV, sKt, qf, df, dqa, lse2, dl, c2, l16, g, valid);
    }
  }

  const int gmax = glob_prefix(hi - 1, W, rpb);
  const int wg_lo = active ? glob_prefix(q0, W, rpb) : 0;
  const int wg_hi = active ? glob_prefix(q_last, W, rpb) : 0;
  int glen[NB];
#pragma unroll
  for (int qb = 0; qb < NB; ++qb) glen[qb] = glob_prefix(qi[qb], W, rpb);
  for (int ts = 0; ts < gmax; ts += Tr::kBN) {
    stk.load(gkp, D, ts, 0, gmax, tid);
    stv.load(gvp, D, ts, 0, gmax, tid);
    __syncthreads();
    stk.template store_rows<Tr::kLD>(sK, tid);
    stk.template store_cols<Tr::kLDTN>(sKt, tid);
    stv.template store_rows<Tr::kLD>(sV, tid);
    __syncthreads();
    if (active && ts < wg_hi) {
      auto valid = [&](int ko, int qb) { return ts + ko < glen[qb]; };
      if (ts + Tr::kBN <= wg_lo)
        dq_tile<T, D, NB, false>(sK, sV, sKt, qf, df, dqa, lse2, dl, c2, l16, g, valid);
      else
        dq_tile<T, D, NB, true>(sK, sV, sKt, qf, df, dqa, lse2, dl, c2, l16, g, valid);
    }
  }

  T* dqp = static_cast<T*>(a.dq) + b * a.dqsb + h * a.dqsh + (int64_t)dc.off * a.dqss;
#pragma unroll
  for (int qb = 0; qb < NB; ++qb) {
    if (!active || qi[qb] >= S) continue;
    T* row = dqp + (int64_t)qi[qb] * a.dqss;
#pragma unroll
    for (int db = 0; db < Tr::kDB; ++db) store4<T>(row + 16 * db + 4 * g, dqa[db][qb], a.scale);
  }
}

// ---------------------------------------------------------------------------
// 3/5. dK, dV, key-centric. GLOB: the keys are packed global rows and the
// result is an fp32 partial per query chunk; LOC: the keys are rows of k/v,
// the queries their local band, and the epilogue folds in the global rows.
// ---------------------------------------------------------------------------
template <typename T, int D, int NB, bool GLOB, bool MASK>
__device__ __forceinline__ void dkdv_tile(const T* sQ, const T* sO, const T* sQt, const T* sOt,
                                          const float* sL, const float* sDl, const int* sGl,
                                          const Frag<T> (&kf)[NB][BwdTraits<T, D, NB>::kDC],
                                          const Frag<T> (&vf)[NB][BwdTraits<T, D, NB>::kDC],
                                          f32x4 (&dka)[BwdTraits<T, D, NB>::kDB][NB],
                                          f32x4 (&dva)[BwdTraits<T, D, NB>::kDB][NB], float c2,
                                          int l16, int g, int ts, int kw, int W, int q_hi) {
  using Tr = BwdTraits<T, D, NB>;
  constexpr int kQS = Tr::kBQ / 32;  // 32-query steps per tile
#pragma unroll
  for (int qs = 0; qs < kQS; ++qs) {
    float p[2][NB][4], ds[2][NB][4];  // [query block][key block][r]
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int qo = 32 * qs + 16 * qb;
      f32x4 sc[NB], dd[NB];
#pragma unroll
      for (int kb = 0; kb < NB; ++kb) sc[kb] = dd[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < Tr::kDC; ++c) {
        const Frag<T> qa = lds_frag_row<T>(sQ + (qo + l16) * Tr::kLD + 32 * c + 8 * g);
        const Frag<T> oa = lds_frag_row<T>(sO + (qo + l16) * Tr::kLD + 32 * c + 8 * g);
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) sc[kb] = mma(sc[kb], qa, kf[kb][c]);
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) dd[kb] = mma(dd[kb], oa, vf[kb][c]);
      }
      const f32x4 lq = *reinterpret_cast<const f32x4*>(sL + qo + 4 * g);
      const f32x4 dq = *reinterpret_cast<const f32x4*>(sDl + qo + 4 * g);
      int gq[4] = {0, 0, 0, 0};
      if (GLOB && MASK) {
        const int4 t4 = *reinterpret_cast<const int4*>(sGl + qo + 4 * g);
        gq[0] = t4.x; gq[1] = t4.y; gq[2] = t4.z; gq[3] = t4.w;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int qabs = ts + qo + 4 * g + r;
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
          float x = sc[kb][r] * c2 - lq[r];
          if (MASK) {
            const int j = kw + 16 * kb + l16;
            const bool vis = GLOB ? (qabs < q_hi && j < gq[r])
                                  : (qabs < q_hi && j <= qabs && j >= qabs - W + 1);
            if (!vis) x = -__builtin_huge_valf();
          }
          p[qb][kb][r] = __builtin_amdgcn_exp2f(x);
          ds[qb][kb][r] = p[qb][kb][r] * (dd[kb][r] - dq[r]);
        }
      }
    }
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) {
      const float pv[8] = {p[0][kb][0], p[0][kb][1], p[0][kb][2], p[0][kb][3],
                           p[1][kb][0], p[1][kb][1], p[1][kb][2], p[1][kb][3]};
      const float dv8[8] = {ds[0][kb][0], ds[0][kb][1], ds[0][kb][2], ds[0][kb][3],
                            ds[1][kb][0], ds[1][kb][1], ds[1][kb][2], ds[1][kb][3]};
      const Frag<T> pf = pack8<T>(pv);
      const Frag<T> sf = pack8<T>(dv8);
#pragma unroll
      for (int db = 0; db < Tr::kDB; ++db) {
        const T* orow = sOt + (16 * db + l16) * Tr::kLDTQ + 32 * qs;
        const T* qrow = sQt + (16 * db + l16) * Tr::kLDTQ + 32 * qs;
        const Frag<T> ot = lds_frag_2x4<T>(orow + 4 * g, orow + 16 + 4 * g);
        const Frag<T> qt = lds_frag_2x4<T>(qrow + 4 * g, qrow + 16 + 4 * g);
        dva[db][kb] = mma(dva[db][kb], ot, pf);
        dka[db][kb] = mma(dka[db][kb], qt, sf);
      }
    }
  }
}

template <typename T, int D, int NB, bool GLOB>
__global__ __launch_bounds__(256) void dkdv_kernel(BwdArgs a) {
  using Tr = BwdTraits<T, D, NB>;
  __shared__ __attribute__((aligned(16))) T sQ[Tr::kBQ * Tr::kLD];
  __shared__ __attribute__((aligned(16))) T sO[Tr::kBQ * Tr::kLD];
  __shared__ __attribute__((aligned(16))) T sQt[D * Tr::kLDTQ];
  __shared__ __attribute__((aligned(16))) T sOt[D * Tr::kLDTQ];
  __shared__ __attribute__((aligned(16))) float sL[Tr::kBQ];
  __shared__ __attribute__((aligned(16))) float sDl[Tr::kBQ];
  __shared__ __attribute__((aligned(16))) int sGl[Tr::kBQ];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int nbh = a.B * a.Hkv;
  const int bhk = blockIdx.x % nbh;
  const int rest = blockIdx.x / nbh;
  const Doc dc = find_doc(a.docs, rest);
  const int chunk = GLOB ? dc.item % a.nchunk : 0;
  const int tile = GLOB ? dc.item / a.nchunk : dc.item;
  const int b = bhk / a.Hkv, hk = bhk % a.Hkv;
  const int grp = a.Hq / a.Hkv;
  const int S = dc.len, W = dc.W, rpb = dc.rpb;
  const bool relay = rpb > 1;
  const int nrows = GLOB ? (S + W - 1) / W * rpb : S;  // keys: global rows or rows
  const int k0 = tile * Tr::kBK;
  const int kw = k0 + wave * Tr::kKW;

  const T* kbase;
  const T* vbase;
  int64_t kstride, vstride;
  if (GLOB) {
    const int64_t gb = ((int64_t)bhk * a.G + dc.gofs) * D;
    kbase = static_cast<const T*>(a.gk) + gb;
    vbase = static_cast<const T*>(a.gv) + gb;
    kstride = D;
    vstride = D;
  } else {
    kbase = static_cast<const T*>(a.k) + b * a.ksb + hk * a.ksh + (int64_t)dc.off * a.kss;
    vbase = static_cast<const T*>(a.v) + b * a.vsb + hk * a.vsh + (int64_t)dc.off * a.vss;
    kstride = a.kss;
    vstride = a.vss;
  }

  // K^T, V^T as B operands: lane holds row kw + 16kb + l16, dims 32c + 8g ..
  Frag<T> kf[NB][Tr::kDC], vf[NB][Tr::kDC];
#pragma unroll
  for (int kb = 0; kb < NB; ++kb) {
    const int row = kw + 16 * kb + l16;
#pragma unroll
    for (int c = 0; c < Tr::kDC; ++c) {
      if (row < nrows) {
        kf[kb][c] = lds_frag_row<T>(kbase + (int64_t)row * kstride + 32 * c + 8 * g);
        vf[kb][c] = lds_frag_row<T>(vbase + (int64_t)row * vstride + 32 * c + 8 * g);
      } else {
        zero_frag(kf[kb][c]);
        zero_frag(vf[kb][c]);
      }
    }
  }
  f32x4 dka[Tr::kDB][NB], dva[Tr::kDB][NB];
#pragma unroll
  for (int db = 0; db < Tr::kDB; ++db)
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) dka[db][kb] = dva[db][kb] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Query range of the workgroup and of this wave.
  const bool active = kw < nrows;
  int q_lo, q_hi, wq_lo, wq_hi;
  if (GLOB) {
    const int chunk_len = chunk_len_for(S, a.nchunk);
    const int c_lo = chunk * chunk_len;
    const int c_hi = min(S, c_lo + chunk_len);
    q_lo = max(c_lo, glob_row_first_query(k0, W, rpb));
    q_hi = c_hi;
    wq_lo = active ? max(c_lo, glob_row_first_query(kw, W, rpb)) : S;
    wq_hi = c_hi;
    // no query of this chunk sees the tile's rows: gsum_kernel skips the
    // chunk for them (with a single chunk the zeros are written instead)
    if (q_hi <= q_lo && a.nchunk > 1) return;
  } else {
    q_lo = k0;
    q_hi = min(S, k0 + Tr::kBK - 1 + W);
    wq_lo = kw;
    wq_hi = min(S, kw + Tr::kKW - 1 + W);
  }
  const int k_last = min(kw + Tr::kKW, nrows) - 1;
  const float c2 = a.scale * kLog2e;
  TileStage<T, D, Tr::kBQ, Tr::kThreads> stq, sto;

  for (int j = 0; j < grp; ++j) {
    const int h = hk * grp + j;
    const int bh = b * a.Hq + h;
    const T* qp = static_cast<const T*>(a.q) + b * a.qsb + h * a.qsh + (int64_t)dc.off * a.qss;
    const T* dop =
        static_cast<const T*>(a.dout) + b * a.dosb + h * a.dosh + (int64_t)dc.off * a.doss;
    const float* lse = a.lse + (int64_t)bh * a.S + dc.off;
    const float* delta = a.delta + (int64_t)bh * a.S + dc.off;
    for (int ts = q_lo; ts < q_hi; ts += Tr::kBQ) {
      stq.load(qp, a.qss, ts, 0, q_hi, tid);
      sto.load(dop, a.doss, ts, 0, q_hi, tid);
      __syncthreads();
      stq.template store_rows<Tr::kLD>(sQ, tid);
      stq.template store_cols<Tr::kLDTQ>(sQt, tid);
      sto.template store_rows<Tr::kLD>(sO, tid);
      sto.template store_cols<Tr::kLDTQ>(sOt, tid);
      if (tid < Tr::kBQ) {
        const int qabs = ts + tid;
        const bool ok = qabs < q_hi;
        sL[tid] = ok ? lse[qabs] * kLog2e : 0.f;
        sDl[tid] = ok ? delta[qabs] : 0.f;
        if (GLOB) sGl[tid] = ok ? glob_prefix(qabs, W, rpb) : 0;
      }
      __syncthreads();
      const int t_last = min(ts + Tr::kBQ, q_hi) - 1;
      if (active && t_last >= wq_lo && ts < wq_hi) {
        bool full;
        if (GLOB)
          full = ts + Tr::kBQ <= q_hi && glob_prefix(ts, W, rpb) > k_last;
        else
          full = ts >= k_last && ts + Tr::kBQ - 1 - W + 1 <= kw && ts + Tr::kBQ <= q_hi;
        if (full)
          dkdv_tile<T, D, NB, GLOB, false>(sQ, sO, sQt, sOt, sL, sDl, sGl, kf, vf, dka, dva, c2,
                                           l16, g, ts, kw, W, q_hi);
        else
          dkdv_tile<T, D, NB, GLOB, true>(sQ, sO, sQt, sOt, sL, sDl, sGl, kf, vf, dka, dva, c2,
                                          l16, g, ts, kw, W, q_hi);
      }
    }
  }

  // Epilogue. Lane owns key row kw + 16kb + l16, dims 16db + 4g .. +4.
  if (GLOB) {
    float* part = a.gpart + (((int64_t)chunk * nbh + bhk) * a.G + dc.gofs) * 2 * D;
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) {
      const int row = kw + 16 * kb + l16;
      if (row >= nrows) continue;
      float* pk = part + (int64_t)row * 2 * D;
#pragma unroll
      for (int db = 0; db < Tr::kDB; ++db) {
        *reinterpret_cast<f32x4*>(pk + 16 * db + 4 * g) = dka[db][kb] * a.scale;
        *reinterpret_cast<f32x4*>(pk + D + 16 * db + 4 * g) = dva[db][kb];
      }
    }
    return;
  }
  T* dkp = static_cast<T*>(a.dk) + b * a.dksb + hk * a.dksh + (int64_t)dc.off * a.dkss;
  T* dvp = static_cast<T*>(a.dv) + b * a.dvsb + hk * a.dvsh + (int64_t)dc.off * a.dvss;
  const float rsc = (relay && a.rscale) ? a.rscale[hk] : 1.f;
#pragma unroll
  for (int kb = 0; kb < NB; ++kb) {
    const int j = kw + 16 * kb + l16;
    if (j >= S) continue;
#pragma unroll
    for (int db = 0; db < Tr::kDB; ++db) dka[db][kb] *= a.scale;
    // Global rows whose source is row j: the strided row of its block and
    // any relay row selected from it (reference scatter, core.py:2767-2815).
    const int rblk = j / W;
    int grow[5];
    float gsc[5];
    int nm = 0;
    if (j == rblk * W) {
      grow[nm] = rblk * rpb;
      gsc[nm++] = 1.f;
    }
    if (relay) {
      const int32_t* src = a.src + ((int64_t)bhk * a.NB + dc.bofs + rblk) * a.top_k;
      for (int t = 0; t < a.top_k; ++t) {
        if (src[t] == j) {
          grow[nm] = rblk * rpb + 1 + t;
          gsc[nm++] = rsc;
        }
      }
    }
    // the chunk partials of the global rows are summed into chunk 0
    for (int m = 0; m < nm; ++m) {
      const float* pk = a.gpart + ((int64_t)bhk * a.G + dc.gofs + grow[m]) * 2 * D;
#pragma unroll
      for (int db = 0; db < Tr::kDB; ++db) {
        dka[db][kb] += *reinterpret_cast<const f32x4*>(pk + 16 * db + 4 * g) * gsc[m];
        dva[db][kb] += *reinterpret_cast<const f32x4*>(pk + D + 16 * db + 4 * g) * gsc[m];
      }
    }
#pragma unroll
    for (int db = 0; db < Tr::kDB; ++db) {
      store4<T>(dkp + (int64_t)j * a.dkss + 16 * db + 4 * g, dka[db][kb], 1.f);
      store4<T>(dvp + (int64_t)j * a.dvss + 16 * db + 4 * g, dva[db][kb], 1.f);
    }
  }
}

// ---------------------------------------------------------------------------
// 3b. Chunk partials of the global rows summed into chunk 0, in chunk order
// (one float4 per thread; work items: the documents' rows x 2D / 4 / 256).
// Only chunks with a query that sees the row are read.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void gsum_kernel(BwdArgs a) {
  constexpr int kVec = 2 * D / 4;  // float4 per row (dK and dV)
  const int nbh = a.B * a.Hkv;
  const int bhk = blockIdx.x % nbh;
  const Doc dc = find_doc(a.docs, (int)(blockIdx.x / nbh));
  const int rows = (dc.len + dc.W - 1) / dc.W * dc.rpb;
  const int e = dc.item * 256 + (int)threadIdx.x;
  if (e >= rows * kVec) return;
  // Chunks [c_lo, c_hi) hold queries that see the row; the global-row
  // kernel wrote no partial for the others (their workgroups had no query
  // that sees the tile), so they are skipped rather than read.
  const int L = chunk_len_for(dc.len, a.nchunk);
  const int first = glob_row_first_query(e / kVec, dc.W, dc.rpb);
  const int c_lo = first / L;
  const int c_hi = first < dc.len ? min(a.nchunk, (dc.len + L - 1) / L) : c_lo;
  float* p0 = a.gpart + ((int64_t)bhk * a.G + dc.gofs) * 2 * D + 4 * (int64_t)e;
  const int64_t cstride = (int64_t)nbh * a.G * 2 * D;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c = c_lo; c < c_hi; ++c) acc += *reinterpret_cast<const f32x4*>(p0 + c * cstride);
  *reinterpret_cast<f32x4*>(p0) = acc;
}

// ---------------------------------------------------------------------------
// 4. d(relay_log_scale)[hk] = sum over b and relay rows of dRK.RK + dRV.RV
// (reference core.py:3363-3366), one workgroup per kv head, fixed order.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void dalpha_kernel(BwdArgs a) {
  const int hk = blockIdx.x;
  const int tid = threadIdx.x;
  const int nbh = a.B * a.Hkv;
  float acc = 0.f;
  for (int b = 0; b < a.B; ++b) {
    const int bhk = b * a.Hkv + hk;
    const T* gk = static_cast<const T*>(a.gk) + (int64_t)bhk * a.G * D;
    const T* gv = static_cast<const T*>(a.gv) + (int64_t)bhk * a.G * D;
    for (int doc = 0; doc < a.docs.n; ++doc) {
      const int rpb = a.docs.rpb[doc];
      if (rpb == 1) continue;  // no relay rows in this document
      const int nrel = (a.docs.len[doc] + a.docs.W[doc] - 1) / a.docs.W[doc] * a.top_k;
      for (int e = tid; e < nrel * D; e += 256) {
        const int t = e / D, d = e % D;
        const int row = a.docs.gofs[doc] + (t / a.top_k) * rpb + 1 + t % a.top_k;
        const float* pk = a.gpart + ((int64_t)bhk * a.G + row) * 2 * D;  // summed chunks
        const float dk = pk[d], dv = pk[D + d];
        acc += dk * to_f32(gk[(int64_t)row * D + d]) + dv * to_f32(gv[(int64_t)row * D + d]);
      }
    }
  }
  __shared__ float red[256];
  red[tid] = acc;
  __syncthreads();
  for (int off = 128; off >= 1; off >>= 1) {
    if (tid < off) red[tid] += red[tid + off];
    __syncthreads();
  }
  if (tid == 0) a.dalpha[hk] = (a.group ? a.dalpha[hk] : 0.f) + red[0];
}

// ---------------------------------------------------------------------------
// fp16/bf16 backward kernels on the gfx950 tile machinery (see SwzTile):
// K/V (dq2) or Q/dO (dkdv2) tiles of 64 rows double-buffered in swizzled LDS,
// filled by buffer loads straight into LDS while the previous tile is
// computed; transposed operands (K^T for dQ, Q^T and dO^T for dK/dV) are
// read with ds_read_b64_tr_b16 from the same row-major tiles.
// ---------------------------------------------------------------------------
template <int D>
struct LaneOffs {
  int row[D / 32];  // row fragment, chunk 4c + g, row lane%16
  int tr[D / 16];   // transposed fragment, columns 16 db ..
};

template <int D>
__device__ __forceinline__ LaneOffs<D> lane_offs(int lane) {
  using Tile = SwzTile<D, 64>;
  LaneOffs<D> o;
  const int g = lane >> 4;
#pragma unroll
  for (int c = 0; c < D / 32; ++c) o.row[c] = Tile::row_lane_off(lane, 4 * c + g);
#pragma unroll
  for (int db = 0; db < D / 16; ++db) o.tr[db] = Tile::tr_lane_off(lane, 16 * db);
  return o;
}

// Query-centric dQ for QB blocks of 16 queries per wave against one BN-key
// tile, in 32-key halves: S = K . Q^T and dP - Delta = V . dO^T - Delta (key
// on rows; the products accumulate onto -Delta, so no subtraction per
// element), dS = P * (dP - Delta), dQ^T += K^T . dS^T.
template <typename T, int D, int QB, int BN, bool MASK>
__device__ __forceinline__ void dq2_tile(const char* tK, const char* tV, const LaneOffs<D>& lo,
                                         const Frag<T> (&qf)[QB][D / 32],
                                         const Frag<T> (&df)[QB][D / 32],
                                         f32x4 (&dqa)[D / 16][QB], const float (&lse2)[QB],
                                         const float (&ndl)[QB], float c2, int g,
                                         const TileMask<QB>& mk, bool half0, bool half1) {
  using Tile = SwzTile<D, BN>;
  constexpr int NC = D / 32;
#pragma unroll
  for (int kc = 0; kc < BN / 32; ++kc) {
    // masked tiles: a 32-key half with no key visible to the wave is skipped
    if (MASK && !(kc ? half1 : half0)) continue;
    float ds[2][QB][4];  // [h][qb][r]
    // K and V row fragments are read two steps ahead of their MFMAs; fences
    // keep the compiler from moving the reads next to their uses
    constexpr int NT = 2 * NC;
    auto row_kv = [&](int t, Frag<T>& k_, Frag<T>& v_) {
      const int kn = 2 * kc + t / NC, cn = t % NC;
      k_ = Tile::template row_frag_at<T>(tK + kn * Tile::kBlk16 + lo.row[cn]);
      v_ = Tile::template row_frag_at<T>(tV + kn * Tile::kBlk16 + lo.row[cn]);
    };
    Frag<T> kf[3], vf[3];
    row_kv(0, kf[0], vf[0]);
    row_kv(1, kf[1], vf[1]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      f32x4 sc[QB], dp[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        sc[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
        dp[qb] = f32x4{ndl[qb], ndl[qb], ndl[qb], ndl[qb]};
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int t = h * NC + c;
        if (t + 2 < NT) row_kv(t + 2, kf[(t + 2) % 3], vf[(t + 2) % 3]);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          sc[qb] = mma(sc[qb], kf[t % 3], qf[qb][c]);
          dp[qb] = mma(dp[qb], vf[t % 3], df[qb][c]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      const int kb = 2 * kc + h;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ko = 16 * kb + 4 * g + r;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          float x = fmaf(sc[qb][r], c2, -lse2[qb]);
          if (MASK && !mk.ok(ko, qb)) x = -__builtin_huge_valf();
          ds[h][qb][r] = __builtin_amdgcn_exp2f(x) * dp[qb][r];
        }
      }
    }
    Frag<T> dsf[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const float v8[8] = {ds[0][qb][0], ds[0][qb][1], ds[0][qb][2], ds[0][qb][3],
                           ds[1][qb][0], ds[1][qb][1], ds[1][qb][2], ds[1][qb][3]};
      dsf[qb] = pack8<T>(v8);
    }
    // transposed K fragments, also two steps ahead
    Frag<T> kt[3];
    auto tr_k = [&](int db) {
      const char* pa = tK + (2 * kc) * Tile::kBlk16 + lo.tr[db];
      return Tile::template tr_frag_at<T>(pa, pa + Tile::kBlk16);
    };
    kt[0] = tr_k(0);
    kt[1] = tr_k(1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      if (db + 2 < D / 16) kt[(db + 2) % 3] = tr_k(db + 2);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) dqa[db][qb] = mma(dqa[db][qb], kt[db % 3], dsf[qb]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// NW waves of QB blocks of 16 queries each cover the workgroup's
// 16 * NW * QB queries; key tiles of BN rows; at least WPE waves per SIMD.
template <typename T, int D, int NW, int QB, int BN, int WPE>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WPE)))
void dq2_kernel(BwdArgs a) {
  using Tile = SwzTile<D, BN>;
  constexpr int kQW = 16 * QB, kBM = NW * kQW, kBN = BN;
  // Two pipeline stages as separate LDS objects (see fwd2_kernel).
  __shared__ __attribute__((aligned(1024))) char stage0[2][Tile::kBytes];  // K, V
  __shared__ __attribute__((aligned(1024))) char stage1[2][Tile::kBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int nbh = a.B * a.Hq;
  int item = (int)blockIdx.x;
  if (a.xcd_nt > 0) {
    item = xcd_item(item, nbh, a.xcd_nt);
    if (item < 0) return;  // padding block
  }
  const int bh = item % nbh;
  const Doc dc = find_doc(a.docs, item / nbh);
  const int tile = (dc.len + kBM - 1) / kBM - 1 - dc.item;  // heaviest first
  const int b = bh / a.Hq, h = bh % a.Hq;
  const int hk = h / (a.Hq / a.Hkv);
  const int m0 = tile * kBM;
  const int q0 = m0 + wave * kQW;
  const int S = dc.len, W = dc.W, rpb = dc.rpb;

  const T* qp = static_cast<const T*>(a.q) + b * a.qsb + h * a.qsh + (int64_t)dc.off * a.qss;
  const T* dop =
      static_cast<const T*>(a.dout) + b * a.dosb + h * a.dosh + (int64_t)dc.off * a.doss;
  const T* kp = static_cast<const T*>(a.k) + b * a.ksb + hk * a.ksh + (int64_t)dc.off * a.kss;
  const T* vp = static_cast<const T*>(a.v) + b * a.vsb + hk * a.vsh + (int64_t)dc.off * a.vss;
  const float* lse = a.lse + (int64_t)bh * a.S + dc.off;
  float* delta = a.delta + (int64_t)bh * a.S + dc.off;
  float* nlse2 = a.nlse2 + (int64_t)bh * a.S + dc.off;
  const int64_t gbase = ((int64_t)(b * a.Hkv + hk) * a.G + dc.gofs) * D;
  const T* gkp = static_cast<const T*>(a.gk) + gbase;
  const T* gvp = static_cast<const T*>(a.gv) + gbase;

  const int lo_k = max(0, m0 - W + 1);
  const int hi = min(S, m0 + kBM);
  const int gmax = glob_prefix(hi - 1, W, rpb);
  const int nloc = (hi - lo_k + kBN - 1) / kBN;
  // global tiles first: their first fill is an L2 hit; then the local
  // window from its highest key tile down, in step with the neighbouring
  // query tile's workgroup (see fwd2_kernel; 7% fewer HBM reads)
  const int nglob = (gmax + kBN - 1) / kBN;
  const int ntot = nloc + nglob;
  // Buffer resources over the rows this workgroup may read (local rows below
  // hi, global rows below gmax): loads past them return zeros.
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

  const LaneOffs<D> lo = lane_offs<D>(lane);
  Frag<T> qf[QB][D / 32], df[QB][D / 32];
  int qi[QB];
  float lse2[QB], ndl[QB];
  // Delta = rowsum(O * dO) of this wave's queries, computed here and stored
  // negated (-Delta, the initial value of the dP accumulators) for the dK/dV
  // kernels, with -lse * log2(e) (their exponent's offset): lane (l16, g)
  // sums its 32 columns, then the four lanes of a query add theirs in a
  // fixed order.
  const T* opp = static_cast<const T*>(a.o) + b * a.osb + h * a.osh + (int64_t)dc.off * a.oss;
  // All of the wave's Q, dO and O fragments are loaded before any is used
  // (rows past the document read its last row: those queries' results are
  // never stored), so the loads are in flight together.
  Frag<T> of[QB][D / 32];
  float lv[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    qi[qb] = q0 + 16 * qb + l16;
    const int qr = min(qi[qb], S - 1);
    lv[qb] = lse[qr];
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
      qf[qb][c] = lds_frag_row<T>(qp + (int64_t)qr * a.qss + 32 * c + 8 * g);
      df[qb][c] = lds_frag_row<T>(dop + (int64_t)qr * a.doss + 32 * c + 8 * g);
      of[qb][c] = lds_frag_row<T>(opp + (int64_t)qr * a.oss + 32 * c + 8 * g);
    }
  }
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const bool ok = qi[qb] < S;
    lse2[qb] = ok ? lv[qb] * kLog2e : 0.f;
    float od = 0.f;
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
      const T* eo = reinterpret_cast<const T*>(of[qb][c].w);
      const T* ed = reinterpret_cast<const T*>(df[qb][c].w);
#pragma unroll
      for (int i = 0; i < 8; ++i) od = fmaf(to_f32(eo[i]), to_f32(ed[i]), od);
    }
    od += __shfl_xor(od, 16);
    od += __shfl_xor(od, 32);
    ndl[qb] = -od;
    if (ok && g == 0) {
      delta[qi[qb]] = -od;
      nlse2[qi[qb]] = -lse2[qb];
    }
  }
  const float c2 = a.scale * kLog2e;
  f32x4 dqa[D / 16][QB];
#pragma unroll
  for (int db = 0; db < D / 16; ++db)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) dqa[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bool active = q0 < S;
  const int q_last = min(q0 + kQW, S) - 1;
  const int w_lo = max(0, q0 - W + 1);
  const int wg_lo = active ? glob_prefix(q0, W, rpb) : 0;
  const int wg_hi = active ? glob_prefix(q_last, W, rpb) : 0;
  int glen[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) glen[qb] = glob_prefix(qi[qb], W, rpb);

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
    TileMask<QB> mk;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      mk.hi[qb] = loc ? qi[qb] - ts : glen[qb] - 1 - ts;
      mk.span[qb] = loc ? (unsigned)(W - 1) : 0x7fffffffu;
    }
    if (work) {
      // keys of the tile visible to some query of the wave: [vis_lo, vis_hi]
      const int vis_lo = loc ? w_lo - ts : 0;
      const int vis_hi = loc ? q_last - ts : wg_hi - 1 - ts;
      const bool half0 = vis_lo <= 31, half1 = vis_hi >= 32;
      if (full)
        dq2_tile<T, D, QB, BN, false>(tK, tV, lo, qf, df, dqa, lse2, ndl, c2, g, mk, true, true);
      else
        dq2_tile<T, D, QB, BN, true>(tK, tV, lo, qf, df, dqa, lse2, ndl, c2, g, mk, half0, half1);
    }
  };
  for (int it = 0; it < ntot; it += 2) {
    step(std::integral_constant<int, 0>{}, it);
    if (it + 1 < ntot) step(std::integral_constant<int, 1>{}, it + 1);
  }

  T* dqp = static_cast<T*>(a.dq) + b * a.dqsb + h * a.dqsh + (int64_t)dc.off * a.dqss;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    if (!active || qi[qb] >= S) continue;
    T* row = dqp + (int64_t)qi[qb] * a.dqss;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) store4<T>(row + 16 * db + 4 * g, dqa[db][qb], a.scale);
  }
}

// Key-centric dK/dV: each wave owns KB blocks of 16 key rows (rows of k/v,
// or packed global rows with GLOB), B operands in registers; query tiles of
// BQ rows of Q and dO stream through LDS with their -lse * log2(e) (sL) and
// -Delta (sDl), both written by dq2_kernel. A key row
// j sees the queries [j, j+W-1] (local) or [first_query(j), S) (global rows),
// so every mask is a per-key interval.
template <typename T, int D, int KB, int BQ, bool MASK, bool LOC>
__device__ __forceinline__ void dkdv2_tile(const char* tQ, const char* tO, const float* sL,
                                           const float* sDl, const LaneOffs<D>& lo,
                                           const Frag<T> (&kf)[KB][D / 32],
                                           const Frag<T> (&vf)[KB][D / 32],
                                           f32x4 (&dka)[D / 16][KB], f32x4 (&dva)[D / 16][KB],
                                           float c2, int g, int ts, const int (&qmin)[KB],
                                           const int (&qmax)[KB], const unsigned (&qspan)[KB]) {
  using Tile = SwzTile<D, BQ>;
  constexpr int NS = BQ / 32;  // 32-query subtiles
  // LDS fragments are read PF MFMA steps ahead of their use; scheduling
  // fences keep the compiler from moving the reads next to their uses
  constexpr int PF = 2;
  // S = Q . K^T and dP - Delta = dO . V^T - Delta of subtile qs (two
  // 16-query blocks; sDl holds -Delta, the dP accumulators' initial value)
  auto scores = [&](int qs, f32x4 (&sc)[2][KB], f32x4 (&dp)[2][KB]) {
    constexpr int NC = D / 32, NT = 2 * NC;
    auto row_qo = [&](int t, Frag<T>& q_, Frag<T>& o_) {
      const int qn = 2 * qs + t / NC, cn = t % NC;
      q_ = Tile::template row_frag_at<T>(tQ + qn * Tile::kBlk16 + lo.row[cn]);
      o_ = Tile::template row_frag_at<T>(tO + qn * Tile::kBlk16 + lo.row[cn]);
    };
    Frag<T> qa[PF + 1], oa[PF + 1];
#pragma unroll
    for (int t = 0; t < PF; ++t) row_qo(t, qa[t], oa[t]);
#pragma unroll
    for (int qb2 = 0; qb2 < 2; ++qb2) {
      const f32x4 ndq = *reinterpret_cast<const f32x4*>(sDl + 16 * (2 * qs + qb2) + 4 * g);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        sc[qb2][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
        dp[qb2][kb] = ndq;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int qb2 = t / NC, c = t % NC;
      if (t + PF < NT) row_qo(t + PF, qa[(t + PF) % (PF + 1)], oa[(t + PF) % (PF + 1)]);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        sc[qb2][kb] = mma(sc[qb2][kb], qa[t % (PF + 1)], kf[kb][c]);
        dp[qb2][kb] = mma(dp[qb2][kb], oa[t % (PF + 1)], vf[kb][c]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Each subtile's scores, then its exponentials, in sequence: 165 VGPRs,
  // 3 waves per SIMD. (A software pipeline over the subtiles, the next
  // subtile's score MFMAs beside this one's exponentials, needs 225
  // registers and 2 waves per SIMD: 4.2% slower backward with the local
  // kernel.) LOC (local rows) tests each mask with one unsigned compare;
  // the global-row kernel keeps two compares. Unrolled by two only: the four
  // subtiles of a 128-row tile fully unrolled spill (the compiler hoists the
  // next subtiles' fragment reads).
  f32x4 sc[2][KB], dp[2][KB];  // [qb2][kb]
#pragma unroll 2
  for (int qs = 0; qs < NS; ++qs) {
    scores(qs, sc, dp);
    float p[2][KB][4], ds[2][KB][4];  // [qb2][kb][r]
    // query 16 qblk + 4g + r of the tile is visible to key kb iff
    // (unsigned)(16 qblk + r - q0[kb]) <= qspan[kb]
    int q0[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) q0[kb] = qmin[kb] - ts - 4 * g;
#pragma unroll
    for (int qb2 = 0; qb2 < 2; ++qb2) {
      const int qblk = 2 * qs + qb2;
      const f32x4 nlq = *reinterpret_cast<const f32x4*>(sL + 16 * qblk + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          float x = fmaf(sc[qb2][kb][r], c2, nlq[r]);
          if (MASK) {
            const bool out = LOC ? (unsigned)(16 * qblk + r - q0[kb]) > qspan[kb]
                                 : (ts + 16 * qblk + 4 * g + r < qmin[kb] ||
                                    ts + 16 * qblk + 4 * g + r > qmax[kb]);
            if (out) x = -__builtin_huge_valf();
          }
          p[qb2][kb][r] = __builtin_amdgcn_exp2f(x);
          ds[qb2][kb][r] = p[qb2][kb][r] * dp[qb2][kb][r];
        }
      }
    }
    Frag<T> pf[KB], sf[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const float pv[8] = {p[0][kb][0], p[0][kb][1], p[0][kb][2], p[0][kb][3],
                           p[1][kb][0], p[1][kb][1], p[1][kb][2], p[1][kb][3]};
      const float sv[8] = {ds[0][kb][0], ds[0][kb][1], ds[0][kb][2], ds[0][kb][3],
                           ds[1][kb][0], ds[1][kb][1], ds[1][kb][2], ds[1][kb][3]};
      pf[kb] = pack8<T>(pv);
      sf[kb] = pack8<T>(sv);
    }
    // each transposed Q/dO fragment pair serves every key block of the wave
    Frag<T> ot[PF + 1], qt[PF + 1];
    auto tr_pair = [&](int db, Frag<T>& o_, Frag<T>& q_) {
      const char* po = tO + (2 * qs) * Tile::kBlk16 + lo.tr[db];
      const char* pq = tQ + (2 * qs) * Tile::kBlk16 + lo.tr[db];
      o_ = Tile::template tr_frag_at<T>(po, po + Tile::kBlk16);
      q_ = Tile::template tr_frag_at<T>(pq, pq + Tile::kBlk16);
    };
#pragma unroll
    for (int db = 0; db < PF; ++db) tr_pair(db, ot[db], qt[db]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      if (db + PF < D / 16) tr_pair(db + PF, ot[(db + PF) % (PF + 1)], qt[(db + PF) % (PF + 1)]);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        dva[db][kb] = mma(dva[db][kb], ot[db % (PF + 1)], pf[kb]);
        dka[db][kb] = mma(dka[db][kb], qt[db % (PF + 1)], sf[kb]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// NW waves of KB key blocks each cover the workgroup's 16 * NW * KB key
// rows; query tiles of BQ rows. At most 168 VGPRs: 3 waves per SIMD (the
// global-row kernel below D = 128: at most 128, 4 waves per SIMD).
template <typename T, int D, bool GLOB, int NW, int KB, int BQ>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(GLOB && D < 128 ? 4 : 3)))
void dkdv2_kernel(BwdArgs a) {
  using Tile = SwzTile<D, BQ>;
  constexpr int kKW = 16 * KB, kBK = NW * kKW, kBQ = BQ;
  static_assert(BQ == 32 || BQ == 64 || BQ == 128, "query tile rows");
  // Two pipeline stages as separate LDS objects (see fwd2_kernel): Q and dO
  // rows, and their -lse * log2(e) and -Delta.
  __shared__ __attribute__((aligned(1024))) char stage0[2][Tile::kBytes];
  __shared__ __attribute__((aligned(1024))) char stage1[2][Tile::kBytes];
  __shared__ __attribute__((aligned(16))) float sld0[2][kBQ];  // [-lse log2 e, -delta][q]
  __shared__ __attribute__((aligned(16))) float sld1[2][kBQ];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int nbh = a.B * a.Hkv;
  int item = (int)blockIdx.x;
  if (!GLOB && a.xcd_nt > 0) {
    item = xcd_item(item, nbh, a.xcd_nt);
    if (item < 0) return;  // padding block
  }
  const int bhk = item % nbh;
  const int rest = item / nbh;
  const Doc dc = find_doc(a.docs, rest);
  const int chunk = GLOB ? dc.item % a.nchunk : 0;
  const int tile = GLOB ? dc.item / a.nchunk : dc.item;
  const int b = bhk / a.Hkv, hk = bhk % a.Hkv;
  const int grp = a.Hq / a.Hkv;
  const int S = dc.len, W = dc.W, rpb = dc.rpb;
  const bool relay = rpb > 1;
  const int nrows = GLOB ? (S + W - 1) / W * rpb : S;  // keys: global rows or rows
  const int k0 = tile * kBK;
  const int kw = k0 + wave * kKW;

  const T* kbase;
  const T* vbase;
  int64_t kstride, vstride;
  if (GLOB) {
    const int64_t gb = ((int64_t)bhk * a.G + dc.gofs) * D;
    kbase = static_cast<const T*>(a.gk) + gb;
    vbase = static_cast<const T*>(a.gv) + gb;
    kstride = D;
    vstride = D;
  } else {
    kbase = static_cast<const T*>(a.k) + b * a.ksb + hk * a.ksh + (int64_t)dc.off * a.kss;
    vbase = static_cast<const T*>(a.v) + b * a.vsb + hk * a.vsh + (int64_t)dc.off * a.vss;
    kstride = a.kss;
    vstride = a.vss;
  }

  // query interval of the workgroup; per-key intervals for the masks
  int q_lo, q_hi;
  if (GLOB) {
    const int chunk_len = chunk_len_for(S, a.nchunk);
    const int c_lo = chunk * chunk_len;
    q_hi = min(S, c_lo + chunk_len);
    q_lo = max(c_lo, glob_row_first_query(k0, W, rpb));
    // no query of this chunk sees the tile's rows: gsum_kernel skips the
    // chunk for them (with a single chunk the zeros are written instead)
    if (q_hi <= q_lo && a.nchunk > 1) return;
  } else {
    q_lo = k0;
    q_hi = min(S, k0 + kBK - 1 + W);
  }
  const int ntile_q = q_hi > q_lo ? (q_hi - q_lo + kBQ - 1) / kBQ : 0;
  const int ntot = ntile_q * grp;

  const int qbytes = (int)(a.qss * 2), obytes = (int)(a.doss * 2);
  // the first FW (a power of two) waves fill the tiles
  constexpr int FW = NW >= 8 ? 8 : NW;
  using Fill = typename Tile::template Fill<FW>;
  const int fq = Fill::lane_off(wave & (FW - 1), lane, qbytes);
  const int fo = Fill::lane_off(wave & (FW - 1), lane, obytes);

  const LaneOffs<D> lo = lane_offs<D>(lane);
  Frag<T> kf[KB][D / 32], vf[KB][D / 32];
  int qmin[KB], qmax[KB];
  unsigned qspan[KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int row = kw + 16 * kb + l16;
    // query rows at or past q_hi load as zeros: excluded
    if (GLOB) {
      qmin[kb] = row < nrows ? glob_row_first_query(row, W, rpb) : S;
      qmax[kb] = q_hi - 1;
    } else {
      qmin[kb] = row;
      qmax[kb] = min(row + W, q_hi) - 1;
    }
    // masks test (unsigned)(q - qmin) <= qspan; an empty interval gets a qmin
    // no query reaches
    qspan[kb] = qmax[kb] >= qmin[kb] ? (unsigned)(qmax[kb] - qmin[kb]) : 0u;
    if (!GLOB && qmax[kb] < qmin[kb]) qmin[kb] = 1 << 30;
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
      if (row < nrows) {
        kf[kb][c] = lds_frag_row<T>(kbase + (int64_t)row * kstride + 32 * c + 8 * g);
        vf[kb][c] = lds_frag_row<T>(vbase + (int64_t)row * vstride + 32 * c + 8 * g);
      } else {
        zero_frag(kf[kb][c]);
        zero_frag(vf[kb][c]);
      }
    }
  }
  f32x4 dka[D / 16][KB], dva[D / 16][KB];
#pragma unroll
  for (int db = 0; db < D / 16; ++db)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) dka[db][kb] = dva[db][kb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bool active = kw < nrows;
  const int k_last = min(kw + kKW, nrows) - 1;
  // queries this wave can see at all
  const int wq_lo = GLOB ? (active ? max(q_lo, glob_row_first_query(kw, W, rpb)) : S) : kw;
  const int wq_hi = GLOB ? q_hi : min(q_hi, kw + kKW - 1 + W);
  const int full_lo = GLOB ? (active ? glob_row_first_query(k_last, W, rpb) : S) : k_last;
  const int full_hi = GLOB ? q_hi : kw + W;  // exclusive
  const float c2 = a.scale * kLog2e;

  // Tiles run head by head of the kv group (tile `it` is query tile
  // it % ntile_q of group head it / ntile_q). The (head, tile) counters of
  // the next tile to load and of the tile being computed advance by one per
  // step, and the buffer resources are rebuilt only when the head changes:
  // no per-tile division or 64-bit address arithmetic.
  struct HeadRes {
    __amdgpu_buffer_rsrc_t q, o, l, d;
  };
  auto head_res = [&](int j) {
    const int hq = hk * grp + j;
    const int64_t bh = (int64_t)b * a.Hq + hq;
    // query rows at or past q_hi load as zeros
    HeadRes r;
    r.q = make_rsrc(static_cast<const T*>(a.q) + b * a.qsb + hq * a.qsh + (int64_t)dc.off * a.qss,
                    (uint32_t)((q_hi - 1) * qbytes + D * 2));
    r.o = make_rsrc(
        static_cast<const T*>(a.dout) + b * a.dosb + hq * a.dosh + (int64_t)dc.off * a.doss,
        (uint32_t)((q_hi - 1) * obytes + D * 2));
    r.l = make_rsrc(a.nlse2 + bh * a.S + dc.off, (uint32_t)(S * 4));
    r.d = make_rsrc(a.delta + bh * a.S + dc.off, (uint32_t)(S * 4));
    return r;
  };
  HeadRes ld_res = head_res(0);
  int ld_j = 0, ld_t = 0;  // next tile to load
  auto load_tile = [&](char (&dst)[2][Tile::kBytes], float (&dsl)[2][kBQ]) {
    const int ts = q_lo + ld_t * kBQ;
    if (NW == FW || wave < FW) {
      Fill::load(dst[0], ld_res.q, fq, qbytes, ts, wave);
      Fill::load(dst[1], ld_res.o, fo, obytes, ts, wave);
    }
    // one lane per query row of the tile (lane i of pass c lands at
    // dsl[.][64 c + i])
    if (wave == 0) {
#pragma unroll
      for (int c = 0; c < (kBQ + 63) / 64; ++c) {
        if (kBQ >= 64 || lane < kBQ) {
          const int qrow = min(ts + 64 * c + lane, q_hi - 1);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(ld_res.l, CRA_LDS(&dsl[0][64 * c]), 4,
                                                   qrow * 4, 0, 0, 0);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(ld_res.d, CRA_LDS(&dsl[1][64 * c]), 4,
                                                   qrow * 4, 0, 0, 0);
        }
      }
    }
    if (++ld_t == ntile_q) {
      ld_t = 0;
      if (++ld_j < grp) ld_res = head_res(ld_j);
    }
  };
  if (ntot > 0) load_tile(stage0, sld0);
  int cu_t = 0;  // query tile being computed

  auto step = [&](auto BUFC, int it) {
    constexpr int BUF = decltype(BUFC)::value;
    char(&cur)[2][Tile::kBytes] = BUF ? stage1 : stage0;
    float(&csl)[2][kBQ] = BUF ? sld1 : sld0;
    wait_vmem();
    __syncthreads();
    if (it + 1 < ntot) {
      if (BUF)
        load_tile(stage0, sld0);
      else
        load_tile(stage1, sld1);
    }
    const int ts = q_lo + cu_t * kBQ;
    if (++cu_t == ntile_q) cu_t = 0;
    const int t_last = min(ts + kBQ, q_hi) - 1;
    if (active && t_last >= wq_lo && ts < wq_hi) {
      const bool full = ts >= full_lo && ts + kBQ <= full_hi && ts + kBQ <= q_hi;
      if (full)
        dkdv2_tile<T, D, KB, BQ, false, !GLOB>(cur[0], cur[1], csl[0], csl[1], lo, kf, vf, dka,
                                               dva, c2, g, ts, qmin, qmax, qspan);
      else
        dkdv2_tile<T, D, KB, BQ, true, !GLOB>(cur[0], cur[1], csl[0], csl[1], lo, kf, vf, dka, dva, c2, g,
                                   ts, qmin, qmax, qspan);
    }
  };
  for (int it = 0; it < ntot; it += 2) {
    step(std::integral_constant<int, 0>{}, it);
    if (it + 1 < ntot) step(std::integral_constant<int, 1>{}, it + 1);
  }

  if (GLOB) {
    float* part = a.gpart + (((int64_t)chunk * nbh + bhk) * a.G + dc.gofs) * 2 * D;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int row = kw + 16 * kb + l16;
      if (row >= nrows) continue;
      float* pk = part + (int64_t)row * 2 * D;
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        *reinterpret_cast<f32x4*>(pk + 16 * db + 4 * g) = dka[db][kb] * a.scale;
        *reinterpret_cast<f32x4*>(pk + D + 16 * db + 4 * g) = dva[db][kb];
      }
    }
    return;
  }
  T* dkp = static_cast<T*>(a.dk) + b * a.dksb + hk * a.dksh + (int64_t)dc.off * a.dkss;
  T* dvp = static_cast<T*>(a.dv) + b * a.dvsb + hk * a.dvsh + (int64_t)dc.off * a.dvss;
  const float rsc = (relay && a.rscale) ? a.rscale[hk] : 1.f;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int j = kw + 16 * kb + l16;
    if (j >= S) continue;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) dka[db][kb] *= a.scale;
    const int rblk = j / W;
    int grow[5];
    float gsc[5];
    int nm = 0;
    if (j == rblk * W) {
      grow[nm] = rblk * rpb;
      gsc[nm++] = 1.f;
    }
    if (relay) {
      const int32_t* src = a.src + ((int64_t)bhk * a.NB + dc.bofs + rblk) * a.top_k;
      for (int t = 0; t < a.top_k; ++t) {
        if (src[t] == j) {
          grow[nm] = rblk * rpb + 1 + t;
          gsc[nm++] = rsc;
        }
      }
    }
    // the chunk partials of the global rows are summed into chunk 0
    for (int m = 0; m < nm; ++m) {
      const float* pk = a.gpart + ((int64_t)bhk * a.G + dc.gofs + grow[m]) * 2 * D;
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        dka[db][kb] += *reinterpret_cast<const f32x4*>(pk + 16 * db + 4 * g) * gsc[m];
        dva[db][kb] += *reinterpret_cast<const f32x4*>(pk + D + 16 * db + 4 * g) * gsc[m];
      }
    }
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      store4<T>(dkp + (int64_t)j * a.dkss + 16 * db + 4 * g, dka[db][kb], 1.f);
      store4<T>(dvp + (int64_t)j * a.dvss + 16 * db + 4 * g, dva[db][kb], 1.f);
    }
  }
}

// dK/dV workgroups: waves of 16 key rows (no register file spill into AGPR
// copies at D = 128; 32 rows per wave measured 14% slower). The global-row
// kernel uses 12 waves (192 rows): at 164 VGPRs a SIMD holds 3 of its
// waves, and one 12-wave workgroup fills them, where a second 8-wave
// workgroup did not fit beside the first (8 waves measured 1.7% slower
// backward, 4 waves 3% slower than 8); the local
// kernel 4 waves (64 rows: its band of queries, 64 + W - 1, wastes fewer
// pairs than with 128 rows; measured 7% faster). dQ workgroups: 4 waves of
// 32 queries, 64-key tiles, 2 waves per SIMD at 246 VGPRs (each K/V
// fragment read from LDS serves two query blocks). 16 queries per wave
// lose that reuse: 8 waves measured 27% slower, and with 32-key tiles at
// 3 or 4 waves per SIMD still 5-10% slower backward at D = 128.
// Below D = 128 the global-row kernel needs at most 128 VGPRs (114 at
// D = 64), so two 8-wave workgroups share a CU at 4 waves per SIMD, where
// one 12-wave workgroup left it at 3: backward 1.4% faster at B=1 H=12
// S=131072 D=64 and 3.3% at H=8 S=65536 (16-wave workgroups: 0.8%).
// Below D = 128 the local kernel's waves take 32 key rows each (two 16-key
// blocks sharing every Q/dO fragment read from LDS; 168 VGPRs, 3 waves per
// SIMD): twice the MFMAs per LDS read and per barrier of its 32-query
// tiles. Config 4 training (B=1 H=12 D=64) 1.2-1.7% faster at S = 8192,
// 32768 and 131072 (three alternating runs).
template <int D>
constexpr int kDkdvGlobWaves = D == 128 ? 12 : 8;
constexpr int kDkdvLocalWaves = 4;
constexpr int kDkdvKB = 1;  // 16-key blocks per wave (global-row kernel)
template <int D>
constexpr int kDkdvLocalKB = D == 128 ? 1 : 2;  // local kernel
constexpr int kDqWaves = 4;
constexpr int kDqQB = 2;    // 16-query blocks per dQ wave
constexpr int kDqBN = 64;   // key rows per dQ tile
constexpr int kDqWPE = 2;   // dQ waves per SIMD (register budget)
// Query rows per dK/dV tile. The local kernel's 32-row tiles keep its LDS
// at 33 KB, so three 4-wave workgroups (3 waves per SIMD, 165 VGPRs) fit on
// a CU; with 64-row tiles only two fit. The global-row kernel (one 12-wave
// workgroup per CU, 130 KB of LDS) takes 128-row tiles: one barrier per 128
// queries instead of 64 (backward 1.7% faster).
constexpr int kDkdvGlobBQ = 128;
constexpr int kDkdvLocalBQ = 32;

// The gfx950-tiled kernels (dq2, dkdv2) serve fp16/bf16 up to D = 128; the
// generic kernels serve fp32 and every dtype at D = 256.
template <typename T, int D>
constexpr bool kTiledBwd = sizeof(T) == 2 && D <= 128;
template <int D>
constexpr int kGenericNB = D > 128 ? 1 : 2;

template <typename T, int D>
hipError_t launch_TD(const BwdArgs& a, hipStream_t st) {
  constexpr bool kTiled = kTiledBwd<T, D>;
  constexpr int NB = kGenericNB<D>;
  using Tr = BwdTraits<T, D, NB>;
  constexpr int kRows = 256 / (D / 8);
  // tiled path: dq2_kernel computes Delta for its own queries and stores
  // -Delta (with -lse * log2(e)) for the dK/dV kernels
  if (!kTiled && a.group == 0)
    hipLaunchKernelGGL((delta_kernel<T, D>), dim3((a.S + kRows - 1) / kRows, a.B * a.Hq),
                       dim3(256), 0, st, a);
  // work items per document: query tiles (dQ), global-row tiles x query
  // chunks (global dK/dV), key tiles (local dK/dV), each of its kernel's
  // workgroup size
  BwdArgs aq = a, ag = a, al = a;
  constexpr int kQM = kTiled ? 16 * kDqWaves * kDqQB : Tr::kBM;  // dQ queries per workgroup
  set_items(aq.docs, [&](int d) { return (a.docs.len[d] + kQM - 1) / kQM; });
  constexpr int kGK = kTiled ? 16 * kDkdvGlobWaves<D> * kDkdvKB : Tr::kBK;   // rows per workgroup
  constexpr int kLK = kTiled ? 16 * kDkdvLocalWaves * kDkdvLocalKB<D> : Tr::kBK;
  set_items(ag.docs, [&](int d) {
    const int g = (a.docs.len[d] + a.docs.W[d] - 1) / a.docs.W[d] * a.docs.rpb[d];
    return (g + kGK - 1) / kGK * a.nchunk;
  });
  set_items(al.docs, [&](int d) { return (a.docs.len[d] + kLK - 1) / kLK; });
  const int nq = aq.docs.item0[a.docs.n], ng = ag.docs.item0[a.docs.n];
  const int nl = al.docs.item0[a.docs.n];
  // one document, D = 128 and a head count that is not a multiple of 8: the
  // dQ and local dK/dV kernels run in the XCD-aware order (as the forward)
  const bool xq = kTiled && D == 128 && a.docs.n == 1 && (a.B * a.Hq) % 8 != 0;
  const bool xl = kTiled && D == 128 && a.docs.n == 1 && (a.B * a.Hkv) % 8 != 0;
  aq.xcd_nt = xq ? nq : 0;
  al.xcd_nt = xl ? nl : 0;
  const int gq = xq ? xcd_grid(a.B * a.Hq, nq) : nq * a.B * a.Hq;
  const int gl = xl ? xcd_grid(a.B * a.Hkv, nl) : nl * a.B * a.Hkv;
  if constexpr (kTiled) {
    hipLaunchKernelGGL((dq2_kernel<T, D, kDqWaves, kDqQB, kDqBN, kDqWPE>), dim3(gq),
                       dim3(64 * kDqWaves), 0, st, aq);
    hipLaunchKernelGGL((dkdv2_kernel<T, D, true, kDkdvGlobWaves<D>, kDkdvKB, kDkdvGlobBQ>),
                       dim3(ng * a.B * a.Hkv), dim3(64 * kDkdvGlobWaves<D>), 0, st, ag);
  } else {
    hipLaunchKernelGGL((dq_kernel<T, D, NB>), dim3(nq * a.B * a.Hq), dim3(256), 0, st, aq);
    hipLaunchKernelGGL((dkdv_kernel<T, D, NB, true>), dim3(ng * a.B * a.Hkv), dim3(256), 0, st,
                       ag);
  }
  if (a.nchunk > 1) {
    BwdArgs as = a;
    set_items(as.docs, [&](int d) {
      const int g = (a.docs.len[d] + a.docs.W[d] - 1) / a.docs.W[d] * a.docs.rpb[d];
      return (g * (2 * D / 4) + 255) / 256;
    });
    hipLaunchKernelGGL((gsum_kernel<D>), dim3(as.docs.item0[a.docs.n] * a.B * a.Hkv), dim3(256),
                       0, st, as);
  }
  if (a.dalpha) hipLaunchKernelGGL((dalpha_kernel<T, D>), dim3(a.Hkv), dim3(256), 0, st, a);
  if constexpr (kTiled)
    hipLaunchKernelGGL((dkdv2_kernel<T, D, false, kDkdvLocalWaves, kDkdvLocalKB<D>, kDkdvLocalBQ>),
                       dim3(gl), dim3(64 * kDkdvLocalWaves), 0, st, al);
  else
    hipLaunchKernelGGL((dkdv_kernel<T, D, NB, false>), dim3(nl * a.B * a.Hkv), dim3(256), 0, st,
                       al);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_T(int D, const BwdArgs& a, hipStream_t st) {
  switch (D) {
    case 32: return launch_TD<T, 32>(a, st);
    case 64: return launch_TD<T, 64>(a, st);
    case 128: return launch_TD<T, 128>(a, st);
    case 256: return launch_TD<T, 256>(a, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace

size_t bwd_workspace_bytes(int D, int B, int Hq, int Hkv, int S, int n, const int* len,
                           const int* W, const int* rpb, int64_t G, int cus, int* nchunk) {
  // Query chunks of the global-row kernel: each document's query range is
  // cut into the same number of chunks (multiples of 64 queries), one
  // workgroup per (row tile, chunk). More chunks balance the uneven
  // workgroups better (a late row tile sees only the last queries) and
  // shorten the last round; each chunk costs a partial dK/dV of its rows,
  // written once and summed once by gsum_kernel. Measured on gfx950 over
  // 1-48 chunks (training step, 2 sweeps): the best counts fill the kernel's
  // resident slots about 1.5 times over (the device's CUs, one 12-wave
  // workgroup per CU at D = 128, two 8-wave ones below) until chunks would
  // exceed about 6144 queries, from which on 6144-query chunks keep the
  // balance. On the 256-CU MI355X:
  //   B=1 H=16 D=128 S=131072: 22 chunks (16 and 32 within 0.6%)
  //   B=1 H=12 D=64 S=8192 / 32768 / 131072: 22 / 13 / 22 chunks
  //   B=2 H=32 D=128 S=4096: 6 (the previous rule's 16 was 12% slower)
  //   B=1 H=8 D=64 S=16384: 32 (64 was 10% slower)
  // (D = 256 runs the generic global-row kernel: 64 rows per 4-wave
  // workgroup, two workgroups per CU by their 71 KB of LDS)
  const int rows = D > 128    ? BwdTraits<f16, 256, 1>::kBK
                   : D == 128 ? 16 * kDkdvGlobWaves<128> * kDkdvKB
                              : 16 * kDkdvGlobWaves<64> * kDkdvKB;
  const int slots = (cus > 0 ? cus : 256) * (D == 128 ? 1 : 2);
  int64_t row_tiles = 0;
  int max_len = 1;
  for (int d = 0; d < n; ++d) {
    const int64_t g = (int64_t)(len[d] + W[d] - 1) / W[d] * rpb[d];
    row_tiles += (g + rows - 1) / rows;
    if (len[d] > max_len) max_len = len[d];
  }
  const int64_t base = row_tiles * B * Hkv;
  int64_t nc = (3 * slots + 2 * base - 1) / (2 * base);  // 1.5 rounds of workgroups
  const int64_t by_len = (max_len + 6143) / 6144;
  if (nc < by_len) nc = by_len;
  const int64_t max_nc = (max_len + 255) / 256;
  if (nc > max_nc) nc = max_nc;
  if (nc < 1) nc = 1;
  *nchunk = (int)nc;
  return bwd_workspace_layout(D, B, Hq, Hkv, S, G, (int)nc);
}

size_t bwd_workspace_layout(int D, int B, int Hq, int Hkv, int S, int64_t G, int nchunk) {
  // Delta (2-byte path: -Delta) and -lse * log2(e) per query, then the chunk
  // partials
  const size_t delta = (((size_t)B * Hq * S * 4) + 255) / 256 * 256;
  const size_t part = (size_t)nchunk * B * Hkv * G * 2 * D * 4;
  return 2 * delta + part;
}

bool bwd_tile_config(int dtype, int D, int out[9]) {
  if (dtype < 0 || dtype > 2 || (D != 32 && D != 64 && D != 128 && D != 256)) return false;
  if (D == 256) {
    using Tr = BwdTraits<f16, 256, 1>;  // the same geometry for every dtype
    const int waves = Tr::kThreads / 64;
    const int v[9] = {waves, Tr::kBM, Tr::kBN, waves, Tr::kBK, Tr::kBQ, waves, Tr::kBK, Tr::kBQ};
    for (int i = 0; i < 9; ++i) out[i] = v[i];
  } else if (dtype == 2) {
    using Tr = BwdTraits<float, 128>;
    const int waves = Tr::kThreads / 64;
    const int v[9] = {waves, Tr::kBM, Tr::kBN, waves, Tr::kBK, Tr::kBQ, waves, Tr::kBK, Tr::kBQ};
    for (int i = 0; i < 9; ++i) out[i] = v[i];
  } else {
    const int gw = D == 128 ? kDkdvGlobWaves<128> : kDkdvGlobWaves<64>;
    const int lkb = D == 128 ? kDkdvLocalKB<128> : kDkdvLocalKB<64>;
    const int v[9] = {kDqWaves,        16 * kDqWaves * kDqQB,        kDqBN,
                      gw,              16 * gw * kDkdvKB,            kDkdvGlobBQ,
                      kDkdvLocalWaves, 16 * kDkdvLocalWaves * lkb,   kDkdvLocalBQ};
    for (int i = 0; i < 9; ++i) out[i] = v[i];
  }
  return true;
}

hipError_t launch_bwd(int dtype, int D, const BwdArgs& a, hipStream_t st) {
  switch (dtype) {
    case 0: return launch_T<f16>(D, a, st);
    case 1: return launch_T<bf16>(D, a, st);
    case 2: return launch_T<float>(D, a, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace cra

/*
 * cra.h -- C ABI of the MI355X (gfx950) sqrt(N) sparse-attention library
 * (libcra_hip.so).
 *
 * The attention computed is the reference's three-phase pattern: for query i
 * with ls = max(0, i-W+1) the keys are the local window [ls, i], the strided
 * rows s*W < ls, and (when relay is on) the top_k highest-||k||^2 rows of
 * every W-block that ends before ls; one softmax runs over the multiset.
 *
 * Conventions (every entry point):
 *  - Return value: 0 on success, a negative CRA_E_* code otherwise; the
 *    message of the last failure on the calling thread is available from
 *    cra_last_error(). No exceptions cross the ABI, no host synchronisation
 *    happens, nothing is allocated: the caller passes every buffer (the one
 *    exception, cra_bwd_noalloc, uses a fixed device array of the library).
 *  - Tensors of shape [B, H, S, D] are passed as cra_tensor: a device pointer
 *    and element strides for B, H and S; D must be contiguous (stride 1), the
 *    pointer and every row start must be 16-byte aligned.
 *  - `stream` is a hipStream_t (0 = the null stream); all work is enqueued on it.
 *  - Concurrent calls on different streams are safe; the library keeps no
 *    mutable global state (except the scratch of cra_bwd_noalloc, whose
 *    concurrent calls on one device race).
 */
#ifndef CRA_H_
#define CRA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CRA_ABI_VERSION 1

enum {
  CRA_OK = 0,
  CRA_E_INVALID = -1,     /* bad shape, size or argument */
  CRA_E_LAYOUT = -2,      /* stride/alignment the kernels cannot take */
  CRA_E_DTYPE = -3,       /* unknown dtype code */
  CRA_E_UNSUPPORTED = -4, /* valid but not built (e.g. head dim) */
  CRA_E_HIP = -5,         /* HIP runtime error (launch, device query) */
  CRA_E_WORKSPACE = -6    /* workspace missing or too small */
};

enum { CRA_F16 = 0, CRA_BF16 = 1, CRA_F32 = 2 };

/* One attention problem. W, relay and top_k are the planner's choices
 * (the reference uses W = ceil(sqrt(S)), relay = S > 2048, top_k = 2;
 * core.py:3479, 3507, 3771). `scale` is the logit scale (1/sqrt(head dim)). */
typedef struct {
  int32_t B, H_q, H_kv, S, D;
  int32_t W;
  int32_t relay; /* 0 or 1 */
  int32_t top_k; /* relay rows per block, 1..4 (ignored when relay == 0) */
  int32_t dtype; /* CRA_F16, CRA_BF16 or CRA_F32 */
  float scale;
} cra_problem;

typedef struct {
  void* ptr;
  int64_t sb, sh, ss; /* element strides of B, H, S; D is contiguous */
} cra_tensor;

typedef struct {
  int32_t cu_count;
  int32_t lds_bytes_per_cu;
  int32_t arch_major, arch_minor; /* 9, 50 for gfx950 */
  char arch_name[64];
  char device_name[128];
} cra_device_info_t;

/* Head dims the kernels are built for: 32, 64, 128 and 256 (others up to
 * 256: pad to the next one; the reference takes any D, core.py:3495). */
int cra_supported_head_dim(int32_t D);

/* Rows of the packed "global" key/value array per (b, kv head):
 * ceil(S/W) * (1 + top_k) with relay, ceil(S/W) without. Block r occupies
 * rows r*(1+top_k) .. : first k[r*W] (its strided row), then its top_k relay
 * rows in rank order. Query i sees exactly the prefix of length
 * (1+top_k)*floor(ls/W) + (ls % W != 0) (relay) or ceil(ls/W) (no relay). */
int64_t cra_global_rows(const cra_problem* p);

/* Builds the packed global rows and the relay source rows.
 *   k, v:       [B, H_kv, S, D]
 *   glob_k/v:   contiguous [B, H_kv, cra_global_rows(p), D], dtype of k
 *   relay_src:  contiguous int32 [B, H_kv, ceil(S/W) * top_k] (may be NULL
 *               when relay == 0)
 *   relay_scale: NULL, or fp32 [H_kv] multipliers applied to the relay rows
 *               (the caller passes exp(relay_log_scale) already rounded to
 *               the input dtype).
 * Replaces the relay pre-computation kernel `_relay_precompute_topk`
 * (reference core.py:2630-2748, launched at core.py:3516-3534) and the
 * relay_log_scale multiply (core.py:3541-3544); also gathers the strided
 * rows the reference's forward reads in place (core.py:1042-1087). */
int cra_build_global(const cra_problem* p, cra_tensor k, cra_tensor v, void* glob_k,
                     void* glob_v, int32_t* relay_src, const float* relay_scale, void* stream);

/* Forward: o [B, H_q, S, D] (dtype of q) and lse fp32 contiguous [B, H_q, S]
 * (natural-log log-sum-exp per query). Query head h reads kv head
 * h / (H_q / H_kv).
 * Replaces the tiled forward `_cron_root_attn_fwd_v14_tiled`
 * (reference core.py:907-1158, launched at core.py:3588-3610). */
int cra_fwd(const cra_problem* p, cra_tensor q, cra_tensor k, cra_tensor v,
            const void* glob_k, const void* glob_v, cra_tensor o, float* lse, void* stream);

/* cra_fwd as a persistent kernel: a grid of one round of resident
 * workgroups (CUs x workgroups per CU) that take the 128-query tiles, heaviest
 * first, from the device counter *work_counter, which must be zero on entry
 * (it ends at the number of tiles plus the number of workgroups; zero it
 * again before the next call). Same results as cra_fwd, bit for bit (fp32
 * inputs run cra_fwd's kernel). Replaces the reference's persistent forward
 * `_cron_root_attn_fwd_v14_persistent` (core.py:711-900) with its atomic work
 * queue, launched for use_persistent on sequences without relay
 * (core.py:3548-3569). */
int cra_fwd_persistent(const cra_problem* p, cra_tensor q, cra_tensor k, cra_tensor v,
                       const void* glob_k, const void* glob_v, cra_tensor o, float* lse,
                       int32_t* work_counter, void* stream);

/* Key phases for cra_fwd_phases. */
#define CRA_PHASE_LOCAL 1  /* the local window [ls, i] */
#define CRA_PHASE_GLOBAL 2 /* the packed strided and relay rows */

/* cra_fwd over a subset of the key phases: o and lse are the attention of
 * each query over the keys of the selected phases only (a query with no such
 * key gets o = 0, lse = -inf). phase_mask = CRA_PHASE_LOCAL | CRA_PHASE_GLOBAL
 * is cra_fwd. No counterpart in the reference, whose forward interleaves the
 * phases in one kernel (core.py:976-1142); it exists so that the MFMA
 * utilisation of each phase can be measured on its own. */
int cra_fwd_phases(const cra_problem* p, cra_tensor q, cra_tensor k, cra_tensor v,
                   const void* glob_k, const void* glob_v, cra_tensor o, float* lse,
                   int32_t phase_mask, void* stream);

/* Workspace the backward needs, in bytes (0 is possible). */
size_t cra_bwd_workspace_bytes(const cra_problem* p);

/* Backward: dq [B,H_q,S,D], dk/dv [B,H_kv,S,D] in the input dtype, given
 * the forward's o and lse and the upstream gradient do. The gradient of the
 * relay rows is added to their source rows (times relay_scale when given);
 * with kv groups the kv gradients are summed over the group's query heads.
 * If dalpha is not NULL it receives fp32 [H_kv]: sum over relay rows of
 * dRK*RK + dRV*RV (the gradient of relay_log_scale), else it is skipped.
 * Replaces the backward `CronRootAttentionV14Function.backward`
 * (reference core.py:3626-3759) and its kernels: dQ (core.py:1165-1316),
 * local dK/dV (core.py:1650-1745), strided dK/dV (core.py:1755-1889), relay
 * dK/dV (core.py:2381-2492) and the relay scatter (core.py:2767-2815). */
int cra_bwd(const cra_problem* p, cra_tensor q, cra_tensor k, cra_tensor v, cra_tensor o,
            cra_tensor dout, const float* lse, const void* glob_k, const void* glob_v,
            const int32_t* relay_src, const float* relay_scale, cra_tensor dq, cra_tensor dk,
            cra_tensor dv, float* dalpha, void* workspace, size_t workspace_bytes, void* stream);

/* Size of the fixed device scratch of cra_bwd_noalloc, per device. */
#define CRA_NOALLOC_SCRATCH_BYTES (64u << 20)

/* cra_bwd without a workspace argument and without any allocation: for
 * callers that cannot allocate device memory (tight serving loops, harnesses
 * that forbid hipMalloc). No counterpart in the reference. Its use under HIP
 * graph capture is untested: the first call on a device looks up the
 * scratch address with hipGetSymbolAddress, so make one call on each device
 * before any capture.
 * The workspace is a file-scope device array of CRA_NOALLOC_SCRATCH_BYTES
 * (64 MiB) that every device the library runs on holds until the process
 * ends; its address is looked up once per device on the first call there.
 * The stream must belong to the current device (else CRA_E_INVALID). The
 * global-row partials keep cra_bwd's query-chunk count when it fits (the
 * results are then bit-identical to cra_bwd's) and use fewer chunks
 * otherwise (same gradients up to the fp32 summation order); a problem
 * whose workspace exceeds the scratch even with one chunk returns
 * CRA_E_WORKSPACE. Nothing in the scratch needs clearing: every call writes
 * what it reads. All calls on one device share that device's scratch, so
 * calls that overlap on one device (two streams, two threads) race: the
 * caller must order them. Other arguments and results as cra_bwd. */
int cra_bwd_noalloc(const cra_problem* p, cra_tensor q, cra_tensor k, cra_tensor v, cra_tensor o,
                    cra_tensor dout, const float* lse, const void* glob_k, const void* glob_v,
                    const int32_t* relay_src, const float* relay_scale, cra_tensor dq,
                    cra_tensor dk, cra_tensor dv, float* dalpha, void* stream);

/* Documents packed along S (varlen): document d is rows
 * cu_seqlens[d] .. cu_seqlens[d+1]-1 of every [B, H, S, D] tensor and is
 * attended on its own (nothing across documents), with its own window and
 * relay switch. All three arrays are host memory, read during the call only.
 * In the cra_problem of a *_varlen call S is the packed length
 * cu_seqlens[n_docs]; W and relay are not used; top_k applies to every
 * document with relay on. */
typedef struct {
  int32_t n_docs;
  const int32_t* cu_seqlens; /* n_docs + 1 entries rising strictly from 0 to S */
  const int32_t* window;     /* n_docs entries, 1 <= window[d] <= length of d
                                (the reference: ceil(sqrt(length)), core.py:3479) */
  const int32_t* relay;      /* n_docs entries, 0 or 1 (the reference: length > 2048,
                                core.py:3507) */
} cra_docs;

/* Sizes of the packed global rows and relay source rows of a varlen call,
 * per (b, kv head): the documents' blocks in document order, document d
 * taking ceil(len/W) * (1 + top_k) (relay) or ceil(len/W) rows of glob_k/v
 * laid out as for one sequence (cra_global_rows), and ceil(len/W) * top_k
 * relay_src entries (row indices relative to the document's first row; the
 * entries of a document without relay are not written). */
int cra_varlen_sizes(const cra_problem* p, const cra_docs* docs, int64_t* global_rows,
                     int64_t* relay_src_len);

/* The varlen forms of cra_build_global, cra_fwd, cra_bwd_workspace_bytes and
 * cra_bwd: same buffers and contracts with the sizes of cra_varlen_sizes; one
 * call covers every document (launches take up to 64 documents each).
 * relay_scale and dalpha are per kv head over all documents.
 * Replace the per-document loop of `cron_root_attention_varlen` (reference
 * core.py:3836-3954), which calls the whole op once per document on narrow()
 * views and copies each result into the output. */
int cra_build_global_varlen(const cra_problem* p, const cra_docs* docs, cra_tensor k,
                            cra_tensor v, void* glob_k, void* glob_v, int32_t* relay_src,
                            const float* relay_scale, void* stream);
int cra_fwd_varlen(const cra_problem* p, const cra_docs* docs, cra_tensor q, cra_tensor k,
                   cra_tensor v, const void* glob_k, const void* glob_v, cra_tensor o, float* lse,
                   void* stream);
size_t cra_bwd_workspace_bytes_varlen(const cra_problem* p, const cra_docs* docs);
int cra_bwd_varlen(const cra_problem* p, const cra_docs* docs, cra_tensor q, cra_tensor k,
                   cra_tensor v, cra_tensor o, cra_tensor dout, const float* lse,
                   const void* glob_k, const void* glob_v, const int32_t* relay_src,
                   const float* relay_scale, cra_tensor dq, cra_tensor dk, cra_tensor dv,
                   float* dalpha, void* workspace, size_t workspace_bytes, void* stream);

/* Host (CPU) forward for CPU tensors: q, k, v, o are host memory in the
 * layout above (any element strides, D contiguous). The attention
 * set is the one above with p->W, p->relay and p->top_k, except that the
 * relay rows of the last, partial block are chosen over the block padded
 * with zero rows and relay rows are ranked by ||k||^2 rounded to the input
 * dtype (earlier row first on equal norms). Arithmetic in fp32, one
 * rounding of o to the input dtype; `threads` worker threads (>= 1).
 * Replaces the reference's CPU dispatch `cra_cpu_fast_compiled(q, k, v)`
 * (core.py:3794-3796; cra_cpu_fast, cpu_reference.py:198-339), whose plan
 * the caller passes: W = isqrt(S), relay = 1, top_k = 2. No backward (the
 * reference's CPU path has none that runs). */
int cra_fwd_cpu(const cra_problem* p, cra_tensor q, cra_tensor k, cra_tensor v, cra_tensor o,
                int32_t threads);

/* Device facts for get_num_sms()/get_gpu_info() (reference core.py:137-188,
 * __init__.py:183-202). */
int cra_device_info(int32_t device, cra_device_info_t* out);

/* The tile geometry compiled for (dtype, D): waves per workgroup, rows per
 * workgroup (queries or key rows) and rows per streamed tile of the forward
 * and the three backward kernels. Serves calibrate(), which in the reference
 * times Triton (num_warps, num_stages) candidates per (op, H, D)
 * (_KernelAutoTuner, core.py:250-596; __init__.py:84-180); here the
 * geometry is fixed per (gfx950, dtype, D) at build time. */
typedef struct {
  int32_t fwd_waves, fwd_queries, fwd_key_tile;
  int32_t dq_waves, dq_queries, dq_key_tile;
  int32_t dkdv_global_waves, dkdv_global_rows, dkdv_global_query_tile;
  int32_t dkdv_local_waves, dkdv_local_keys, dkdv_local_query_tile;
} cra_tile_config_t;
int cra_tile_config(int32_t dtype, int32_t D, cra_tile_config_t* out);

const char* cra_strerror(int32_t code);
const char* cra_last_error(void);
int32_t cra_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CRA_H_ */

/*
 * sfa.h — C ABI of libsfa.so, the MI355X (gfx950) top-k sparse flash attention.
 *
 * The boundary replaces the three kernel launches of the reference's autograd
 * host launcher `SparseFlashAttentionTriton` (lilac-me/ops SFA.py:69-306):
 *
 *   sfa_fwd  <- `_attn_fwd[grid](...)`            SFA.py:122-159 (forward, SFA.py:75-164)
 *   sfa_bwd  <- `_attn_bwd_dq_dsink[grid](...)`   SFA.py:199-251
 *             + `_attn_bwd_dk_dv[grid](...)`      SFA.py:266-298 (backward, SFA.py:166-306)
 *
 * plus the workspace sizing the reference does inline with torch.empty
 * (SFA.py:117-120, 188-194, 253-261) and its ValueError paths
 * (SFA.py:52-53, 63-64).
 *
 * Conventions
 *  - Layout is BSHD with element strides for the batch, sequence and head
 *    dimensions; the last (feature) dimension must be contiguous.
 *      q   [B, Sq,  Hq,  Dqk]     k [B, Skv, Hkv, Dqk]     v [B, Skv, Hkv, Dv]
 *      idx [B, Sq,  Hkv, topk]  int32, -1 (or any out-of-range value) = padding
 *      out [B, Sq,  Hq,  Dv]      lse [B, Sq, Hq] float32, natural log
 *    `v` may alias `k` (e.g. MLA: v = k[..., :Dv]); inputs are never written.
 *    Query head h reads KV head h / (Hq / Hkv).
 *  - A slot is valid iff 0 <= idx < bound, bound = kv_lens[b] (if non-NULL,
 *    clamped to Skv) else Skv.  Invalid slots contribute exactly nothing; a
 *    row with no valid slot gives out = 0 and lse = -inf.
 *  - `sink` (optional, float32 [Hq]) adds exp(sink[h]) to every softmax
 *    denominator as SFA.py:469-474 does; NULL means no sink.
 *  - All pointers are device pointers.  The library never allocates, frees
 *    or synchronises: scratch comes from the caller through `workspace`,
 *    whose size the *_workspace_size functions give for the same arguments.
 *    All work is enqueued on `stream` (a hipStream_t; NULL = default stream).
 *  - Return value: 0 on success, a negative SFA_E* code otherwise; the
 *    message for the calling thread is available from sfa_last_error().
 */
#ifndef SFA_H_
#define SFA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SFA_ABI_VERSION 2

#if defined(__GNUC__)
#define SFA_API __attribute__((visibility("default")))
#else
#define SFA_API
#endif

/* Element types of q, k, v, out, dout, dq, dk, dv (F32, BF16), and of the
 * index producer's q / k (BF16, FP8_E4M3: OCP e4m3, one byte). */
enum { SFA_DTYPE_F32 = 0, SFA_DTYPE_BF16 = 1, SFA_DTYPE_FP8_E4M3 = 2 };

/* How the backward produces dK/dV. */
enum {
  SFA_DKV_AUTO = 0,    /* CSR where supported (bf16, d_qk = d_v = 128, G a power of two
                          <= 128, top-k <= 2048, Skv <= 262144) and cheaper: Skv <=
                          64 * top-k and CSR workspace (bitmap, lists, fp32 partials,
                          which grow as Skv * Sq * G / 16 bytes per batch and kv head)
                          <= 4 GiB; otherwise ATOMIC                                   */
  SFA_DKV_ATOMIC = 1,  /* fp32 atomic adds into a workspace accumulator (SFA.py:853)    */
  SFA_DKV_CSR = 2      /* deterministic: membership bitmap inverted into per-key-block
                          lists of referencing query blocks, key-major recompute, fixed-
                          order reduction (index rows that repeat a key take atomics for
                          the repeats); SFA_E_UNSUPPORTED outside the supported shapes
                          (the cost rules of AUTO do not apply).  dsink is reduced in a
                          fixed order in every mode                                     */
};

/* sfa_bwd_args.flags */
#define SFA_BWD_MERGE_KV 1  /* v is the first Dv dims of k's rows (v == k with k's strides, Dv <= Dqk),
                               the reference's single shared kv (SFA.py:88, 116): dk receives the
                               gradient of the shared rows, dK + dV on their first Dv dims, as
                               SFA.py:849-853 sums both into one buffer; dv is not written and may
                               be NULL.  The MLA shape (d_qk 576, d_v 512, 65..128 heads per KV head,
                               bf16) then runs its MFMA backward: AUTO and SFA_DKV_CSR sum per-slot
                               bf16 rows of the shared rows' gradient in a fixed order (Skv <= 65536;
                               slots repeating a key of their row take fp32 atomics), SFA_DKV_ATOMIC
                               adds every slot's fp32 row atomically                              */

/* sfa_fwd_args.flags (the backward ignores them) */
#define SFA_FWD_IDX_SORTED 1  /* every index row lists its valid keys in ascending order before any
                                 padding (what sfa_indexer_topk writes).  Without it the persistent
                                 MLA prefill (the MLA shape, no split-k, >= 4096 work items,
                                 top-k <= 2048, Skv <= 65536; contiguous or paged kv) first writes its rows
                                 in that order into the workspace (valid keys ascending, then -1; a
                                 row that repeats a key is kept as it is) and walks those: the
                                 queries running together on an XCD then gather the same regions
                                 of the prefix at about the same time and share them in its L2.
                                 The result is the same softmax in another summation order
                                 (differences at fp32 rounding).  The flag only skips that pass   */

/* Error codes. */
enum {
  SFA_OK = 0,
  SFA_E_INVALID = -1,   /* bad shape / stride / dtype / null pointer (ValueError) */
  SFA_E_WORKSPACE = -2, /* workspace missing or too small                        */
  SFA_E_UNSUPPORTED = -3,
  SFA_E_HIP = -4        /* a HIP runtime call failed (RuntimeError)               */
};

typedef struct sfa_fwd_args {
  int32_t dtype;                 /* SFA_DTYPE_*                                       */
  int32_t B, Sq, Skv, Hq, Hkv, Dqk, Dv, topk;
  float scale;                   /* softmax scale; <= 0 means 1/sqrt(Dqk) (SFA.py:181-182) */
  const void* q;   int64_t q_sb, q_ss, q_sh;
  const void* k;   int64_t k_sb, k_ss, k_sh;
  const void* v;   int64_t v_sb, v_ss, v_sh;
  const int32_t* idx; int64_t i_sb, i_ss, i_sh;   /* slot stride is 1 */
  const int32_t* kv_lens;        /* [B] or NULL                                        */
  const float* sink;             /* [Hq] or NULL                                       */
  void* out;       int64_t o_sb, o_ss, o_sh;
  float* lse;      int64_t l_sb, l_ss, l_sh;      /* head stride of lse             */
  int32_t num_splits;            /* split-k over the top-k set; 0 = library choice      */
  int32_t flags;                 /* 0 or SFA_FWD_IDX_SORTED                             */
} sfa_fwd_args;

typedef struct sfa_bwd_args {
  sfa_fwd_args fwd;              /* the forward's arguments; out/lse are read here      */
  const void* dout; int64_t do_sb, do_ss, do_sh;
  void* dq;        int64_t dq_sb, dq_ss, dq_sh;
  void* dk;        int64_t dk_sb, dk_ss, dk_sh;
  void* dv;        int64_t dv_sb, dv_ss, dv_sh;
  const float* dlse;             /* gradient w.r.t. lse, float32, lse's strides; NULL = 0 */
  float* dsink;                  /* [Hq] float32, written (not accumulated); NULL if no sink */
  int32_t dkv_mode;              /* SFA_DKV_*                                           */
  int32_t flags;                 /* 0 or SFA_BWD_MERGE_KV                               */
} sfa_bwd_args;

/* Paged KV cache (block table) for sfa_fwd_paged.  k and v then point to
 * page pools [num_pages, page_size, Hkv, D]: k_sb / v_sb are the page strides,
 * k_ss / v_ss the row strides within a page, k_sh / v_sh the head strides.
 * Logical key position i of sequence b (what idx holds) is row
 * i % page_size of page block_table[b * bt_sb + i / page_size].
 * A slot is valid iff 0 <= idx < bound (bound = kv_lens[b] clamped to Skv,
 * else Skv; Skv <= max_pages * page_size) and its page id lies in
 * [0, num_pages); an unmapped page (e.g. -1) makes the slot invalid. */
typedef struct sfa_kv_pages {
  const int32_t* block_table;    /* [B, max_pages] int32 page ids                     */
  int64_t bt_sb;                 /* block-table row stride (elements); the table's
                                    extent, ((B - 1) * bt_sb + max_pages) * 4 bytes,
                                    must stay below 4 GiB                            */
  int32_t max_pages;             /* block-table columns                               */
  int32_t page_size;             /* rows per page, a power of two                     */
  int32_t num_pages;             /* pages in each pool; num_pages * page_size < 2^31  */
  int32_t flags;                 /* reserved, must be 0                               */
} sfa_kv_pages;

/* Top-k index producer (sfa_indexer_topk): creates the index rows sfa_fwd
 * consumes.  The reference takes them as an input (`topk_idxs`, "Sparse
 * indices mapping queries to KV blocks", SFA.py:88-90); the scores are those
 * of DeepSeek-V3.2's lightning indexer:
 *   I[b,t,s] = sum_h w[b,t,h] * max(0, <q[b,t,h,:], k[b,s,:]>)
 * Query t of sequence b may see keys s <= t + L_b - Sq (L_b = kv_lens[b]
 * clamped to Skv, else Skv): causal prefill when Sq = L_b, the whole context
 * for a single decode query.  Row idx[b,t,:] receives the min(topk, allowed)
 * allowed keys with the largest scores (equal scores: the lower key first),
 * in ascending key order, then -1 padding.
 * fp8 (SFA_DTYPE_FP8_E4M3) q / k, as DeepSeek-V3.2 stores them: the score is
 *   I[b,t,s] = k_scale[b,s] * sum_h w[b,t,h] * max(0, <q[b,t,h,:], k[b,s,:]>)
 * with positive per-token k scales (NULL = 1) and the q scales folded into w.
 * Supported: bf16 or fp8 q / k, D = 128, H in {32, 64, 128}, Skv <= 65536. */
typedef struct sfa_indexer_args {
  int32_t B, Sq, Skv, H, D, topk;
  int32_t dtype;                                  /* SFA_DTYPE_BF16 or SFA_DTYPE_FP8_E4M3      */
  const void* q;   int64_t q_sb, q_ss, q_sh;      /* [B, Sq, H, D], unit feature stride       */
  const void* k;   int64_t k_sb, k_ss;            /* [B, Skv, D], unit feature stride         */
  const float* k_scale; int64_t ks_sb;            /* fp8: [B, Skv] positive scales, or NULL   */
  const float* w;  int64_t w_sb, w_ss;            /* [B, Sq, H] float32, unit head stride     */
  const int32_t* kv_lens;                         /* [B] or NULL                              */
  int32_t* idx;    int64_t i_sb, i_ss;            /* [B, Sq, topk] int32 out, unit slot stride */
  float* logits;   int64_t g_sb, g_ss;            /* optional [B, Sq, Skv] float32 out (scores
                                                     of allowed keys; other entries unspecified;
                                                     16-byte aligned rows, g_ss % 4 == 0), or NULL */
  int32_t flags;                                  /* reserved, must be 0                       */
} sfa_indexer_args;

/* Library ABI version (SFA_ABI_VERSION of the build). */
SFA_API int sfa_abi_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
SFA_API const char* sfa_last_error(void);

/* Bytes of device workspace sfa_fwd needs for `a` (0 when none).
 * Replaces the per-launch workspaces of SFA.py:117-120; what remains: the
 * split-k partial results of the decode shape, and for the persistent MLA
 * prefill (>= 4096 work items) 256 bytes of work-claim counters plus, unless
 * SFA_FWD_IDX_SORTED is set, its index rows in ascending order
 * (B * Sq * Hkv * topk int32). */
SFA_API size_t sfa_fwd_workspace_size(const sfa_fwd_args* a);

/* Forward: out = softmax(scale * q k[idx]^T) v[idx], lse = log-sum-exp.
 * Replaces `_attn_fwd` (SFA.py:483-587 via SFA.py:122-159). */
SFA_API int sfa_fwd(const sfa_fwd_args* a, void* workspace, size_t workspace_bytes, void* stream);

/* Size of the static per-GPU scratch of sfa_fwd_noalloc (64 MiB). */
#define SFA_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* Forward that allocates nothing and takes no workspace: the same arguments,
 * kernels and results as sfa_fwd.  No counterpart in the reference; it is for
 * callers that cannot allocate device memory (code under HIP-graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The workspace of
 * sfa_fwd (sfa_fwd_workspace_size(a) bytes: decode split-k partials, prefill
 * claim counters and sorted index rows) goes to a static device
 * buffer of SFA_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds
 * until the process ends; a plan that needs more returns SFA_E_WORKSPACE
 * before any device work, except the prefill's sorted index rows: when they
 * do not fit, the rows are walked in their own order (the result then
 * equals sfa_fwd's with SFA_FWD_IDX_SORTED set; bitwise equal to sfa_fwd
 * whenever the sorted rows fit or the rows are already ascending).  `stream` must belong to the current device; the
 * first call on a device resolves the buffer's address (make it before any
 * graph capture).  All calls on one GPU share the buffer: calls that may
 * overlap on one GPU (unordered streams) race. */
SFA_API int sfa_fwd_noalloc(const sfa_fwd_args* a, void* stream);

/* Bytes of device workspace sfa_fwd_paged needs for `a` and `pages`. */
SFA_API size_t sfa_fwd_paged_workspace_size(const sfa_fwd_args* a, const sfa_kv_pages* pages);

/* Forward over a paged KV cache: the same result as sfa_fwd on the contiguous
 * cache the block table describes.  The reference has no paged variant (its
 * `_attn_fwd`, SFA.py:483-587, reads one contiguous [S_kv, B, D] kv tensor);
 * this is the serving-side layout of the decode step that precedes it. */
SFA_API int sfa_fwd_paged(const sfa_fwd_args* a, const sfa_kv_pages* pages, void* workspace,
                          size_t workspace_bytes, void* stream);

/* Bytes of device workspace sfa_indexer_topk needs: the fp32 scores of a
 * chunk of queries unless `logits` is given (about 1 GiB, less when all Sq
 * rows take less, more when one block of 512 / H queries of all B sequences
 * takes more), then, when a launch holds few long rows (B x queries < 256,
 * Skv >= 16384: a decode step), the candidate lists of its two-phase
 * selection (8 bytes per candidate, topk rounded up to 4 per segment, at
 * most 8 segments per row).  May be 0. */
SFA_API size_t sfa_indexer_topk_workspace_size(const sfa_indexer_args* a);

/* Scores and top-k selection (no counterpart kernel in the reference, which
 * consumes the result: SFA.py:88-90). */
SFA_API int sfa_indexer_topk(const sfa_indexer_args* a, void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of device workspace sfa_bwd needs for `a` (fp32 dK/dV accumulators,
 * delta, the CSR arrays in SFA_DKV_CSR mode).  The MLA backward
 * (SFA_BWD_MERGE_KV at its shape) needs fp32 accumulators of the shared rows
 * (B * Skv * Hkv * Dqk * 4 bytes), delta (B * Sq * Hq * 4 bytes) and one
 * chunk of queries: per query the bf16 P / dS of its slots (about 1 MiB at
 * top-k 2048, G = 128) and, in the deterministic mode, its per-slot bf16
 * gradient rows (top-k * Dqk * 2 bytes) and index maps; a chunk stays within
 * 3.5 GiB in the deterministic mode and 2 GiB with atomics (whole rounds of
 * 256 queries when that many fit, at most 1024 in the deterministic mode,
 * else multiples of 8, at least 8 queries).  The deterministic mode holds
 * the gradient rows and index maps twice (one chunk's reduction reads one
 * set while the next chunk fills the other), so the total is about 5.5 GiB
 * (2 GiB with atomics) plus the accumulators at the full-size shapes.
 * Replaces the workspaces of SFA.py:184-194 and SFA.py:253-261. */
SFA_API size_t sfa_bwd_workspace_size(const sfa_bwd_args* a);

/* Backward: dq, dk, dv (and dsink if requested) from dout, out and lse.
 * Replaces `_attn_bwd_dq_dsink` (SFA.py:856-1002 via SFA.py:199-251) and
 * `_attn_bwd_dk_dv` (SFA.py:1005-1145 via SFA.py:266-298).  dq/dk/dv are
 * fully overwritten (no accumulation into existing contents).  The
 * deterministic MLA backward also enqueues its ordered reductions on a
 * second stream of the device `stream` belongs to (the current device for
 * the null stream), which the library creates on its first such call there
 * (default priority, non-blocking, kept until the process ends) and orders
 * against `stream` with events: when the call returns,
 * `stream` waits for all of that work, and under HIP-graph capture the
 * second stream joins the capture and is joined back.  Such calls on one
 * device enqueue one at a time (a mutex). */
SFA_API int sfa_bwd(const sfa_bwd_args* a, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SFA_H_ */

// C ABI of libsfa.so (declared in include/sfa.h): argument validation,
// workspace sizing and kernel dispatch.  The library never allocates device
// memory, frees or synchronises; all work goes onto the caller's stream,
// except the deterministic MLA backward's reductions, which run on a second
// stream of the device ordered against it by events (MlaSide below).

#include <math.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "sfa_common.h"

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

int hip_fail(hipError_t e, const char* what) {
  return fail(SFA_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

constexpr int kMaxHeadDim = 1024;
constexpr int kGenericMaxTopk = 12288;  // scores of one row stay in 64 KiB of LDS

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Validation shared by forward and backward (SFA.py:52-53, 63-64 raise
// ValueError for an empty or non-positive top-k; this boundary also checks
// everything the kernels assume).
int check_fwd(const sfa_fwd_args* a) {
  if (a == nullptr) return fail(SFA_E_INVALID, "null argument struct");
  if (a->dtype != SFA_DTYPE_F32 && a->dtype != SFA_DTYPE_BF16) return fail(SFA_E_INVALID, "unknown dtype %d", a->dtype);
  if (a->B <= 0 || a->Sq <= 0 || a->Skv <= 0 || a->Hq <= 0 || a->Hkv <= 0)
    return fail(SFA_E_INVALID, "B, Sq, Skv, Hq, Hkv must be positive");
  if (a->topk <= 0) return fail(SFA_E_INVALID, "topk must be positive (got %d)", a->topk);
  if (a->Hq % a->Hkv != 0) return fail(SFA_E_INVALID, "Hq (%d) must be a multiple of Hkv (%d)", a->Hq, a->Hkv);
  if (a->Dqk <= 0 || a->Dv <= 0 || a->Dqk > kMaxHeadDim || a->Dv > kMaxHeadDim)
    return fail(SFA_E_INVALID, "head dims must be in [1, %d]", kMaxHeadDim);
  if (!a->q || !a->k || !a->v || !a->idx || !a->out || !a->lse) return fail(SFA_E_INVALID, "null tensor pointer");
  if ((a->flags & ~SFA_FWD_IDX_SORTED) != 0) return fail(SFA_E_INVALID, "unknown flags 0x%x", (unsigned)a->flags);
  if (a->num_splits < 0) return fail(SFA_E_INVALID, "num_splits must be >= 0");
  if (!(a->scale == a->scale) || isinf(a->scale)) return fail(SFA_E_INVALID, "scale must be finite");
  return SFA_OK;
}

// Page-table checks of sfa_fwd_paged (after check_fwd).
int check_pages(const sfa_fwd_args* a, const sfa_kv_pages* pg) {
  if (pg == nullptr || pg->block_table == nullptr) return fail(SFA_E_INVALID, "null page table");
  if (pg->flags != 0) return fail(SFA_E_INVALID, "page table flags must be 0");
  if (pg->page_size <= 0 || (pg->page_size & (pg->page_size - 1)) != 0)
    return fail(SFA_E_INVALID, "page_size must be a power of two (got %d)", pg->page_size);
  if (pg->max_pages <= 0 || pg->num_pages <= 0) return fail(SFA_E_INVALID, "max_pages and num_pages must be positive");
  if ((int64_t)pg->num_pages * pg->page_size > INT32_MAX)
    return fail(SFA_E_INVALID, "num_pages * page_size must stay below 2^31");
  if (a->B > 1 && pg->bt_sb < pg->max_pages)
    return fail(SFA_E_INVALID, "block-table row stride %lld is below max_pages %d", (long long)pg->bt_sb,
                pg->max_pages);
  if ((int64_t)a->Skv > (int64_t)pg->max_pages * pg->page_size)
    return fail(SFA_E_INVALID, "Skv %d exceeds max_pages * page_size", a->Skv);
  if (4 * ((int64_t)(a->B - 1) * pg->bt_sb + pg->max_pages) >= ((int64_t)1 << 32))
    return fail(SFA_E_INVALID, "block table spans 4 GiB or more");
  return SFA_OK;
}

sfa::Params to_params(const sfa_fwd_args* a, const sfa_kv_pages* pg = nullptr) {
  sfa::Params p;
  memset(&p, 0, sizeof(p));
  if (pg != nullptr) {
    p.block_table = pg->block_table;
    p.bt_sb = pg->bt_sb;
    p.page_shift = __builtin_ctz((unsigned)pg->page_size);
    p.num_pages = pg->num_pages;
    p.pool_shift = sfa::pool_unit_shift(2 * a->k_sb, 2 * a->k_ss);
  }
  p.q = a->q; p.k = a->k; p.v = a->v; p.idx = a->idx; p.kv_lens = a->kv_lens; p.sink = a->sink;
  p.out = a->out; p.lse = a->lse;
  p.q_sb = a->q_sb; p.q_ss = a->q_ss; p.q_sh = a->q_sh;
  p.k_sb = a->k_sb; p.k_ss = a->k_ss; p.k_sh = a->k_sh;
  p.v_sb = a->v_sb; p.v_ss = a->v_ss; p.v_sh = a->v_sh;
  p.i_sb = a->i_sb; p.i_ss = a->i_ss; p.i_sh = a->i_sh;
  p.o_sb = a->o_sb; p.o_ss = a->o_ss; p.o_sh = a->o_sh;
  p.l_sb = a->l_sb; p.l_ss = a->l_ss; p.l_sh = a->l_sh;
  p.B = a->B; p.Sq = a->Sq; p.Skv = a->Skv; p.Hq = a->Hq; p.Hkv = a->Hkv;
  p.Dqk = a->Dqk; p.Dv = a->Dv; p.topk = a->topk; p.G = a->Hq / a->Hkv;
  p.scale = a->scale > 0.f ? a->scale : 1.0f / sqrtf((float)a->Dqk);
  p.scale_log2 = p.scale * sfa::kLog2e;
  p.num_splits = 1;
  p.split_len = a->topk;
  return p;
}

// MFMA eligibility beyond the kernel-variant shape: 16-byte aligned rows.
bool mfma_layout_ok(const sfa_fwd_args* a) {
  if (a->dtype != SFA_DTYPE_BF16) return false;
  if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->out)) return false;
  const int64_t s[] = {a->q_sb, a->q_ss, a->q_sh, a->k_sb, a->k_ss, a->k_sh, a->v_sb, a->v_ss, a->v_sh,
                       a->o_sb, a->o_ss, a->o_sh};
  for (int64_t x : s)
    if (x % 8 != 0) return false;
  return true;
}

// MFMA backward eligibility beyond the kernel-variant shape: 16-byte aligned
// rows of q, k, v and dout, and 8-byte aligned dq rows.
bool bwd_mfma_ok(const sfa_bwd_args* a) {
  if (!mfma_layout_ok(&a->fwd)) return false;
  if (!aligned16(a->dout) || ((uintptr_t)a->dq & 7u) != 0) return false;
  const int64_t s[] = {a->do_sb, a->do_ss, a->do_sh, a->dq_sb, a->dq_ss, a->dq_sh};
  for (int64_t x : s)
    if (x % 8 != 0) return false;
  return true;
}

struct FwdPlan {
  bool mfma;
  int num_splits;
  int split_len;
  size_t part_o_bytes;
  size_t part_lse_bytes;
  size_t sched_bytes;  // claim counters of the persistent forward (0 when not persistent)
  size_t sort_bytes;   // the index rows in ascending key order (0 when not sorted)
  size_t workspace() const { return part_o_bytes + part_lse_bytes + sched_bytes + sort_bytes; }
};

constexpr int kTargetWorkgroups = 512;  // 2 per CU on a 256-CU MI355X
constexpr int kMaxSplits = 64;  // the combine kernel holds one split per lane of a wave

// sort_room: the most workspace bytes the sorted index rows may take
// (sfa_fwd_noalloc: what its static scratch leaves); rows that do not fit
// are used in their own order.
FwdPlan plan_fwd(const sfa_fwd_args* a, const sfa_kv_pages* pg, size_t sort_room = SIZE_MAX) {
  FwdPlan pl{};
  sfa::Params p = to_params(a, pg);
  pl.mfma = mfma_layout_ok(a) && sfa::fwd_mfma_supported(p);
  const int idx_cap = pl.mfma ? sfa::fwd_mfma_idx_cap(p) : 1;
  pl.mfma = pl.mfma && (a->topk + idx_cap - 1) / idx_cap <= kMaxSplits;
  int splits = 1;
  if (pl.mfma) {
    const int nk = sfa::fwd_mfma_tile_keys(p);
    // workgroups before the split: work items times head groups
    const int64_t items = (int64_t)a->B * a->Sq * a->Hkv * sfa::fwd_mfma_head_groups(p);
    if (a->num_splits > 0) {
      splits = a->num_splits;
    } else if (items < kTargetWorkgroups / 2) {
      // decode-like: too few work items to fill the chip -> split the top-k set
      splits = (int)((kTargetWorkgroups / 2 + items - 1) / items);
    }
    // each split must fit the staged index window and hold at least one tile
    const int min_splits = (a->topk + idx_cap - 1) / idx_cap;
    if (splits < min_splits) splits = min_splits;
    int max_splits = (a->topk + nk - 1) / nk;
    if (splits > max_splits) splits = max_splits;
    if (splits > kMaxSplits) splits = kMaxSplits;
    if (splits < 1) splits = 1;
    int len = (a->topk + splits - 1) / splits;
    len = (len + nk - 1) / nk * nk;
    splits = (a->topk + len - 1) / len;
    pl.split_len = len;
  } else {
    if (a->num_splits > 1) splits = 1;  // the generic kernel is not split
    pl.split_len = a->topk;
  }
  pl.num_splits = splits;
  if (splits > 1) {
    const size_t rows = (size_t)a->B * a->Sq * a->Hq;
    pl.part_o_bytes = align_up((size_t)splits * rows * a->Dv * sizeof(__bf16), 256);
    pl.part_lse_bytes = align_up((size_t)splits * rows * sizeof(float), 256);
  }
  if (pl.mfma) {
    p.num_splits = pl.num_splits;
    p.split_len = pl.split_len;
    if (sfa::fwd_mfma_persistent(p)) {
      pl.sched_bytes = 256;
      // the persistent MLA prefill walks ascending rows (L2 sharing between
      // the queries running together on an XCD); paged KV too (the rows hold
      // logical keys), so a paged call walks the same slots as a contiguous one
      if (!(a->flags & SFA_FWD_IDX_SORTED) && sfa::idx_sort_supported(p)) {
        const size_t bytes = align_up((size_t)a->B * a->Sq * a->Hkv * a->topk * sizeof(int32_t), 256);
        if (bytes + pl.sched_bytes <= sort_room) pl.sort_bytes = bytes;
      }
    }
  }
  return pl;
}

int check_generic_fwd(const sfa_fwd_args* a) {
  if (a->topk > kGenericMaxTopk)
    return fail(SFA_E_UNSUPPORTED, "topk %d exceeds %d for this head-dim / group / dtype combination", a->topk,
                kGenericMaxTopk);
  return SFA_OK;
}

// The forward of sfa_fwd (pg == nullptr) and sfa_fwd_paged, after validation.
int run_fwd(const sfa_fwd_args* a, const sfa_kv_pages* pg, void* workspace, size_t workspace_bytes, void* stream,
            size_t sort_room = SIZE_MAX) {
  hipStream_t s = (hipStream_t)stream;
  const FwdPlan pl = plan_fwd(a, pg, sort_room);
  sfa::Params p = to_params(a, pg);
  int rc;
  hipError_t e;
  if (pl.mfma) {
    p.num_splits = pl.num_splits;
    p.split_len = pl.split_len;
    if (pl.workspace() > 0 && (workspace == nullptr || workspace_bytes < pl.workspace()))
      return fail(SFA_E_WORKSPACE, "sfa_fwd needs %zu workspace bytes (got %zu)", pl.workspace(), workspace_bytes);
    if (pl.num_splits > 1) {
      p.part_o = (__bf16*)workspace;
      p.part_lse = (float*)((char*)workspace + pl.part_o_bytes);
    }
    if (pl.sched_bytes > 0) p.sched = (int*)((char*)workspace + pl.part_o_bytes + pl.part_lse_bytes);
    if (pl.sort_bytes > 0) {
      int32_t* sorted = (int32_t*)((char*)workspace + pl.part_o_bytes + pl.part_lse_bytes + pl.sched_bytes);
      e = sfa::launch_idx_sort(p, sorted, s);
      if (e != hipSuccess) return hip_fail(e, "sfa_fwd (index sort)");
      p.idx = sorted;
      p.i_sh = a->topk;
      p.i_ss = (int64_t)a->Hkv * a->topk;
      p.i_sb = (int64_t)a->Sq * a->Hkv * a->topk;
    }
    e = sfa::launch_fwd_mfma(p, s);
    if (e != hipSuccess) return hip_fail(e, "sfa_fwd (mfma)");
    if (pl.num_splits > 1) {
      e = sfa::launch_combine(p, a->dtype, s);
      if (e != hipSuccess) return hip_fail(e, "sfa_fwd (combine)");
    }
    return SFA_OK;
  }
  rc = check_generic_fwd(a);
  if (rc != SFA_OK) return rc;
  e = sfa::launch_fwd_generic(p, a->dtype, s);
  if (e != hipSuccess) return hip_fail(e, "sfa_fwd (generic)");
  return SFA_OK;
}

}  // namespace

extern "C" {

int sfa_abi_version(void) { return SFA_ABI_VERSION; }

const char* sfa_last_error(void) { return g_err; }

size_t sfa_fwd_workspace_size(const sfa_fwd_args* a) {
  if (check_fwd(a) != SFA_OK) return 0;
  const FwdPlan pl = plan_fwd(a, nullptr);
  return pl.workspace();
}

int sfa_fwd(const sfa_fwd_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  const int rc = check_fwd(a);
  if (rc != SFA_OK) return rc;
  return run_fwd(a, nullptr, workspace, workspace_bytes, stream);
}

}  // extern "C"

namespace {

// ---- sfa_fwd_noalloc: the split-k partials in a static device buffer ----
// One copy of `scratch` per GPU (each device that loads the library holds it
// until the process ends).  In host code `scratch` only names the variable:
// its device address is resolved once per device with hipGetSymbolAddress
// (with that device current) and cached; kernels get that address.
constexpr size_t kNoallocBytes = SFA_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kNoallocBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the device `stream` belongs to, which must
// be the current device.
int noalloc_scratch(void* stream, void** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return hip_fail(e, "sfa_fwd_noalloc: hipGetDevice");
  int dev = cur;
  if (stream != nullptr) {
    e = hipStreamGetDevice((hipStream_t)stream, &dev);
    if (e != hipSuccess) return hip_fail(e, "sfa_fwd_noalloc: hipStreamGetDevice");
  }
  if (dev != cur) return fail(SFA_E_INVALID, "sfa_fwd_noalloc: the stream belongs to device %d, device %d is current", dev, cur);
  if (dev < 0 || dev >= kMaxDevices) return fail(SFA_E_UNSUPPORTED, "sfa_fwd_noalloc: device %d >= %d", dev, kMaxDevices);
  void* ptr = g_scratch[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return hip_fail(e, "sfa_fwd_noalloc: hipGetSymbolAddress(scratch)");
      if (ptr == nullptr) return fail(SFA_E_HIP, "sfa_fwd_noalloc: null scratch address");
      g_scratch[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return SFA_OK;
}

}  // namespace

extern "C" {

int sfa_fwd_noalloc(const sfa_fwd_args* a, void* stream) {
  g_err[0] = 0;
  const int rc = check_fwd(a);
  if (rc != SFA_OK) return rc;
  // (index rows whose sorted copy does not fit the scratch are used in their
  // own order)
  const FwdPlan pl = plan_fwd(a, nullptr, kNoallocBytes);
  const size_t need = pl.workspace();
  if (need > kNoallocBytes)
    return fail(SFA_E_WORKSPACE,
                "sfa_fwd_noalloc: the split-k partials need %zu bytes, above its static scratch of %zu bytes "
                "(use sfa_fwd with a workspace, or fewer splits)",
                need, kNoallocBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int r = noalloc_scratch(stream, &ws);
    if (r != SFA_OK) return r;
  }
  return run_fwd(a, nullptr, ws, need > 0 ? kNoallocBytes : 0, stream, kNoallocBytes);
}

size_t sfa_fwd_paged_workspace_size(const sfa_fwd_args* a, const sfa_kv_pages* pages) {
  if (check_fwd(a) != SFA_OK || check_pages(a, pages) != SFA_OK) return 0;
  const FwdPlan pl = plan_fwd(a, pages);
  return pl.workspace();
}

int sfa_fwd_paged(const sfa_fwd_args* a, const sfa_kv_pages* pages, void* workspace, size_t workspace_bytes,
                  void* stream) {
  g_err[0] = 0;
  int rc = check_fwd(a);
  if (rc == SFA_OK) rc = check_pages(a, pages);
  if (rc != SFA_OK) return rc;
  return run_fwd(a, pages, workspace, workspace_bytes, stream);
}

}  // extern "C"

namespace {

// AUTO takes the deterministic scheme only where it is also the cheaper one.
// Its key-major pass evaluates every pair of a non-empty (query block, key
// block): for causal top-k rows about (mean key range / top-k) times the
// selected pairs, and its fp32 partials grow as Skv * Sq * G / 16 bytes per
// (batch, kv head).  Measured on the GQA training shape (Skv = 8192,
// top-k 1024: ~4x dense pairs) it is 4.7x faster than the atomics; the
// per-pair costs put the crossover near 30x dense pairs.  Rules:
constexpr int64_t kCsrMaxKeysPerTopk = 64;        // Skv <= 64 * top-k (<= ~32x dense pairs causally)
constexpr size_t kCsrMaxWorkspace = size_t(4) << 30;  // CSR arrays + partials <= 4 GiB

// dK/dV scheme actually used: CSR (deterministic) when requested or, for
// AUTO, when the shape has the key-major kernel and passes the rules above;
// otherwise atomics.
bool use_csr(const sfa_bwd_args* a, sfa::Params p) {
  if (a->dkv_mode == SFA_DKV_ATOMIC) return false;
  p.do_sb = a->do_sb;  // (the range checks also cover dout)
  p.do_ss = a->do_ss;
  p.do_sh = a->do_sh;
  // the deterministic scheme pairs the key-major dK/dV with the dQ kernel,
  // which adds only the repeated-key slots' dK/dV
  if (!(bwd_mfma_ok(a) && sfa::bwd_csr_supported(p) && sfa::bwd_dq_supported(p))) return false;
  if (a->dkv_mode == SFA_DKV_CSR) return true;
  if ((int64_t)p.Skv > kCsrMaxKeysPerTopk * p.topk) return false;
  sfa::csr_geometry(p);
  return sfa::csr_workspace_bytes(p) <= kCsrMaxWorkspace;
}

size_t bwd_base_bytes(const sfa_fwd_args& f) {
  const size_t dk = align_up((size_t)f.B * f.Skv * f.Hkv * f.Dqk * sizeof(float), 256);
  const size_t dv = align_up((size_t)f.B * f.Skv * f.Hkv * f.Dv * sizeof(float), 256);
  const size_t delta = align_up((size_t)f.B * f.Sq * f.Hq * sizeof(float), 256);
  return dk + dv + delta;
}

bool merge_kv(const sfa_bwd_args* a) { return (a->flags & SFA_BWD_MERGE_KV) != 0; }

// The MLA shared-KV backward: merged gradient, bf16 MFMA layout, MLA shape.
bool use_mla(const sfa_bwd_args* a, const sfa::Params& p) {
  if (!(merge_kv(a) && bwd_mfma_ok(a) && sfa::bwd_mla_supported(p))) return false;
  // the dK/dV pass stages the query's G head rows of q and dout through
  // 32-bit buffer offsets
  const int64_t lim = (int64_t)0x80000000LL;
  return (int64_t)(p.G - 1) * 2 * a->fwd.q_sh + 2 * 576 < lim && (int64_t)(p.G - 1) * 2 * a->do_sh + 2 * 512 < lim;
}

// Its deterministic dK/dV (index maps + ordered reduction of bf16 per-slot
// rows) is used unless atomics are asked for or Skv exceeds its bitmap.
bool mla_det(const sfa_bwd_args* a, const sfa::Params& p) {
  return a->dkv_mode != SFA_DKV_ATOMIC && sfa::bwd_mla_det_supported(p);
}

// Its workspace holds one chunk of work items (P / dS, and the contribution
// rows and index maps when deterministic, those twice): a chunk is sized to
// about 3.5 GiB deterministic (1024 queries at top-k 2048, 3.4 MB each:
// every chunk costs a fixed ~40 us of launches and reduction set-up, so 32
// chunks of 1024 run 2.7 % faster than 64 of 512 at S = 32768) or 2 GiB with
// atomics (larger chunks gain nothing there), in whole rounds of 256 items (one dK/dV workgroup per CU of the
// 256-CU part; a partial last round would leave most CUs idle), at least 8
// items so the dQ pass can place both head groups of an item on one XCD.
constexpr size_t kMlaChunkBytesDet = size_t(3584) << 20;
constexpr size_t kMlaChunkBytes = size_t(2) << 30;
constexpr int64_t kMlaChunkRound = 256;

int mla_chunk_items(const sfa::Params& p, bool det) {
  const int64_t items = (int64_t)p.B * p.Sq * p.Hkv;
  int64_t n = (int64_t)((det ? kMlaChunkBytesDet : kMlaChunkBytes) / sfa::bwd_mla_bytes_per_item(p, det));
  n = n >= kMlaChunkRound ? n / kMlaChunkRound * kMlaChunkRound : (n / 8 * 8 > 8 ? n / 8 * 8 : 8);
  const int64_t cap = sfa::bwd_mla_max_chunk_items(det);  // a multiple of kMlaChunkRound
  if (n > cap) n = cap;
  return (int)(n < items ? n : items);
}

// MLA workspace: fp32 shared-row accumulators | delta | P / dS of a chunk |
// (det) two buffer sets, so that chunk c + 1's dK/dV pass can fill one while
// chunk c's reduction reads the other
size_t mla_bytes(const sfa_fwd_args& f, const sfa::Params& p, bool det) {
  const size_t dk = align_up((size_t)f.B * f.Skv * f.Hkv * f.Dqk * sizeof(float), 256);
  const size_t delta = align_up((size_t)f.B * f.Sq * f.Hq * sizeof(float), 256);
  const size_t n = (size_t)mla_chunk_items(p, det);
  size_t bytes = dk + delta + align_up(n * sfa::bwd_mla_pd_bytes_per_item(p), 256);
  if (det) bytes += 2 * align_up(n * sfa::bwd_mla_set_bytes_per_item(p), 256);
  return bytes;
}

// The deterministic MLA backward's reductions (and the index maps of the
// chunk two ahead) run on a second stream of the device (default priority,
// non-blocking), ordered against the caller's stream by events, so that
// chunk c's reduction (HBM-bound) overlaps chunk c + 1's dQ pass (MFMA- and
// LDS-bound).  One per device, created on first
// use and kept until the process ends; calls on one device enqueue under its
// mutex, so each call's fork and join of the side stream stay together
// (also under HIP-graph capture: the side stream joins the caller's capture
// through the first event and is joined back before the call returns).
struct MlaSide {
  std::mutex mu;
  bool ready = false;
  hipStream_t st = nullptr;
  hipEvent_t dkv_done = nullptr;
  hipEvent_t map_done[2] = {nullptr, nullptr};
  hipEvent_t done = nullptr;
  int cus = 0;
};
MlaSide g_side[kMaxDevices];

// (dev: the device of the caller's stream, which need not be the current
// one; the stream and events are created with dev current, as they must be
// to order work on dev's streams)
hipError_t mla_side_init(MlaSide& m, int dev) {
  if (m.ready) return hipSuccess;
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
  if (e != hipSuccess) return e;
  e = hipDeviceGetAttribute(&m.cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess && m.st == nullptr) e = hipStreamCreateWithFlags(&m.st, hipStreamNonBlocking);
  if (e == hipSuccess && m.dkv_done == nullptr) e = hipEventCreateWithFlags(&m.dkv_done, hipEventDisableTiming);
  if (e == hipSuccess && m.done == nullptr) e = hipEventCreateWithFlags(&m.done, hipEventDisableTiming);
  for (int i = 0; i < 2 && e == hipSuccess; ++i)
    if (m.map_done[i] == nullptr) e = hipEventCreateWithFlags(&m.map_done[i], hipEventDisableTiming);
  if (e == hipSuccess) m.ready = true;
  if (cur != dev) {
    const hipError_t er = hipSetDevice(cur);
    if (e == hipSuccess) e = er;
  }
  return e;
}

}  // namespace

extern "C" {

size_t sfa_bwd_workspace_size(const sfa_bwd_args* a) {
  if (a == nullptr || check_fwd(&a->fwd) != SFA_OK) return 0;
  sfa::Params p = to_params(&a->fwd);
  if (use_mla(a, p)) return mla_bytes(a->fwd, p, mla_det(a, p));
  size_t n = bwd_base_bytes(a->fwd);
  if (use_csr(a, p)) {
    sfa::csr_geometry(p);
    n += sfa::csr_workspace_bytes(p);
  }
  return n;
}

int sfa_bwd(const sfa_bwd_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  if (a == nullptr) return fail(SFA_E_INVALID, "null argument struct");
  int rc = check_fwd(&a->fwd);
  if (rc != SFA_OK) return rc;
  const sfa_fwd_args& f = a->fwd;
  if ((a->flags & ~SFA_BWD_MERGE_KV) != 0) return fail(SFA_E_INVALID, "unknown flags 0x%x", (unsigned)a->flags);
  const bool merge = merge_kv(a);
  if (!a->dout || !a->dq || !a->dk || (!merge && !a->dv)) return fail(SFA_E_INVALID, "null gradient pointer");
  if (f.sink && !a->dsink) return fail(SFA_E_INVALID, "dsink is required when sink is given");
  if (merge && !(f.v == f.k && f.v_sb == f.k_sb && f.v_ss == f.k_ss && f.v_sh == f.k_sh && f.Dv <= f.Dqk))
    return fail(SFA_E_INVALID, "SFA_BWD_MERGE_KV needs v to be the first Dv dims of k's rows");
  if (a->dkv_mode != SFA_DKV_AUTO && a->dkv_mode != SFA_DKV_ATOMIC && a->dkv_mode != SFA_DKV_CSR)
    return fail(SFA_E_INVALID, "unknown dkv_mode %d", a->dkv_mode);
  const size_t need = sfa_bwd_workspace_size(a);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(SFA_E_WORKSPACE, "sfa_bwd needs %zu workspace bytes (got %zu)", need, workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  sfa::Params p = to_params(&f);
  if (use_mla(a, p)) {
    p.dout = a->dout; p.do_sb = a->do_sb; p.do_ss = a->do_ss; p.do_sh = a->do_sh;
    p.dq = a->dq; p.dq_sb = a->dq_sb; p.dq_ss = a->dq_ss; p.dq_sh = a->dq_sh;
    const size_t nk = (size_t)f.B * f.Skv * f.Hkv * f.Dqk;
    p.dk_acc = (float*)workspace;
    p.delta = (float*)((char*)workspace + align_up(nk * sizeof(float), 256));
    void* pd = (char*)p.delta + align_up((size_t)f.B * f.Sq * f.Hq * sizeof(float), 256);
    p.dsink = a->dsink;
    p.dlse = a->dlse;
    // (refused before any device work is queued)
    const bool det = mla_det(a, p);
    if (a->dkv_mode == SFA_DKV_CSR && !det)
      return fail(SFA_E_UNSUPPORTED, "the deterministic MLA backward supports Skv <= 65536 (got %d)", f.Skv);
    // (δ is computed by the chunks' dQ passes, which load O and dO rows anyway;
    // the sink's gradient, which needs every row's δ, follows the last chunk)
    const int64_t items = (int64_t)f.B * f.Sq * f.Hkv;
    const int chunk = mla_chunk_items(p, det);
    void* sets[2] = {nullptr, nullptr};
    MlaSide* side = nullptr;
    std::unique_lock<std::mutex> lock;
    if (det) {
      // the device the caller's stream belongs to (the current one for the
      // null stream): the reductions must run there
      int dev = 0;
      hipError_t e0 = s != nullptr ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
      if (e0 == hipSuccess && (dev < 0 || dev >= kMaxDevices)) e0 = hipErrorInvalidDevice;
      if (e0 == hipSuccess) {
        side = &g_side[dev];
        lock = std::unique_lock<std::mutex>(side->mu);
        e0 = mla_side_init(*side, dev);
      }
      if (e0 != hipSuccess) return hip_fail(e0, "sfa_bwd (mla): the reduction stream");
      const size_t set_bytes = align_up((size_t)chunk * sfa::bwd_mla_set_bytes_per_item(p), 256);
      sets[0] = (char*)pd + align_up((size_t)chunk * sfa::bwd_mla_pd_bytes_per_item(p), 256);
      sets[1] = (char*)sets[0] + set_bytes;
    }
    const int nchunks = (int)((items + chunk - 1) / chunk);
    auto chunk_len = [&](int c) { return (int)(items - (int64_t)c * chunk < chunk ? items - (int64_t)c * chunk : chunk); };
    hipError_t e = sfa::launch_zero_f32(p.dk_acc, nk, s);
    // det: the index maps of chunks 0 and 1 first; chunk c + 2's are built on
    // the side stream right after chunk c's reduction, in the buffer set that
    // reduction frees, so only the dK/dV pass waits for them
    for (int c = 0; det && c < 2 && c < nchunks && e == hipSuccess; ++c)
      e = sfa::launch_bwd_mla_map(p, (int64_t)c * chunk, chunk_len(c), sets[c & 1], s);
    bool forked = false;
    for (int c = 0; e == hipSuccess && c < nchunks; ++c) {
      const int64_t i0 = (int64_t)c * chunk;
      const int n = chunk_len(c);
      e = sfa::launch_bwd_mla_dq(p, i0, n, pd, s);
      if (det && c >= 2 && e == hipSuccess) e = hipStreamWaitEvent(s, side->map_done[c & 1], 0);
      if (e == hipSuccess) e = sfa::launch_bwd_mla_dkv(p, i0, n, pd, sets[c & 1], det, s);
      if (det && e == hipSuccess) {
        e = hipEventRecord(side->dkv_done, s);
        if (e == hipSuccess) e = hipStreamWaitEvent(side->st, side->dkv_done, 0);
        forked = forked || e == hipSuccess;
        if (e == hipSuccess) e = sfa::launch_bwd_mla_reduce(p, i0, n, sets[c & 1], side->cus, side->st);
        if (e == hipSuccess && c + 2 < nchunks) {
          e = sfa::launch_bwd_mla_map(p, i0 + 2 * (int64_t)chunk, chunk_len(c + 2), sets[c & 1], side->st);
          if (e == hipSuccess) e = hipEventRecord(side->map_done[c & 1], side->st);
        }
      }
    }
    // join: everything the side stream ran (in order)
    if (forked) {
      hipError_t ej = hipEventRecord(side->done, side->st);
      if (ej == hipSuccess) ej = hipStreamWaitEvent(s, side->done, 0);
      if (e == hipSuccess) e = ej;
    }
    if (e == hipSuccess) e = sfa::launch_bwd_dsink(p, s);
    if (e == hipSuccess) e = sfa::launch_bwd_finish_merged(p, f.dtype, a->dk, a->dk_sb, a->dk_ss, a->dk_sh, false, s);
    if (e != hipSuccess) return hip_fail(e, "sfa_bwd (mla)");
    return SFA_OK;
  }
  const bool csr = use_csr(a, p);
  if (a->dkv_mode == SFA_DKV_CSR && !csr)
    return fail(SFA_E_UNSUPPORTED,
                "SFA_DKV_CSR needs bf16, d_qk = d_v = 128, G a power of two <= 128, top-k <= 2048, "
                "Skv <= 262144 and row offsets below 2^31 bytes");
  if (!(bwd_mfma_ok(a) && sfa::bwd_mfma_supported(p)) && f.topk > kGenericMaxTopk)
    return fail(SFA_E_UNSUPPORTED, "topk %d exceeds %d", f.topk, kGenericMaxTopk);
  p.dout = a->dout; p.do_sb = a->do_sb; p.do_ss = a->do_ss; p.do_sh = a->do_sh;
  p.dq = a->dq; p.dq_sb = a->dq_sb; p.dq_ss = a->dq_ss; p.dq_sh = a->dq_sh;
  const size_t nk = (size_t)f.B * f.Skv * f.Hkv * f.Dqk, nv = (size_t)f.B * f.Skv * f.Hkv * f.Dv;
  p.dk_acc = (float*)workspace;
  p.dv_acc = (float*)((char*)workspace + align_up(nk * sizeof(float), 256));
  p.delta = (float*)((char*)p.dv_acc + align_up(nv * sizeof(float), 256));
  p.dsink = a->dsink;
  p.dlse = a->dlse;
  if (csr) {
    sfa::csr_geometry(p);
    sfa::csr_bind_workspace(p, (char*)workspace + bwd_base_bytes(f));
  }

  hipError_t e = sfa::launch_zero_f32(p.dk_acc, nk, s);
  if (e == hipSuccess) e = sfa::launch_zero_f32(p.dv_acc, nv, s);
  if (e == hipSuccess) e = sfa::launch_bwd_delta(p, f.dtype, s);
  if (e == hipSuccess) e = sfa::launch_bwd_dsink(p, s);
  if (e == hipSuccess && csr) e = sfa::launch_csr_index(p, s);  // before dQ: it reads the repeat flags
  if (e == hipSuccess && csr) {
    e = sfa::launch_bwd_dq(p, s);
    if (e == hipSuccess) e = sfa::launch_csr_dkv(p, s);
    // (after the ordered dK/dV reduction, which adds into the same
    // accumulators without atomics)
    if (e == hipSuccess) e = sfa::launch_bwd_dup(p, s);
  } else if (e == hipSuccess) {
    if (bwd_mfma_ok(a) && sfa::bwd_mfma_supported(p))
      e = sfa::launch_bwd_mfma(p, s);
    else
      e = sfa::launch_bwd_generic(p, f.dtype, s);
  }
  if (e == hipSuccess) {
    if (merge)
      e = sfa::launch_bwd_finish_merged(p, f.dtype, a->dk, a->dk_sb, a->dk_ss, a->dk_sh, true, s);
    else
      e = sfa::launch_bwd_finish(p, f.dtype, a->dk, a->dk_sb, a->dk_ss, a->dk_sh, a->dv, a->dv_sb, a->dv_ss,
                                 a->dv_sh, s);
  }
  if (e != hipSuccess) return hip_fail(e, "sfa_bwd");
  return SFA_OK;
}

}  // extern "C"

namespace {

// Scores are produced and consumed a chunk of queries at a time, so the
// workspace stays bounded (about 1 GiB) whatever Sq and Skv are.  A chunk of
// 8192 queries of 32768 keys gives the scores kernel 1024 query blocks of 8
// for its 512 resident slots, enough for its heaviest-first order to even out
// the causal rows (a 512 MiB chunk, one block per slot, ran 5 % slower).
constexpr size_t kIndexerChunkBytes = size_t(1024) << 20;
constexpr int kIndexerMaxSkv = 65536;

int check_indexer(const sfa_indexer_args* a) {
  if (a == nullptr) return fail(SFA_E_INVALID, "null argument struct");
  if (a->B <= 0 || a->Sq <= 0 || a->Skv <= 0 || a->H <= 0 || a->D <= 0)
    return fail(SFA_E_INVALID, "B, Sq, Skv, H, D must be positive");
  if (a->topk <= 0) return fail(SFA_E_INVALID, "topk must be positive (got %d)", a->topk);
  if (!a->q || !a->k || !a->w || !a->idx) return fail(SFA_E_INVALID, "null tensor pointer");
  if (a->flags != 0) return fail(SFA_E_INVALID, "flags must be 0");
  if (a->dtype != SFA_DTYPE_BF16 && a->dtype != SFA_DTYPE_FP8_E4M3)
    return fail(SFA_E_INVALID, "indexer dtype must be SFA_DTYPE_BF16 or SFA_DTYPE_FP8_E4M3 (got %d)", a->dtype);
  if (a->k_scale && a->dtype != SFA_DTYPE_FP8_E4M3) return fail(SFA_E_INVALID, "k_scale is for fp8 keys only");
  if (a->D != 128 || (a->H != 32 && a->H != 64 && a->H != 128))
    return fail(SFA_E_UNSUPPORTED, "the indexer supports D = 128 and H in {32, 64, 128} (got D = %d, H = %d)", a->D,
                a->H);
  if (a->Skv > kIndexerMaxSkv) return fail(SFA_E_UNSUPPORTED, "the indexer supports Skv <= %d", kIndexerMaxSkv);
  if (!aligned16(a->q) || !aligned16(a->k)) return fail(SFA_E_INVALID, "q and k rows must be 16-byte aligned");
  const int64_t esize = a->dtype == SFA_DTYPE_FP8_E4M3 ? 1 : 2;
  const int64_t st[] = {a->q_sb, a->q_ss, a->q_sh, a->k_sb, a->k_ss};
  for (int64_t x : st)
    if ((x * esize) % 16 != 0) return fail(SFA_E_INVALID, "q / k strides must be multiples of 16 bytes");
  if (esize * ((int64_t)(a->Skv - 1) * a->k_ss + a->D) >= (int64_t)0x80000000LL)
    return fail(SFA_E_UNSUPPORTED, "k rows of one sequence must lie within 2 GiB");
  if (!sfa::fits_u24(esize * a->k_ss)) return fail(SFA_E_UNSUPPORTED, "the k row stride must be below 16 MiB");
  if (a->logits) {
    if (!aligned16(a->logits) || a->g_ss % 4 != 0 || a->g_sb % 4 != 0 || a->g_ss < a->Skv)
      return fail(SFA_E_INVALID, "logits rows must be 16-byte aligned with a row stride >= Skv, multiple of 4");
  }
  return SFA_OK;
}

sfa::IndexerParams to_iparams(const sfa_indexer_args* a) {
  sfa::IndexerParams p;
  memset(&p, 0, sizeof(p));
  p.q = a->q; p.k = a->k; p.w = a->w; p.kv_lens = a->kv_lens; p.idx = a->idx; p.logits = a->logits;
  p.k_scale = a->k_scale; p.ks_sb = a->ks_sb; p.fp8 = a->dtype == SFA_DTYPE_FP8_E4M3;
  p.q_sb = a->q_sb; p.q_ss = a->q_ss; p.q_sh = a->q_sh;
  p.k_sb = a->k_sb; p.k_ss = a->k_ss;
  p.w_sb = a->w_sb; p.w_ss = a->w_ss;
  p.i_sb = a->i_sb; p.i_ss = a->i_ss;
  p.g_sb = a->g_sb; p.g_ss = a->g_ss;
  p.B = a->B; p.Sq = a->Sq; p.Skv = a->Skv; p.H = a->H; p.D = a->D; p.topk = a->topk;
  return p;
}

// Queries per chunk (a multiple of the logits kernel's query block) and the
// score row stride of the workspace.
void indexer_chunk(const sfa_indexer_args* a, int* rows, int64_t* ld) {
  const sfa::IndexerParams p = to_iparams(a);
  const int qb = sfa::indexer_query_block(p);
  *ld = (int64_t)(a->Skv + 31) / 32 * 32;
  int64_t r = (int64_t)(kIndexerChunkBytes / ((size_t)a->B * (size_t)*ld * sizeof(float)));
  r = r / qb * qb;
  if (r < qb) r = qb;
  // (chunks start on query-block boundaries; one chunk when all Sq rows fit)
  *rows = (int)(r < a->Sq ? r : a->Sq);
}

// Queries per launch (all Sq when the caller holds the scores, else a chunk)
// and the workspace: the chunk's scores, then the candidate lists of a
// segmented selection (launches of few long rows), sized for the largest of
// the launches' plans.
struct IndexerPlan {
  int rows;
  int64_t ld;
  size_t score_bytes, cand_bytes;
};

IndexerPlan indexer_plan(const sfa_indexer_args* a) {
  IndexerPlan pl{a->Sq, 0, 0, 0};
  if (a->logits == nullptr) {
    indexer_chunk(a, &pl.rows, &pl.ld);
    pl.score_bytes = align_up((size_t)a->B * (size_t)pl.rows * (size_t)pl.ld * sizeof(float), 256);
  }
  const sfa::IndexerParams p = to_iparams(a);
  size_t cb = 0;
  const int first = pl.rows < a->Sq ? pl.rows : a->Sq;
  const int last = a->Sq % first ? a->Sq % first : first;
  for (int r : {first, last}) {
    const int nseg = sfa::topk_segments(p, r);
    if (nseg > 1)
      cb = std::max(cb, (size_t)a->B * (size_t)r * (size_t)nseg * (size_t)((a->topk + 3) / 4 * 4) * sizeof(int32_t));
  }
  pl.cand_bytes = 2 * align_up(cb, 256);  // ids, then order keys
  return pl;
}

}  // namespace

extern "C" {

size_t sfa_indexer_topk_workspace_size(const sfa_indexer_args* a) {
  if (check_indexer(a) != SFA_OK) return 0;
  const IndexerPlan pl = indexer_plan(a);
  return pl.score_bytes + pl.cand_bytes;
}

int sfa_indexer_topk(const sfa_indexer_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  const int rc = check_indexer(a);
  if (rc != SFA_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  sfa::IndexerParams p = to_iparams(a);
  const IndexerPlan pl = indexer_plan(a);
  const size_t need = pl.score_bytes + pl.cand_bytes;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(SFA_E_WORKSPACE, "sfa_indexer_topk needs %zu workspace bytes (got %zu)", need, workspace_bytes);
  if (a->logits == nullptr) {
    p.logits = (float*)workspace;
    p.g_ss = pl.ld;
    p.g_sb = (int64_t)pl.rows * pl.ld;
  }
  p.cand = pl.cand_bytes ? (int32_t*)((char*)workspace + pl.score_bytes) : nullptr;
  p.cand_key = pl.cand_bytes ? (uint32_t*)((char*)workspace + pl.score_bytes + pl.cand_bytes / 2) : nullptr;
  for (int t0 = 0; t0 < a->Sq; t0 += pl.rows) {
    const int t1 = t0 + pl.rows < a->Sq ? t0 + pl.rows : a->Sq;
    p.g_t0 = a->logits ? 0 : t0;
    p.nseg = p.cand ? sfa::topk_segments(p, t1 - t0) : 1;
    p.seglen = p.nseg > 1 ? sfa::topk_seglen(p, p.nseg) : 0;
    hipError_t e = sfa::launch_indexer_logits(p, t0, t1, s);
    if (e == hipSuccess) e = sfa::launch_topk_select(p, t0, t1, s);
    if (e != hipSuccess) return hip_fail(e, "sfa_indexer_topk");
  }
  return SFA_OK;
}

}  // extern "C"


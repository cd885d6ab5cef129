// gfx950 MFMA forward of top-k sparse flash attention for DeepSeek MLA
// (G = 128 query heads share one latent KV head, d_qk = 576, d_v = 512, V the
// first 512 dims of the K rows); bf16 in, fp32 accumulate.  The d = 128
// shapes have their own kernel (sfa_fwd_d128.hip).
//
// Reference: `_attn_fwd` / `_inner_fwd` (lilac-me/ops SFA.py:309-587).  The
// math is the same (gather the top-k rows, masked base-2 online softmax, P·V,
// sink, LSE); the schedule is MI355X-native:
//
//  * One workgroup owns one (batch, query, kv-head[, split]) work item and
//    all G query heads of it, so every gathered KV row is used by all G heads
//    (the reference re-gathers per 32-head tile, SFA.py:557).
//  * 4 waves x 32 heads.  A wave computes S^T = K·Q^T for its heads over a
//    32-key tile: keys are MFMA rows, heads MFMA columns.  The fp32 S^T
//    accumulator layout then already is the B-operand layout of
//    O^T = V^T·P^T (contraction over keys), so P never leaves registers, and
//    every lane owns exactly one head: row max / sum and the rescale of the
//    O^T accumulator are per-lane scalars.
//  * V^T operands are read from the row-major LDS tile with
//    ds_read_b64_tr_b16 (gfx950 transposing LDS read).
//  * KV rows are gathered straight into LDS with buffer_load_dwordx4 ... lds
//    (no VGPR staging), double-buffered one tile ahead, the instructions
//    spread over the previous tile's MFMA stream (RowGather).  Invalid slots
//    use an out-of-range buffer offset, so the hardware writes zeros.  Tile
//    rows have a pitch of 72 16-byte slots with the chunks XOR-swizzled by row
//    (tile_swz), which makes both operand read patterns bank-conflict free.
//  * Online softmax with a lazy rescale: the running max used for the
//    exponentials is only raised when a tile's max exceeds it by more than
//    kRescaleSlack (base-2 units).  Exponentials then stay <= 2^kRescaleSlack,
//    and the final normalisation uses the same stale max, so the result is
//    the exact softmax.
//  * Split-k over the top-k slots (decode) writes normalised bf16 partial
//    outputs plus their base-2 LSE; sfa::launch_combine merges them.
//  * Paged KV (PAGED = true, sfa_fwd_paged): the index staging turns each
//    logical key into its pool row through the block table, and the gather
//    uses 64-bit addresses (global_load_lds_dwordx4; a pool can exceed the
//    4 GiB a buffer offset reaches), padding rows reading a zero row.
//
// MFMA register layouts used (gfx950 32x32x16 bf16, 8 values per lane, T = 32):
//   A[m][k]: lane l holds m = l % T, k = 8*(l / T) + j        (j = 0..7)
//   B[k][n]: lane l holds n = l % T, k = 8*(l / T) + j
//   C[m][n]: lane l holds n = l % T, m = 4*LG*(e/4) + 4*(l/T) + e%4,
//            e = 0..15, LG = 64/T = 2.

#include "sfa_common.h"
#include "sfa_lds.h"
#include "sfa_mfma.h"

namespace sfa {
namespace {

constexpr float kRescaleSlack = 8.0f;
constexpr int kIdxCap = 2048;  // slots staged in LDS per work item
#ifndef MLA_QREG
#define MLA_QREG 20
#endif

template <int T_, int DQK_, int DV_, int NSLICE_, int NSPLITW_, bool VK_, int QREG_, bool SWZ_ = false>
struct FwdCfg {
  static constexpr bool SWZ = SWZ_;         // k tile: pitch CHK, chunks swizzled by row (tile_swz)
  static constexpr int T = T_;
  static constexpr int DQK = DQK_;
  static constexpr int DV = DV_;
  static constexpr int NSLICE = NSLICE_;
  static constexpr int NSPLITW = NSPLITW_;
  static constexpr bool VK = VK_;           // v rows are the first DV dims of the k rows
  static constexpr int kWaves = NSLICE * NSPLITW;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int LG = 64 / T;         // lane groups
  static constexpr int KD = 8 * LG;         // MFMA contraction length
  static constexpr int CPL = T * T / 64;    // accumulator values per lane
  static constexpr int MT = 32 / T;         // S^T MFMA tiles per 32-key wave tile
  static constexpr int NKT = 32 * NSPLITW;  // keys per workgroup tile
  static constexpr int QSTEPS = DQK / KD;
  static constexpr int QREG = QREG_;        // contraction steps whose Q^T operand stays in VGPRs
  static constexpr int QL = QSTEPS - QREG;  // steps whose Q^T operand is read from LDS
  static constexpr int QLP = QL * LG + 1;   // LDS pitch (16-byte slots) of a head's LDS-resident q dims
  static constexpr int QBUF = QL > 0 ? NSLICE * T * QLP : 1;
  static constexpr int OT = DV / T;
  static constexpr int CHK = DQK / 8;       // 16-byte chunks per k row
  static constexpr int PK = SWZ ? CHK : CHK + 1;  // LDS row pitch in 16-byte slots (odd unless swizzled)
  static constexpr int KBUF = NKT * PK;     // 16-byte slots per k tile
  static_assert(DQK % KD == 0 && DV % T == 0, "head dims must tile the MFMA");
  static_assert(!VK || DV <= DQK, "v must be a prefix of k");
  static_assert(CHK % 2 == 0, "rows need an even number of 16-byte chunks");
  static_assert(T == 32 && NSPLITW == 1 && VK && SWZ, "the kernel is written for this configuration");
};

// LDS reads through pointers derived from the __shared__ arrays themselves, so
// the compiler keeps per-array alias information and does not make the reads
// of one tile buffer wait for the DMA still filling the other.
// Persistent scheduling (PERSIST): one workgroup per CU claims work items
// from 8 counters, one per XCD.  Counter x hands out the virtual workgroup
// ids x, x + 8, x + 16, ... (the ids the hardware would have dispatched to XCD
// x, so the items keep the L2 locality of item_of's mapping); a workgroup
// takes from its own XCD's counter and, once that is exhausted, from the
// others (XCDs run at different clocks: without this the fastest idle while
// the slowest finish).  nvb: number of virtual ids.  Called by one thread.
// claim_start only issues the own-counter atomic; claim_finish reads its
// result later (so the atomic's latency overlaps other work) and steals when
// the own counter is exhausted.
__device__ __forceinline__ int claim_start(int* ctr, int x) {
  // (an offset the compiler cannot prove uniform: for a uniform address it
  // rewrites the atomic into a wave reduction that needs the returned value
  // at once, i.e. waits for every load in flight right here)
  int o = 0;
  asm volatile("" : "+v"(o));
  return atomicAdd(ctr + x + o, 1);
}
__device__ __forceinline__ int claim_finish(int* ctr, int x, int nvb, int c) {
  if (c < (nvb - x + 7) / 8) return x + 8 * c;
  for (int k = 1; k < 8; ++k) {
    const int y = (x + k) & 7;
    const int cy = atomicAdd(&ctr[y], 1);
    if (cy < (nvb - y + 7) / 8) return y + 8 * cy;
  }
  return -1;
}

__global__ void sched_reset_kernel(int* ctr) {
  if (threadIdx.x < 8) ctr[threadIdx.x] = 0;
}

// A work item: (batch, query, kv head) and its split of the top-k slots.
struct ItemPos {
  int b, t, g, split, nslots;
};

// Virtual workgroup id -> work item.  Workgroups are dispatched to the 8 XCDs
// round-robin (id % 8); with splits, the splits of one item are placed on
// the same XCD (so its L2 serves the item's Q rows to all of them) whenever
// the item count allows a bijective mapping.  Without splits, XCD x gets
// runs of 32 consecutive items (queries), runs dealt round-robin over the
// XCDs: the workgroups running together on one XCD then share the keys their
// queries have in common (e.g. a recency window) in its L2.
__device__ __forceinline__ ItemPos item_of(const Params& p, int vb) {
  ItemPos it;
  int wi = vb;
  const int64_t nitems = (int64_t)p.B * p.Sq * p.Hkv;
  if (p.num_splits > 1 && nitems % 8 == 0) {
    const int x = wi % 8, r = wi / 8;
    it.split = r % p.num_splits;
    wi = (r / p.num_splits) * 8 + x;
  } else if (p.num_splits == 1 && nitems % 256 == 0) {
    const int x = wi % 8, r = wi / 8;
    it.split = 0;
    wi = ((r / 32) * 8 + x) * 32 + r % 32;
  } else {
    it.split = wi % p.num_splits;
    wi /= p.num_splits;
  }
  it.g = wi % p.Hkv;
  wi /= p.Hkv;
  it.t = wi % p.Sq;
  it.b = wi / p.Sq;
  int nslots = p.topk - it.split * p.split_len;
  if (nslots > p.split_len) nslots = p.split_len;
  if (nslots < 0) nslots = 0;
  it.nslots = nslots;
  return it;
}

// LDS-only workgroup barrier: waits for this wave's LDS operations (and for
// all but its last VM vector-memory operations, VM an immediate), not for the
// global stores a __syncthreads fence would also wait for.
#define SFA_LDS_BARRIER(VM) asm volatile("s_waitcnt vmcnt(" #VM ") lgkmcnt(0)\n\ts_barrier" ::: "memory")

// LDS reads go through pointers derived from the __shared__ arrays themselves,
// so the compiler keeps per-array alias information and does not make the reads
// of one tile buffer wait for the DMA still filling the other.
//
// Per work item: a prologue (the index row, tile 0's gather, Q), the tile
// loop, the output.  The persistent kernel (PERSIST) overlaps the next
// item's prologue with this item's output: its loads are issued right after
// the tile loop, its tile 0 is gathered between the two rounds of the output
// staging (which then uses the Q area only), and its ids and Q are staged
// behind one barrier after the output.
template <class C, bool PAGED, bool PERSIST>
__global__ __launch_bounds__(C::kThreads, 1) void fwd_mfma_kernel(Params p_arg) {
  constexpr int T = C::T;
  using M = Mfma<T>;
  typedef typename M::acc_t acc_t;
  // (contiguous rows: the index row is staged as row byte offsets, so a
  // row's gather base costs a select; tile 0's rows come from the global ids)
  // (the prologue gathers -- tile 0 and Q -- are untracked, so the output
  // staging's LDS reads that overlap them in the persistent kernel do not
  // wait for them; item_stage waits for them before its barrier)
  typedef typename std::conditional<PAGED, PoolRows, BufRowsOff>::type Src;
  typedef typename std::conditional<PAGED, PoolRows, BufRowsUT>::type Src0;
  typedef RowGather<C::NKT, C::CHK, C::kWaves, C::SWZ, Src> RG;
  typedef RowGather<C::NKT, C::CHK, C::kWaves, C::SWZ, Src0> RG0;
  static_assert(RG::PITCH == C::PK, "gather and readers agree on the pitch");

  __shared__ int s_idx[kIdxCap];
  __shared__ u32x4 s_k0[C::KBUF];
  __shared__ u32x4 s_k1[C::KBUF];
  __shared__ u32x4 s_q[C::QBUF];
  __shared__ int s_used[C::kWaves];
  // claimed virtual ids, by item parity: item i's successor is published in
  // slot (i + 1) & 1 before item i's staging barrier and read after item i's
  // tile loop; the slot is rewritten two items later, behind barriers
  __shared__ int s_claim[2];

  const int nvb = (int)((int64_t)p_arg.B * p_arg.Sq * p_arg.Hkv * p_arg.num_splits);  // virtual workgroup ids
  constexpr bool kUntracked = Src::kUntrackedDma;

  // ---- prologue pieces ------------------------------------------------
  // Loop-carried: the item and its Q^T B operands in VGPRs (QREG steps; the
  // rest are gathered into s_q).
  ItemPos it{};
  bf16x8 qb[C::QREG > 0 ? C::QREG : 1];
  IdxStage<kIdxCap, C::kThreads> istage;
  int raw[RG::RPW];
  int klen = 0;     // the item's kv_lens entry as loaded (0 without kv_lens); see item_bound
  int claim_c = 0;  // (thread 0) the pending claim's raw count
  // the gather source of an item: the (batch, kv head) slice's rows
  auto make_src = [&](const Params& p, const ItemPos& q) {
    Src s;
    if constexpr (PAGED) {
      s.base = reinterpret_cast<const char*>(p.k) + 2 * q.g * p.k_sh;
      s.shift = p.pool_shift;
    } else {
      const char* kbase = reinterpret_cast<const char*>(p.k) + 2 * (q.b * p.k_sb + q.g * p.k_sh);
      s.rs = make_rsrc(kbase, (uint32_t)(2 * ((int64_t)(p.Skv - 1) * p.k_ss + C::DQK)));
      s.row_bytes = (uint32_t)(2 * p.k_ss);
    }
    return s;
  };
  // (1) the item's loads, all in flight together: the claim of the item
  // after it, its index row (coalesced), the ids of the wave's 8 rows of
  // tile 0 (uniform addresses; slots past the split re-read its last slot,
  // whose id is then discarded), the register steps of Q.  Loads complete in
  // order, so each later wait covers only what was issued before it.
  // (Buffer loads whose out-of-range lanes read zeros: a select on loaded
  // data would make the wave wait for each load right here.)
  auto item_loads = [&](const Params& p, const ItemPos& q, int tid, int wave, int lane) {
    if constexpr (PERSIST) {
      if (tid == 0) claim_c = claim_start(p.sched, blockIdx.x & 7);
    }
    // (one work item per workgroup, e.g. a decode step with kv_lens) the key
    // bound first, as a buffer load (no kv_lens: an empty range, which reads
    // 0) whose value is only used at the staging: a load used at once makes
    // the wave wait there for every load issued before it, the Q loads
    // included, and used late it is waited for alone
    if constexpr (!PERSIST)
      klen = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(p.kv_lens, p.kv_lens ? 4u * (uint32_t)p.B : 0u),
                                                  4u * (uint32_t)q.b, 0, 0);
    const int32_t* irow = p.idx + q.b * p.i_sb + q.t * p.i_ss + q.g * p.i_sh + q.split * p.split_len;
    istage.load_buf(make_rsrc(irow, 4u * (uint32_t)q.nslots), tid);
#pragma unroll
    for (int r = 0; r < RG::RPW; ++r) raw[r] = irow[min(wave * RG::RPW + r, max(q.nslots - 1, 0))];
    const int hl = (wave % C::NSLICE) * T + (lane % T);
    const char* qbase = reinterpret_cast<const char*>(p.q) + 2 * (q.b * p.q_sb + q.t * p.q_ss + (int64_t)q.g * p.G * p.q_sh);
    const uint32_t hbytes = (uint32_t)(2 * p.q_sh);
    // (heads past G: offsets >= G * hbytes, past the range, read zeros)
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(qbase, (uint32_t)(p.G - 1) * hbytes + 2u * C::DQK);
    const uint32_t qoff = (uint32_t)hl * hbytes + 16u * (uint32_t)(lane / T);
#pragma unroll
    for (int s = 0; s < C::QREG; ++s) {
      typedef int i32x4 __attribute__((ext_vector_type(4)));
      const i32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + 2u * (uint32_t)(s * C::KD), 0, 0);
      qb[s] = __builtin_bit_cast(bf16x8, x);
    }
  };
  // the item's key bound: kv_lens[b] (at most Skv), or Skv without kv_lens
  auto item_bound = [&](const Params& p, const ItemPos& q) {
    if constexpr (PERSIST) return bound_of(p, q.b);
    return p.kv_lens ? min(klen, p.Skv) : p.Skv;
  };
  // (1b) the LDS-resident steps of Q straight into s_q (buffer_load ... lds,
  // no VGPRs): head h's steps QREG.. are its dims [16 QREG, DQK), contiguous
  // in memory, and go to slots h * QLP .. h * QLP + 2 QL - 1 (chunk (s - QREG)
  // * LG + j = dims 16 s + 8 j); the slot after them is padding (it re-reads
  // the last chunk).  Instruction k of the workgroup writes slots [64 k, 64 k
  // + 64); heads past G read zeros (out of range).
  auto item_qdma = [&](const Params& p, const ItemPos& q, int wave, int lane) {
    const char* qbase = reinterpret_cast<const char*>(p.q) + 2 * (q.b * p.q_sb + q.t * p.q_ss + (int64_t)q.g * p.G * p.q_sh);
    const uint32_t hbytes = (uint32_t)(2 * p.q_sh);
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(qbase, (uint32_t)(p.G - 1) * hbytes + 2u * C::DQK);
    constexpr int NSLOT = C::QBUF, NINST = (NSLOT + 63) / 64;
#pragma unroll
    for (int k0 = 0; k0 < NINST; k0 += C::kWaves) {
      const int k = k0 + wave;
      const int u = 64 * k + lane;
      const int h = u / C::QLP;
      const int c = min(u - h * C::QLP, 2 * C::QL - 1);
      const uint32_t off = h < p.G ? (uint32_t)h * hbytes + 32u * C::QREG + 16u * (uint32_t)c : kOOB;
      static_assert(NSLOT % 64 == 0, "whole instructions");
      if (k < NINST) dma_lds16_untracked(rq, s_q + 64 * k, off);
    }
  };
  // (2) tile 0's gather into s_k0, from the ids of (1)
  auto item_gather0 = [&](const Params& p, const ItemPos& q, int wave, int lane) {
    const Src s = make_src(p, q);
    Src0 s0;
    if constexpr (PAGED) {
      s0 = s;
    } else {
      s0.rs = s.rs;
      s0.row_bytes = s.row_bytes;
    }
    const int bound = item_bound(p, q);
    RG0 rg0;
    if constexpr (PAGED) {
      // (all 8 block-table loads in flight together)
      int id[RG::RPW], st[RG::RPW];
#pragma unroll
      for (int r = 0; r < RG::RPW; ++r) id[r] = wave * RG::RPW + r < q.nslots ? raw[r] : -1;
      paged_rows<RG::RPW, true>(p, q.b, id, bound, st);
#pragma unroll
      for (int r = 0; r < RG::RPW; ++r) rg0.set_row(r, st[r], true, s0);
    } else {
#pragma unroll
      for (int r = 0; r < RG::RPW; ++r)
        rg0.set_row(r, (wave * RG::RPW + r < q.nslots) ? staged_id<false>(p, q.b, raw[r], bound) : -1, true, s0);
    }
#pragma unroll
    for (int k = 0; k < RG::NI; ++k) rg0.issue(k, s0, s_k0, wave, lane);
  };
  // (3) stage the index row, publish the next claim, wait for this wave's
  // gathers (tile 0 and Q; VM: the vector-memory operations issued after
  // them, which need not complete), barrier.  Returns
  // the item's tile count, trimmed to the last valid slot (tiles of trailing
  // padding, e.g. a causal row shorter than top-k, contribute nothing).
  int ipar = 0;  // parity of the current item
  auto item_stage = [&](const Params& p, const ItemPos& q, int tid, int wave, int lane, bool vm24) -> int {
    const int ntiles0 = (q.nslots + C::NKT - 1) / C::NKT;
    const int bound = item_bound(p, q);
    int used;
    if constexpr (PAGED)
      used = istage.store_pool_offsets(p, q.b, bound, q.nslots, ntiles0 * C::NKT, s_idx, tid);
    else
      used = istage.store_offsets(bound, q.nslots, ntiles0 * C::NKT, s_idx, tid, (uint32_t)(2 * p.k_ss), kOOBRow);
    used = wave_max_int(used);
    if (lane == 0) s_used[wave] = used;
    if constexpr (PERSIST) {
      if (tid == 0) s_claim[ipar ^ 1] = claim_finish(p.sched, blockIdx.x & 7, nvb, claim_c);
    }
    // (the gathers are untracked: this wait and the barrier are what make the
    // other waves' rows and Q chunks visible)
    if (vm24)
      SFA_LDS_BARRIER(24);
    else
      SFA_LDS_BARRIER(0);
    int u = s_used[0];
#pragma unroll
    for (int w = 1; w < C::kWaves; ++w) u = max(u, s_used[w]);
    return (u + C::NKT - 1) / C::NKT;
  };

  int vb = blockIdx.x;
  if constexpr (PERSIST) {
    if (threadIdx.x == 0) s_claim[0] = claim_finish(p_arg.sched, blockIdx.x & 7, nvb, claim_start(p_arg.sched, blockIdx.x & 7));
    __syncthreads();
    // (read as uniform: a value loaded from LDS is a per-lane value to the
    // compiler, and every address derived from it would be built per lane)
    vb = __builtin_amdgcn_readfirstlane(s_claim[0]);
  }
  int ntiles = 0;
  if (vb >= 0) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    it = item_of(p_arg, vb);
    item_loads(p_arg, it, tid, wave, lane);
    item_qdma(p_arg, it, wave, lane);
    item_gather0(p_arg, it, wave, lane);
    ntiles = item_stage(p_arg, it, tid, wave, lane, false);
  }

  while (vb >= 0) {
  // The parameters are read through a pointer the compiler cannot see
  // through, once per item: otherwise it hoists every parameter load out of
  // the item loop and keeps the values live (and spilled) across it.
#if __HIP_DEVICE_COMPILE__
  typedef __attribute__((address_space(4))) const Params* kparams_t;
  kparams_t pp = (kparams_t)__builtin_amdgcn_kernarg_segment_ptr();
  if constexpr (PERSIST) asm volatile("" : "+s"(pp));
  const Params& p = *pp;
#else
  const Params& p = p_arg;  // (host pass: the body is only type-checked)
#endif
  // (the thread index likewise, so that lane-dependent constants are formed
  // per item rather than held, and spilled, across the item loop)
  int tid = threadIdx.x;
  if constexpr (PERSIST) asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slice = wave % C::NSLICE;
  const int ks = wave / C::NSLICE;
  const int b = it.b, t = it.t, g = it.g, split = it.split;
  const Src ksrc = make_src(p, it);
  const int hl = slice * T + (lane % T);  // head within the group
  const bool hvalid = hl < p.G;

  // DMA instruction k follows MFMA number kDmaFirst + kDmaStride * k of the
  // tile's MFMA sequence (QSTEPS S^T MFMAs, then the O^T MFMAs)
#ifndef SFA_DMA_STRIDE
#define SFA_DMA_STRIDE 3
#endif
#ifndef SFA_DMA_FIRST
#define SFA_DMA_FIRST 2
#endif
  constexpr int kDmaStride = SFA_DMA_STRIDE, kDmaFirst = SFA_DMA_FIRST;
  constexpr int kOtMfmas = 32 / 16 * C::OT;
  static_assert(kDmaFirst + kDmaStride * (RG::NI - 1) < C::QSTEPS + kOtMfmas, "schedule fits");
  // (on the last tile the offsets are all out of range: the instructions
  // still issue, so the MFMA stream has no branches, and write zeros into the
  // idle buffer)
  auto dma_at = [&](int m, const RG& rg, u32x4* ndst) {
    if (m >= kDmaFirst && (m - kDmaFirst) % kDmaStride == 0 && (m - kDmaFirst) / kDmaStride < RG::NI)
      rg.issue((m - kDmaFirst) / kDmaStride, ksrc, ndst, wave, lane);
  };

  // ---- accumulators ----------------------------------------------------
  acc_t oacc[C::OT];
#pragma unroll
  for (int i = 0; i < C::OT; ++i) oacc[i] = acc_t{};
  float m_used = kNegInf;  // running max (base 2) the exponentials are taken against
  float m_off = 0.f;       // -m_used, or 0 while m_used is -inf (the exponent offset)
  float l_part = 0.f;      // this lane's share of the row sum

  const int hq = lane / T;  // lane group: which k-slice of the MFMA operands
  const int lt = lane % T;

  // vmcnt(0) before the barriers that publish a gathered tile, where the
  // compiler does not see the DMA (PoolRows)
  auto dma_done = [&]() {
    if constexpr (kUntracked) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  };

  // compute(tile) also issues the gather of the next tile into ndst (rg
  // holds that tile's row offsets), and, inside its O^T MFMA stream (all of
  // that gather has been issued by then), reads the row ids of tile + 2 into
  // rg and the validity mask of tile + 1 into vmask_io (on entry: this
  // tile's), so no LDS round trip sits between the end of one tile's MFMAs
  // and the next tile's.  Its first PDK K operands are in kbuf on entry; after
  // O^T MFMA kBarAt it runs the barrier that publishes tile + 1 (and ends
  // every read of this tile's buffer), then reads the first K operands of
  // tile + 1 into kbuf while its last MFMAs execute.
  constexpr int PDK = 4;
  // S^T A operands: step s of lane (key lt, k-slice hq) is chunk 2s + hq = 8 (s >> 2) + v
  // with v = 2 (s & 3) + hq, at slot 8 (s >> 2) + (v ^ swz(row)): four bases
  uint32_t kb[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    kb[j] = (uint32_t)((ks * 32 + lt) * C::PK + ((2 * j + hq) ^ tile_swz(ks * 32 + lt))) * 16u;
  auto load_k_at = [&](const u32x4* buf, int s) { return lds_read_b128(buf, kb[s & 3] + (uint32_t)(s >> 2) * 128u); };
  auto compute = [&](int tile, const u32x4* kt, const u32x4* vt, RG& rg, u32x4* ndst, uint32_t& vmask_io,
                     bf16x8 (&kbuf)[PDK]) {
    const uint32_t vmask = vmask_io;  // validity of this wave's 32 keys

    // S^T = K Q^T
    acc_t sacc[C::MT];
    const uint32_t q_off = (uint32_t)(hl * C::QLP + hq) * 16u;
    // one 32-key M-tile: operands of step s + PDK are loaded before MFMA s
    auto load_k = [&](int s) { return load_k_at(kt, s); };
    auto load_q = [&](int s) { return lds_read_b128(s_q, q_off + (uint32_t)((s - C::QREG) * C::LG) * 16u); };
    bf16x8 qbuf[PDK];
#pragma unroll
    for (int i = 0; i < PDK; ++i)
      if (i >= C::QREG) qbuf[i] = load_q(i);
    // V^T operand reads of the O^T stream (below): the first PD are issued
    // during the last S^T MFMAs, so they land while the softmax runs
    // O^T += V^T P^T.  Operand i = kk * OT + ot; the two transposed LDS reads
    // of operand i + PD are issued before MFMA i (software pipeline).
    constexpr int VP = C::PK;  // V rows are the K rows
    const int gi = lane & 15;         // lane within its 16-lane transpose group
    const int rr = gi >> 2;           // row within a run of 4 keys this lane loads
    const int cc = gi & 3;            // 4-dim column piece this lane loads
    const int mgrp = (lt >> 4) << 4;  // first MFMA row (dim) of the 16-lane group
    // the two runs of 4 consecutive keys feeding k = 0..3 and k = 4..7
    const int run0 = 4 * hq;
    const int run1 = 8 + 4 * hq;
    // Operand (kk, ot) of a lane: its dims ot*32 + mgrp + 4cc .. +3 are in
    // chunk 4 ot + cl, cl = mgrp / 8 + cc / 2, i.e. chunk 8 (ot >> 1) + v
    // with v = 4 (ot & 1) + cl, at slot 8 (ot >> 1) + (v ^ swz(row)) of rows
    // 16 kk + run + rr; rows r and r + 16 share swz, so each run needs one
    // base per parity of ot.
    uint32_t vb[2][2];
    {
      const int rows[2] = {ks * 32 + run0 + rr, ks * 32 + run1 + rr};
      const int cl = mgrp / 8 + cc / 2;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int par = 0; par < 2; ++par)
          vb[h][par] = (uint32_t)(rows[h] * VP + ((4 * par + cl) ^ tile_swz(rows[h]))) * 16u + (uint32_t)(cc & 1) * 8u;
    }
    auto load_a = [&](int i) -> bf16x8 {
      const int kk = i / C::OT, ot = i % C::OT;
      const uint32_t off = (uint32_t)(16 * kk * VP) * 16u + (uint32_t)(ot >> 1) * 128u;
      const uint32_t o0 = vb[0][ot & 1] + off;
      const uint32_t o1 = vb[1][ot & 1] + off;
      const bf16x4 lo = lds_read_tr16(vt, o0);
      const bf16x4 hi = lds_read_tr16(vt, o1);
      return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    constexpr int NI = 2 * C::OT;  // O^T MFMAs (two 16-key contraction steps per 32 keys)
    constexpr int PD = 3;          // V^T operand reads in flight ahead of the O^T MFMAs
    bf16x8 abuf[PD];
    bf16x8 pa = {}, pq = {};
#pragma unroll
    for (int s = 0; s < C::QSTEPS; ++s) {
      const bf16x8 a = kbuf[s % PDK];
      const bf16x8 bq = (s < C::QREG) ? qb[s < C::QREG ? s : 0] : qbuf[s % PDK];
      if (s + PDK < C::QSTEPS) {
        kbuf[s % PDK] = load_k(s + PDK);
        if (s + PDK >= C::QREG) qbuf[s % PDK] = load_q(s + PDK);
      }
      if (s == 0)
        M::mma_v0(a, bq, sacc[0]);
      else
        M::mma_v(a, bq, sacc[0], pa, pq);
      pa = a;
      pq = bq;
      dma_at(s, rg, ndst);
      if (s >= C::QSTEPS - PD) abuf[s - (C::QSTEPS - PD)] = load_a(s - (C::QSTEPS - PD));
    }
    M::drain_v(sacc[0], pa, pq);

    // Raw scores; invalid keys -> -inf.  A tile whose 32 keys are all valid
    // (the common case) skips the per-element mask.  The softmax scale is
    // applied inside the exponent (fma), and the max is taken on raw scores
    // (scale > 0 preserves the order).
    constexpr int NV = C::MT * C::CPL;
    float sv[NV];
    if (vmask == 0xffffffffu) {
#pragma unroll
      for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
        for (int e = 0; e < C::CPL; ++e) sv[mt * C::CPL + e] = sacc[mt][e];
    } else {
#pragma unroll
      for (int mt = 0; mt < C::MT; ++mt) {
#pragma unroll
        for (int e = 0; e < C::CPL; ++e) {
          const int key = mt * T + 4 * C::LG * (e / 4) + 4 * hq + (e % 4);
          sv[mt * C::CPL + e] = ((vmask >> key) & 1u) ? sacc[mt][e] : kNegInf;
        }
      }
    }
    // P^T = 2^(scale_log2 * s - m) as the B operand of O^T = V^T P^T; -inf
    // scores give exactly 0.  The exponentials are first taken against the
    // running max m_used, independently of this tile's max, so the max
    // reduction and the exponentials overlap; only when the tile's max
    // exceeds m_used by more than kRescaleSlack (rare after the first valid
    // tile) are O^T and l rescaled and the exponentials recomputed.  While no
    // valid key has been seen m_used is -inf: the offset is then 0, and the
    // first valid tile always takes the recompute path.
    // Only the NE0 values of the first O^T contraction step are needed before
    // the first O^T MFMA; the rest are computed while the MFMAs of that step
    // run (late_exps, after the max test, so never recomputed).
    constexpr int NE0 = NV < 8 ? NV : 8;
    float ex[NV];
    float moff = m_off;
    {
#pragma unroll
      for (int i = 0; i < NE0; ++i) ex[i] = __builtin_amdgcn_exp2f(fmaf(sv[i], p.scale_log2, moff));
      // Materialise them here: the rescale path below overwrites them, so
      // the compiler would otherwise sink this computation into the
      // no-rescale branch, behind the max reduction.
#pragma unroll
      for (int i = 0; i < NE0; ++i) asm volatile("" : "+v"(ex[i]));
    }
    static_assert(NV == 16, "the max tree below covers 16 values");
    const float t0 = max3_raw(sv[0], sv[1], sv[2]), t1 = max3_raw(sv[3], sv[4], sv[5]),
                t2 = max3_raw(sv[6], sv[7], sv[8]), t3 = max3_raw(sv[9], sv[10], sv[11]),
                t4 = max3_raw(sv[12], sv[13], sv[14]);
    float tmax = max_raw(max3_raw(t0, t1, t2), max3_raw(t3, t4, sv[15]));  // depth 3, not a 15-long chain
    tmax = xor32_max_raw(tmax);
    tmax *= p.scale_log2;
    const float m_new = max_raw(m_used, tmax);
    if (__any(m_new > m_used + kRescaleSlack)) {
      const float alpha = (m_new == kNegInf) ? 1.f : exp2f(m_used - m_new);
      l_part *= alpha;
#pragma unroll
      for (int i = 0; i < C::OT; ++i) M::scale_agpr(oacc[i], alpha);
      m_used = m_new;
      moff = m_off = (m_used == kNegInf) ? 0.f : -m_used;
#pragma unroll
      for (int i = 0; i < NE0; ++i) ex[i] = __builtin_amdgcn_exp2f(fmaf(sv[i], p.scale_log2, moff));
    }
    constexpr int KSTEPS = NV / 8;  // O^T contraction steps per 32 keys
    bf16x8 pb[KSTEPS];
#pragma unroll
    for (int i = 0; i < NE0; ++i) pb[i / 8][i % 8] = (bf16)ex[i];
    // One wave per SIMD issues in order, so VALU work only overlaps an MFMA
    // that is already running: the late exponentials and the row sum are
    // spread over the O^T MFMA stream, one small piece after each MFMA (the
    // pins keep the compiler from hoisting a piece in front of its MFMA).
    constexpr int NLATE = NV - NE0;
    auto late_exp = [&](int j) {  // value NE0 + j
      const int i = NE0 + j;
      asm volatile("" : "+v"(sv[i]));
      ex[i] = __builtin_amdgcn_exp2f(fmaf(sv[i], p.scale_log2, moff));
      if (j & 1) {
        pb[i / 8][(i - 1) % 8] = (bf16)ex[i - 1];
        pb[i / 8][i % 8] = (bf16)ex[i];
      }
    };
    // pairwise sum of ex[lo, lo + n) (short dependency chain), into ex[lo]
    auto sum_range = [&](int lo, int n) {
#pragma unroll
      for (int i = 0; i < n; ++i) asm volatile("" : "+v"(ex[lo + i]));
#pragma unroll
      for (int w = 1; w < n; w *= 2)
#pragma unroll
        for (int i = 0; i + w < n; i += 2 * w) ex[lo + i] += ex[lo + i + w];
    };

    static_assert(NI == KSTEPS * C::OT, "O^T MFMA count");
    // O^T MFMA after which the ids of tile + 2 are read, and the lag (in
    // MFMAs) after which they are used
    constexpr int kIdsAt = NLATE + 3, kIdsLag = 4;
    // the barrier after the last V^T read has been issued
    constexpr int kBarAt = NI - PD - 1;
    static_assert(kIdsAt + kIdsLag + RG::RPW < kBarAt && NLATE + 2 < kBarAt, "id prefetch and softmax pieces precede the barrier");
    static_assert(kDmaFirst + kDmaStride * (RG::NI - 1) < C::QSTEPS + kIdsAt,
                  "the gather of tile + 1 is issued before rg is overwritten");
    int ids_raw[RG::RPW];
    bool ids_ok = false;
    int vm_raw = 0;
    static_assert(NI >= NLATE + 3 && NLATE <= C::OT && NE0 % 2 == 0 && NLATE % 2 == 0,
                  "late softmax pieces must finish before the MFMAs that use them");
    bf16x8 prev_a = {}, prev_b = {};
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const bf16x8 a = abuf[i % PD];
      if (i + PD < NI) abuf[i % PD] = load_a(i + PD);
      if (i % C::OT == 0)  // first use of pb[kk], just written by VALU
        M::template mma_agpr<true>(a, pb[i / C::OT], oacc[i % C::OT], prev_a, prev_b);
      else
        M::template mma_agpr<false>(a, pb[i / C::OT], oacc[i % C::OT], prev_a, prev_b);
      prev_a = a;
      prev_b = pb[i / C::OT];
      dma_at(C::QSTEPS + i, rg, ndst);
      if (i == kIdsAt) {
        ids_ok = tile + 2 < ntiles;
        RG::fetch(s_idx + (ids_ok ? tile + 2 : 0) * C::NKT, wave, ids_raw);
        vm_raw = s_idx[(tile + 1 < ntiles ? tile + 1 : 0) * C::NKT + ks * 32 + (lane & 31)];
      }
      // one row offset per MFMA from kIdsAt + kIdsLag on (each pinned at its
      // MFMA, so the wait for the reads is not hoisted next to them and the
      // scalar work does not bunch up between two MFMAs)
      if (i >= kIdsAt + kIdsLag && i < kIdsAt + kIdsLag + RG::RPW) {
        const int r = i - kIdsAt - kIdsLag;
        asm volatile("" : "+v"(ids_raw[r]));
        rg.set_row(r, ids_raw[r], ids_ok, ksrc);
        asm volatile("" : "+s"(rg.base[r]));
      }
      if (i == kIdsAt + kIdsLag + RG::RPW) {
        asm volatile("" : "+v"(vm_raw));
        vmask_io = (uint32_t)__ballot(vm_raw >= 0);
        asm volatile("" : "+s"(vmask_io));
      }
      if (i < NLATE) late_exp(i);
      if (i == NLATE) sum_range(0, NE0);
      if (NLATE > 0 && i == NLATE + 1) sum_range(NE0, NLATE);
      if (i == NLATE + 2) l_part += (NLATE > 0) ? ex[0] + ex[NE0] : ex[0];
      if (i == kBarAt) {
        dma_done();
        __syncthreads();  // tile + 1 in place in ndst; every read of this tile's buffer done
#pragma unroll
        for (int j = 0; j < PDK; ++j) kbuf[j] = load_k_at(ndst, j);
      }
    }
    M::tail(prev_a, prev_b);
  };

  // row offsets of tile 1 (gathered during tile 0) and the validity mask of
  // tile 0; compute() fetches those of the following tiles itself
  RG rg;
  rg.load_ids(s_idx + (ntiles > 1 ? C::NKT : 0), ntiles > 1, wave, ksrc);
  uint32_t vmask = (uint32_t)__ballot(s_idx[ks * 32 + (lane & 31)] >= 0);
  bf16x8 kbuf[PDK];
#pragma unroll
  for (int j = 0; j < PDK; ++j) kbuf[j] = load_k_at(s_k0, j);
  for (int j = 0; j < ntiles; j += 2) {
    compute(j, s_k0, s_k0, rg, s_k1, vmask, kbuf);
    if (j + 1 < ntiles) compute(j + 1, s_k1, s_k1, rg, s_k0, vmask, kbuf);
  }

#pragma unroll
  for (int i = 0; i < C::OT; ++i) M::drain(oacc[i]);

  // ---- finish: row sums over the lane groups sharing a head -------------------
  const float l_sum = xor32_sum(l_part);
  const float m_fin = m_used;
  const int h = g * p.G + (hvalid ? hl : 0);
  const int64_t row = ((int64_t)b * p.Sq + t) * p.Hq + h;
  // Split partials: normalised O of this split in bf16 plus its base-2 LSE
  // (no sink: the combine adds it once).  Final output: the sink joins the
  // denominator (SFA.py:469-478).
  const bool partial = p.num_splits > 1;
  const int64_t nrows = (int64_t)p.B * p.Sq * p.Hq;
  float scale_o;
  if (partial) {
    scale_o = l_sum > 0.f ? 1.f / l_sum : 0.f;
    if (hvalid && hq == 0) p.part_lse[split * nrows + row] = l_sum > 0.f ? m_fin + log2f(l_sum) : kNegInf;
  } else {
    const float sink2 = p.sink ? p.sink[h] * kLog2e : kNegInf;
    const float mm = fmaxf(m_fin, sink2);
    const float fo = (m_fin == kNegInf) ? 0.f : exp2f(m_fin - mm);
    float lt_ = l_sum * fo;
    if (p.sink && mm != kNegInf) lt_ += exp2f(sink2 - mm);
    scale_o = lt_ > 0.f ? fo / lt_ : 0.f;
    if (hvalid && hq == 0)
      p.lse[b * p.l_sb + t * p.l_ss + (int64_t)h * p.l_sh] = lt_ > 0.f ? (mm + log2f(lt_)) * kLn2 : kNegInf;
  }
  // destination of the group's first head row, the same for every lane
  // (lanes of absent heads included: they take part in the staged stores):
  // output (strided) or partial buffer (dense); head hl's row is obase +
  // hl * orstride
  const int64_t row0 = ((int64_t)b * p.Sq + t) * p.Hq + (int64_t)g * p.G;
  bf16* const obase = partial ? p.part_o + ((int64_t)split * nrows + row0) * C::DV
                              : reinterpret_cast<bf16*>(p.out) + b * p.o_sb + t * p.o_ss + (int64_t)(g * p.G) * p.o_sh;
  const int64_t orstride = partial ? C::DV : p.o_sh;

  // the next item (persistent): its loads go out now, under this output
  const int vb2 = PERSIST ? __builtin_amdgcn_readfirstlane(s_claim[ipar ^ 1]) : -1;
  ItemPos it2{};
  if (vb2 >= 0) {
    it2 = item_of(p, vb2);
    item_loads(p, it2, tid, wave, lane);
    item_qdma(p, it2, wave, lane);  // (the Q area is idle: the last S^T has run)
  }

  // ---- output, staged through LDS ---------------------------------------
  // The accumulator layout gives each lane 4-dim pieces of one head, i.e.
  // stores that touch 32 rows per instruction.  Each wave instead writes its
  // heads' bf16 values into a private LDS area, then streams them out with
  // 16-byte stores that each cover whole row segments; every lane takes part
  // in the stores (lanes of absent heads only skip their own writes).
  //  * one pass (not persistent): all DV dims of the wave's 32 heads (row
  //    pitch DV + 8, so the 8-byte writes of the heads fall in distinct banks)
  //    in the tile buffers and the Q area, idle after the tile loop's last
  //    barrier; one 1 KB row per store instruction;
  //  * persistent: four rounds of DV / 4 dims (4 accumulators each, row pitch
  //    DV / 4 + 4) in s_k1 alone, while the next item's Q is gathered into the
  //    Q area and, after the first round, its tile 0 into s_k0; four 256-byte
  //    row segments per store instruction.
  if constexpr (!PERSIST) {
    constexpr int SP = C::DV + 8;
    static_assert(T * SP * 2 <= C::KBUF * 16 && T * SP * 2 <= C::QBUF * 8, "a wave's output block fits an idle buffer");
    char* const stg = wave == 0 ? reinterpret_cast<char*>(s_k0)
                    : wave == 1 ? reinterpret_cast<char*>(s_k1)
                                : reinterpret_cast<char*>(s_q) + (wave - 2) * (C::QBUF * 8);
    bf16* srow = reinterpret_cast<bf16*>(stg) + lt * SP;
#pragma unroll
    for (int ot = 0; ot < C::OT; ++ot) {
#pragma unroll
      for (int q4 = 0; q4 < C::CPL / 4; ++q4) {
        const int dim = ot * T + 4 * C::LG * q4 + 4 * hq;
        bf16x4 v4 = {(bf16)(oacc[ot][4 * q4 + 0] * scale_o), (bf16)(oacc[ot][4 * q4 + 1] * scale_o),
                     (bf16)(oacc[ot][4 * q4 + 2] * scale_o), (bf16)(oacc[ot][4 * q4 + 3] * scale_o)};
        *reinterpret_cast<bf16x4*>(srow + dim) = v4;
      }
      // one accumulator at a time (see the persistent rounds below)
      if (ot + 1 < C::OT) asm volatile("" : "+a"(oacc[ot + 1 < C::OT ? ot + 1 : 0])::"memory");
    }
    const bf16* sbase = reinterpret_cast<const bf16*>(stg);
    bf16* const wbase = obase + (int64_t)(slice * T) * orstride;
#pragma unroll 4
    for (int r = 0; r < T; ++r) {
      if (slice * T + r >= p.G) break;
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(sbase + r * SP + 8 * lane);
      *reinterpret_cast<bf16x8*>(wbase + (int64_t)r * orstride + 8 * lane) = v;
    }
  } else {
    constexpr int NR = 4;                  // rounds
    constexpr int OTR = C::OT / NR;        // accumulators (32-dim tiles) per round
    constexpr int DR = OTR * T;            // dims per round
    constexpr int SPR = DR + 4;            // row pitch (bf16): 66 dwords, so the 32 rows' 8-byte writes fall in distinct banks
    constexpr int LPR = DR / 8;            // lanes per row segment (16 bytes each)
    constexpr int RPI = 64 / LPR;          // row segments per store instruction
    static_assert(C::OT % NR == 0 && 64 % LPR == 0 && T % RPI == 0, "round geometry");
    static_assert(C::kWaves * T * SPR * 2 <= C::KBUF * 16, "the rounds fit one tile buffer");
    bf16* const stg = reinterpret_cast<bf16*>(s_k1) + wave * (T * SPR);
    const int sr = lane / LPR, sc = lane % LPR;  // row within an instruction's group, 16-byte chunk
#pragma unroll
    for (int rd = 0; rd < NR; ++rd) {
#pragma unroll
      for (int o = 0; o < OTR; ++o) {
        const int ot = rd * OTR + o;
#pragma unroll
        for (int q4 = 0; q4 < C::CPL / 4; ++q4) {
          const int dim = o * T + 4 * C::LG * q4 + 4 * hq;
          bf16x4 v4 = {(bf16)(oacc[ot][4 * q4 + 0] * scale_o), (bf16)(oacc[ot][4 * q4 + 1] * scale_o),
                       (bf16)(oacc[ot][4 * q4 + 2] * scale_o), (bf16)(oacc[ot][4 * q4 + 3] * scale_o)};
          *reinterpret_cast<bf16x4*>(stg + lt * SPR + dim) = v4;
        }
        // one accumulator at a time: its writes are issued before the next
        // one's values are read (else the compiler reads all 256 up front)
        if (ot + 1 < C::OT) asm volatile("" : "+a"(oacc[ot + 1 < C::OT ? ot + 1 : 0])::"memory");
      }
#pragma unroll
      for (int j = 0; j < T / RPI; ++j) {
        const int r = j * RPI + sr;  // head within the wave's slice
        const bf16x8 v = *reinterpret_cast<const bf16x8*>(stg + r * SPR + 8 * sc);
        if (slice * T + r < p.G)
          *reinterpret_cast<bf16x8*>(obase + (int64_t)(slice * T + r) * orstride + rd * DR + 8 * sc) = v;
      }
      if (rd == 0 && vb2 >= 0) item_gather0(p, it2, wave, lane);
    }
  }
  if constexpr (!PERSIST) break;
  if (vb2 >= 0) {
    // the wave's last three rounds issued 24 stores after its gathers unless
    // its head slice is partly absent (then some lanes' stores are skipped and
    // the count is not known here): then wait for everything.  (The barrier
    // also ends every staging read of s_k1, which the next item's tile 1
    // overwrites.)
    const bool vm24 = p.G - slice * T >= T;
    ipar ^= 1;
    ntiles = item_stage(p, it2, tid, wave, lane, vm24);
  }
  it = it2;
  vb = vb2;
  }  // items
}

// The one variant: DeepSeek MLA, G = 128 heads (65..128 accepted), d_qk 576 /
// d_v 512 with V the first 512 dims of the K rows.
using CfgMla = FwdCfg<32, 576, 512, 4, 1, true, MLA_QREG, true>;

template <class C>
hipError_t launch(const Params& p, hipStream_t s) {
  const int64_t n = (int64_t)p.B * p.Sq * p.Hkv * p.num_splits;
  if (p.sched) {
    // persistent: one workgroup per CU (the LDS use allows one)
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    const unsigned grid = (unsigned)(n < cus ? n : cus);
    hipLaunchKernelGGL(sched_reset_kernel, dim3(1), dim3(64), 0, s, p.sched);
    if (p.block_table)
      hipLaunchKernelGGL((fwd_mfma_kernel<C, true, true>), dim3(grid), dim3(C::kThreads), 0, s, p);
    else
      hipLaunchKernelGGL((fwd_mfma_kernel<C, false, true>), dim3(grid), dim3(C::kThreads), 0, s, p);
    return hipGetLastError();
  }
  if (p.block_table)
    hipLaunchKernelGGL((fwd_mfma_kernel<C, true, false>), dim3((unsigned)n), dim3(C::kThreads), 0, s, p);
  else
    hipLaunchKernelGGL((fwd_mfma_kernel<C, false, false>), dim3((unsigned)n), dim3(C::kThreads), 0, s, p);
  return hipGetLastError();
}

bool v_is_k_prefix(const Params& p) {
  return p.v == p.k && p.v_sb == p.k_sb && p.v_ss == p.k_ss && p.v_sh == p.k_sh;
}

// contiguous rows are addressed by 32-bit buffer offsets; paged pools by
// 64-bit addresses (pool rows fit an int by the API's check)
bool rows_fit_32bit(const Params& p) {
  if (p.block_table) {
    // the staged pool offsets (units of 2^pool_shift bytes) must fit 31 bits
    const int64_t page_bytes = 2 * p.k_sb, row_bytes = 2 * p.k_ss;
    const int64_t rows_per_page = (int64_t)1 << p.page_shift;
    const int64_t last = (int64_t)(p.num_pages - 1) * page_bytes + (rows_per_page - 1) * row_bytes;
    return p.pool_shift == pool_unit_shift(page_bytes, row_bytes) && (last >> p.pool_shift) < ((int64_t)1 << 31);
  }
  const int64_t kb = 2 * ((int64_t)(p.Skv - 1) * p.k_ss + p.Dqk);
  const int64_t vb = 2 * ((int64_t)(p.Skv - 1) * p.v_ss + p.Dv);
  return kb < (int64_t)kOOB && vb < (int64_t)kOOB && fits_u24(2 * p.k_ss) && fits_u24(2 * p.v_ss);
}

bool mla_supported(const Params& p) {
  return p.Dqk == 576 && p.Dv == 512 && p.G <= 128 && p.G > 64 && v_is_k_prefix(p) && rows_fit_32bit(p);
}

}  // namespace

// Dispatch over the MFMA forward kernels: the MLA kernel above and the
// register-direct d = 128 kernel (sfa_fwd_d128.hip).
int fwd_mfma_tile_keys(const Params& p) {
  if (p.Dqk == 576 && p.Dv == 512) return CfgMla::NKT;
  return 32;  // d = 128 kernel: 32-key tiles
}

int fwd_mfma_idx_cap(const Params& p) { return mla_supported(p) ? kIdxCap : fwd_d128_idx_cap(p); }

// Whether the forward of p runs persistent (its Params then need sched, 8
// zeroed ints): the MLA kernel without split-k over enough items to keep
// every CU busy for many rounds.
bool fwd_mfma_persistent(const Params& p) {
  return mla_supported(p) && p.num_splits == 1 && (int64_t)p.B * p.Sq * p.Hkv >= 4096;
}

bool fwd_mfma_supported(const Params& p) { return mla_supported(p) || fwd_d128_supported(p); }

// The MLA kernel holds all G heads of an item in one workgroup; the d = 128
// kernel one head group of 16.
int fwd_mfma_head_groups(const Params& p) { return mla_supported(p) ? 1 : fwd_d128_head_groups(p); }

hipError_t launch_fwd_mfma(const Params& p, hipStream_t s) {
  if (mla_supported(p)) return launch<CfgMla>(p, s);
  if (fwd_d128_supported(p)) return launch_fwd_d128(p, s);
  return hipErrorNotSupported;
}

}  // namespace sfa

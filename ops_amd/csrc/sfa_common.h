// Shared definitions of the gfx950 sparse flash attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/sfa.h"

namespace sfa {

constexpr float kLog2e = 1.4426950408889634f;  // base-2 softmax, SFA.py:13
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_huge_valf();

// Internal launch parameters shared by every kernel (passed by value as
// kernel arguments).  Element strides; feature dimension contiguous.
struct Params {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* idx;
  const int32_t* kv_lens;
  const float* sink;
  void* out;
  float* lse;
  int64_t q_sb, q_ss, q_sh;
  int64_t k_sb, k_ss, k_sh;
  int64_t v_sb, v_ss, v_sh;
  int64_t i_sb, i_ss, i_sh;
  int64_t o_sb, o_ss, o_sh;
  int64_t l_sb, l_ss, l_sh;
  int B, Sq, Skv, Hq, Hkv, Dqk, Dv, topk, G;
  // paged KV (sfa_fwd_paged): k / v are pools [num_pages][page][Hkv][D] with
  // k_sb / v_sb the page strides; logical key i of sequence b is row
  // i & (page - 1) of page block_table[b * bt_sb + (i >> page_shift)]
  const int32_t* block_table;  // nullptr: contiguous [B][Skv][Hkv][D] k / v
  int64_t bt_sb;
  int page_shift;
  int num_pages;
  int pool_shift;     // paged MLA gathers: staged pool offsets are in units of 2^pool_shift bytes
  float scale;        // softmax scale
  float scale_log2;   // scale * log2(e): scores in base-2 units
  // split-k partial results (forward, num_splits > 1)
  int num_splits;
  int split_len;      // slots per split (multiple of the key tile)
  __bf16* part_o;     // [num_splits][B*Sq*Hq][Dv] bf16, normalised by the split's own sum
  float* part_lse;    // [num_splits][B*Sq*Hq], base-2 log-sum-exp of the split (-inf if empty)
  int* sched;         // persistent forward: 8 claim counters (one per XCD), zeroed before the launch
  // backward
  const void* dout;
  int64_t do_sb, do_ss, do_sh;
  void* dq;
  int64_t dq_sb, dq_ss, dq_sh;
  float* dk_acc;      // [B, Skv, Hkv, Dqk] fp32 accumulators
  float* dv_acc;      // [B, Skv, Hkv, Dv]  fp32 accumulators
  float* delta;       // [B*Sq*Hq] Σ O·dO − dlse
  const float* dlse;  // gradient w.r.t. lse (lse's strides) or nullptr
  float* dsink;       // [Hq] written by dsink_kernel (fixed-order reduction over the rows)
  // deterministic dK/dV (SFA_DKV_CSR): index inversion at block granularity
  uint32_t* kmap;     // [B][Hkv][Sq][kmap_w] membership bitmap: bit k of row t = key k is selected
  int kmap_w;         // 32-bit words per bitmap row (multiple of 4)
  uint8_t* dup;       // [B][Sq][Hkv][topk] 1 = slot repeats an earlier slot's key (handled by atomics)
  int* blist;         // [B][Hkv][nkb][nqb] non-empty query blocks of each key block, ascending
  int* bstart;        // [B][Hkv][nkb][max_chunks + 1] blist index of each 128-query-block chunk's first entry
  float* dkv_part;    // [B][Hkv][nkb][max_chunks][128][2 D] fp32 partial dK | dV per chunk
  float* rowc;        // [2][B*Sq*Hq] per row: -lse / scale, then -δ (written by the δ pass)
  int* kctr;          // key-major claims: [0] counter, [1] listed units (both set by unit_order_kernel)
  int* uorder;        // [B*Hkv*nkb*max_chunks] key-major units in claim order (non-empty ones only)
  int nkb, nqb;       // key blocks (128 keys), query blocks (128 / G queries)
  int lg_g;           // log2(G)
  int max_chunks;     // chunks per key block (query blocks / chunk, rounded up)
};

typedef __bf16 bf16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ float to_f32(T x) { return static_cast<float>(x); }

template <typename T>
__device__ __forceinline__ T from_f32(float x) { return static_cast<T>(x); }

__device__ __forceinline__ int bound_of(const Params& p, int b) {
  if (p.kv_lens == nullptr) return p.Skv;
  int n = p.kv_lens[b];
  return n < p.Skv ? n : p.Skv;
}

// Pool row (page * page_size + offset) of logical key id of sequence b in
// paged mode, or -1 when the slot is invalid (id outside [0, bound)) or its
// page is unmapped (block-table entry outside [0, num_pages)).
__device__ __forceinline__ int paged_row(const Params& p, int b, int id, int bound) {
  if (id < 0 || id >= bound) return -1;
  const int pg = p.block_table[b * p.bt_sb + (id >> p.page_shift)];
  if (pg < 0 || pg >= p.num_pages) return -1;
  return (pg << p.page_shift) | (id & ((1 << p.page_shift) - 1));
}

// Unit (log2 bytes) of the pool offsets the paged MLA gathers stage: the
// largest power of two up to 2^7 that divides both the page and the row
// stride, so an offset of a pool up to 2^(31 + shift) bytes fits 31 bits.
__host__ __device__ inline int pool_unit_shift(int64_t page_bytes, int64_t row_bytes) {
  const uint64_t m = (uint64_t)(page_bytes | row_bytes);
  int sh = 0;
  while (sh < 7 && ((m >> sh) & 1u) == 0) ++sh;
  return sh;
}

// The staged id of a slot: the key row itself (contiguous k / v) or its pool
// row (paged), -1 for an invalid slot.
template <bool PAGED>
__device__ __forceinline__ int staged_id(const Params& p, int b, int id, int bound) {
  if (PAGED) return paged_row(p, b, id, bound);
  return (id >= 0 && id < bound) ? id : -1;
}

// The staged form of a slot for the paged MLA gathers: the byte offset of its
// pool row from the (kv head's) pool base in units of 2^pool_shift bytes, -1
// for an invalid slot (the tile loop then forms a row's 64-bit address with
// one shift and one add instead of the page arithmetic).
__device__ __forceinline__ uint64_t pool_row_offset(uint32_t r, int shift, uint64_t page_bytes, uint32_t row_bytes);
__device__ __forceinline__ int staged_pool_off(const Params& p, int b, int id, int bound) {
  const int r = paged_row(p, b, id, bound);
  if (r < 0) return -1;
  return (int)(pool_row_offset((uint32_t)r, p.page_shift, (uint64_t)(2 * p.k_sb), (uint32_t)(2 * p.k_ss)) >> p.pool_shift);
}

// paged_row() of N slots at once: the N block-table loads are issued before
// any of them is used (buffer loads over the table's rows up to the last page
// any valid key can use; invalid slots read out of range, i.e. 0, and are
// dropped), so they cost one memory round trip, not N.  OFFS: return
// staged_pool_off() values instead of pool rows.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes);
template <int N, bool OFFS>
__device__ __forceinline__ void paged_rows(const Params& p, int b, const int (&id)[N], int bound, int (&out)[N]) {
  const int64_t pages = ((int64_t)p.Skv + (1 << p.page_shift) - 1) >> p.page_shift;
  const uint32_t tbytes = (uint32_t)(4 * ((int64_t)(p.B - 1) * p.bt_sb + pages));
  const __amdgpu_buffer_rsrc_t rt = make_rsrc(p.block_table, tbytes);
  int pg[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const bool ok = id[i] >= 0 && id[i] < bound;
    const uint32_t off = ok ? 4u * (uint32_t)((int64_t)b * p.bt_sb + (id[i] >> p.page_shift)) : tbytes;
    pg[i] = (int)__builtin_amdgcn_raw_buffer_load_b32(rt, off, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const bool ok = id[i] >= 0 && id[i] < bound && pg[i] >= 0 && pg[i] < p.num_pages;
    const int r = (pg[i] << p.page_shift) | (id[i] & ((1 << p.page_shift) - 1));
    if constexpr (OFFS)
      out[i] = ok ? (int)(pool_row_offset((uint32_t)r, p.page_shift, (uint64_t)(2 * p.k_sb), (uint32_t)(2 * p.k_ss)) >>
                          p.pool_shift)
                  : -1;
    else
      out[i] = ok ? r : -1;
  }
}

// Index row of a work item, in two phases so that its global loads are in
// flight together with whatever the caller issues in between (a loop that
// stores each value to LDS as it arrives compiles to one memory round trip
// per iteration).  load(): thread tid reads slots tid, tid + THREADS, ...
// (CAP / THREADS coalesced loads, slots past nslots read nothing); store():
// writes the staged ids (invalid -> -1, padding -1 up to nstage <= CAP) and
// returns 1 + the last of this thread's slots that holds a valid id (0 if
// none), from which the caller can drop the trailing all-padding tiles.
template <int CAP, int THREADS>
struct IdxStage {
  static constexpr int IPT = CAP / THREADS;
  static_assert(CAP % THREADS == 0, "slots split evenly over the threads");
  int v[IPT];
  __device__ __forceinline__ void load(const int32_t* irow, int nslots, int tid) {
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const int i = tid + j * THREADS;
      v[j] = i < nslots ? irow[i] : -1;
    }
  }
  // load() through a buffer resource over the row's nslots ids: slots past it
  // read 0 instead of being selected to -1 (store() and store_offsets() test
  // the slot index), so no instruction waits for the loads here
  __device__ __forceinline__ void load_buf(__amdgpu_buffer_rsrc_t rs, int tid) {
#pragma unroll
    for (int j = 0; j < IPT; ++j) v[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, 4u * (uint32_t)(tid + j * THREADS), 0, 0);
  }
  template <bool PAGED>
  __device__ __forceinline__ int store(const Params& p, int b, int bound, int nslots, int nstage, int* s_idx,
                                       int tid) {
    int st[IPT];
    if constexpr (PAGED) {
      int id[IPT];
#pragma unroll
      for (int j = 0; j < IPT; ++j) id[j] = tid + j * THREADS < nslots ? v[j] : -1;
      paged_rows<IPT, false>(p, b, id, bound, st);
    } else {
#pragma unroll
      for (int j = 0; j < IPT; ++j) st[j] = tid + j * THREADS < nslots ? staged_id<false>(p, b, v[j], bound) : -1;
    }
    int used = 0;
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      if (tid + j * THREADS < nstage) s_idx[tid + j * THREADS] = st[j];
      if (st[j] >= 0) used = tid + j * THREADS + 1;
    }
    return used;
  }
  // store() for the paged MLA gathers: each slot's scaled pool offset
  // (staged_pool_off)
  __device__ __forceinline__ int store_pool_offsets(const Params& p, int b, int bound, int nslots, int nstage,
                                                    int* s_idx, int tid) {
    int st[IPT], id[IPT];
#pragma unroll
    for (int j = 0; j < IPT; ++j) id[j] = tid + j * THREADS < nslots ? v[j] : -1;
    paged_rows<IPT, true>(p, b, id, bound, st);
    int used = 0;
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      if (tid + j * THREADS < nstage) s_idx[tid + j * THREADS] = st[j];
      if (st[j] >= 0) used = tid + j * THREADS + 1;
    }
    return used;
  }
  // store() for contiguous rows, staging each slot's row byte offset
  // id * row_bytes instead of the id (invalid: oob, which has bit 31 set, so
  // the sign still tells validity); offsets must stay below 2^31.
  __device__ __forceinline__ int store_offsets(int bound, int nslots, int nstage, int* s_idx, int tid,
                                               uint32_t row_bytes, uint32_t oob) {
    int used = 0;
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const bool ok = tid + j * THREADS < nslots && v[j] >= 0 && v[j] < bound;
      if (tid + j * THREADS < nstage) s_idx[tid + j * THREADS] = ok ? (int)__umul24((uint32_t)v[j], row_bytes) : (int)oob;
      if (ok) used = tid + j * THREADS + 1;
    }
    return used;
  }
};

__device__ __forceinline__ int wave_max_int(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = max(x, __shfl_xor(x, o, 64));
  return x;
}
__device__ __forceinline__ int wave_sum_int(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

// Byte offset of pool row r from the pool base (paged mode): page r >> shift
// at page_bytes, row r & mask at row_bytes (64-bit: pools may exceed 4 GiB).
__device__ __forceinline__ uint64_t pool_row_offset(uint32_t r, int shift, uint64_t page_bytes, uint32_t row_bytes) {
  return (uint64_t)(r >> shift) * page_bytes + (uint64_t)(r & ((1u << shift) - 1u)) * row_bytes;
}

// Zeros that padding rows of the 64-bit (paged) gathers read instead of an
// out-of-range buffer offset: one row of up to 1280 bytes (one copy per
// translation unit that uses it).
static __device__ const u32x4 kZeroRow[80] = {};

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  return x;
}

// Buffer resource over [base, base + bytes): loads at offsets >= bytes return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

constexpr uint32_t kOOB = 0x80000000u;  // buffer offset that always reads 0
// cache-policy operand of the buffer load/store builtins on gfx950: nt
// (non-temporal), for data one pass writes and another reads exactly once
constexpr int kCpolNT = 2;

// The contiguous-row gathers form row offsets with __umul24(row id, row
// bytes), which multiplies the low 24 bits of each operand: a kernel that
// does so is only eligible when its row byte strides are below 2^24 (row ids
// are below 2^24 whenever the offsets fit 31 bits and a row is >= 256 bytes).
inline bool fits_u24(int64_t x) { return x >= 0 && x < ((int64_t)1 << 24); }

// Top-k index producer (sfa_indexer.hip): indexer scores + top-k selection.
struct IndexerParams {
  const void* q;          // [B, Sq, H, D] bf16 or fp8 e4m3
  const void* k;          // [B, Skv, D] bf16 or fp8 e4m3
  const float* k_scale;   // fp8: [B, Skv] positive per-token scales, or nullptr
  int64_t ks_sb;
  const float* w;         // [B, Sq, H] float32, head stride 1
  const int32_t* kv_lens; // [B] or nullptr
  int32_t* idx;           // [B, Sq, topk] int32 out, slot stride 1
  float* logits;          // rows [g_t0, ...) of the scores: [B, rows, Skv], row stride g_ss
  int64_t q_sb, q_ss, q_sh;
  int64_t k_sb, k_ss;
  int64_t w_sb, w_ss;
  int64_t i_sb, i_ss;
  int64_t g_sb, g_ss;
  int g_t0;               // query of logits row 0 (the workspace holds a chunk of queries)
  int B, Sq, Skv, H, D, topk;
  bool fp8;
  // segmented selection (nseg > 1): per launched row nseg candidate lists
  // of topk keys (rounded up to 4) and their order keys, segments of seglen
  // keys
  int32_t* cand;
  uint32_t* cand_key;
  int nseg, seglen;
};

}  // namespace sfa

// Launchers implemented in the .hip translation units; return a HIP error.
namespace sfa {
hipError_t launch_fwd_generic(const Params& p, int dtype, hipStream_t s);
hipError_t launch_bwd_generic(const Params& p, int dtype, hipStream_t s);
hipError_t launch_zero_f32(float* ptr, size_t n, hipStream_t s);
hipError_t launch_bwd_delta(const Params& p, int dtype, hipStream_t s);
hipError_t launch_bwd_dsink(const Params& p, hipStream_t s);  // after launch_bwd_delta
hipError_t launch_bwd_finish(const Params& p, int dtype, void* dk, int64_t dk_sb, int64_t dk_ss, int64_t dk_sh,
                             void* dv, int64_t dv_sb, int64_t dv_ss, int64_t dv_sh, hipStream_t s);
// shared K/V rows: dk = dK (+ dV on the first Dv dims when add_dv; the MLA
// backward accumulates both into dk_acc itself)
hipError_t launch_bwd_finish_merged(const Params& p, int dtype, void* dk, int64_t dk_sb, int64_t dk_ss,
                                    int64_t dk_sh, bool add_dv, hipStream_t s);
hipError_t launch_combine(const Params& p, int dtype, hipStream_t s);
// MFMA paths: return hipErrorNotSupported when the shape has no variant.
hipError_t launch_fwd_mfma(const Params& p, hipStream_t s);  // paged when p.block_table != nullptr
bool fwd_mfma_supported(const Params& p);
int fwd_mfma_tile_keys(const Params& p);
int fwd_mfma_idx_cap(const Params& p);  // index slots one work item (split) stages
bool fwd_mfma_persistent(const Params& p);  // needs Params::sched (8 ints of workspace)
// index rows in ascending key order, then -1 (sfa_idx_sort.hip): out holds
// B * Sq * Hkv rows of topk slots, contiguous
bool idx_sort_supported(const Params& p);
hipError_t launch_idx_sort(const Params& p, int32_t* out, hipStream_t s);
int fwd_mfma_head_groups(const Params& p);  // workgroups per (work item, split): head groups
int fwd_d128_idx_cap(const Params& p);
// d = 128: register-direct gather, 16 heads per wave (sfa_fwd_d128.hip)
bool fwd_d128_supported(const Params& p);
bool fwd_d128g_supported(const Params& p);  // 16 < G <= 128, contiguous: one workgroup per item, a shared tile
int fwd_d128_head_groups(const Params& p);  // workgroups per (item, split): ceil(G / 16), or 1 (shared tile)
hipError_t launch_fwd_d128(const Params& p, hipStream_t s);
hipError_t launch_bwd_mfma(const Params& p, hipStream_t s);
bool bwd_mfma_supported(const Params& p);
// MLA shared-KV backward (sfa_bwd_mla.hip): dQ pass + dK/dV pass over a chunk
// of work items (det: plus index maps and the ordered reduction, each
// launched on its own so that they can run beside the dQ passes); a chunk needs
// P / dS (bwd_mla_pd_bytes_per_item per item) and, det, a buffer set
// (bwd_mla_set_bytes_per_item per item)
bool bwd_mla_supported(const Params& p);
bool bwd_mla_det_supported(const Params& p);  // deterministic dK/dV: Skv <= 65536
int bwd_mla_max_chunk_items(bool det);  // the deterministic reduction stages a chunk's items in LDS
size_t bwd_mla_bytes_per_item(const Params& p, bool det);
size_t bwd_mla_pd_bytes_per_item(const Params& p);   // P / dS
size_t bwd_mla_set_bytes_per_item(const Params& p);  // deterministic: contributions and index maps
hipError_t launch_bwd_mla_map(const Params& p, int64_t item0, int n, void* set, hipStream_t s);
hipError_t launch_bwd_mla_dq(const Params& p, int64_t item0, int n, void* pd, hipStream_t s);
hipError_t launch_bwd_mla_dkv(const Params& p, int64_t item0, int n, const void* pd, void* set, bool det,
                              hipStream_t s);
hipError_t launch_bwd_mla_reduce(const Params& p, int64_t item0, int n, void* set, int cus, hipStream_t s);
// dQ / dsink pass of the deterministic backward, d = 128 (sfa_bwd_dq.hip)
bool bwd_dq_supported(const Params& p);
hipError_t launch_bwd_dq(const Params& p, hipStream_t s);   // dQ of the deterministic scheme
hipError_t launch_bwd_dup(const Params& p, hipStream_t s);  // dK/dV of repeated-key slots (fp32 atomics)
// deterministic dK/dV
bool bwd_csr_supported(const Params& p);
void csr_geometry(Params& p);                 // fills kmap_w, nkb, nqb, lg_g, max_chunks
size_t csr_workspace_bytes(const Params& p);  // after csr_geometry
void csr_bind_workspace(Params& p, void* ws); // carves kmap / dup / blist / bcount / dkv_part / rowc
hipError_t launch_csr_index(const Params& p, hipStream_t s);  // bitmap, duplicate flags, block lists
hipError_t launch_csr_dkv(const Params& p, hipStream_t s);    // key-major dK/dV partials + reduction
// top-k index producer: queries [t_begin, t_end) of every sequence
int indexer_query_block(const IndexerParams& p);
hipError_t launch_indexer_logits(const IndexerParams& p, int t_begin, int t_end, hipStream_t s);
hipError_t launch_topk_select(const IndexerParams& p, int t_begin, int t_end, hipStream_t s);
// Segments per row of the selection for a launch of `rows` queries per
// sequence (1: one workgroup per row), and their length.
int topk_segments(const IndexerParams& p, int rows);
int topk_seglen(const IndexerParams& p, int nseg);
}  // namespace sfa

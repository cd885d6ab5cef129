// Deterministic dK/dV for the gfx950 sparse flash attention backward
// (SFA_DKV_CSR), d_qk = d_v = 128 and G = 1, 2, 4, ..., 128 query heads per
// KV head (a power of two).
//
// Reference: `_attn_bwd_dk_dv` / `_inner_dkv` (SFA.py:1005-1145, 719-853)
// gathers, per query tile, the selected K/V rows and scatters dK/dV with
// atomics (SFA.py:849-853).  This path produces the same sums without
// atomics and in a fixed order:
//
//  1. Index inversion.  A membership bitmap kmap[b][g][t] (bit k = key k is
//     selected by query t) is built from the index rows; a slot whose key
//     already has its bit (a repeated key in one row) is flagged in `dup`
//     and its contribution is added by the query-major kernel with atomics
//     instead (repeats are the only non-deterministic case; the workloads
//     have none).  Then, for every key block of 128 keys, the ascending list
//     of query blocks (128 query-head rows = 128 / G queries) that select at
//     least one of its keys (`blist`, a per-key-block CSR at block
//     granularity), with `bstart` marking where each chunk of kChunk
//     consecutive query blocks (an absolute query range) begins in it.
//  2. Key-major recompute.  A work unit is a key block (each wave 32 keys, K
//     and V rows kept in registers) and one chunk: the listed query blocks in
//     one absolute range of kChunk query blocks.  One persistent workgroup
//     per CU claims units from a counter, longest first and otherwise in
//     chunk-descending order, so the units that run together are key blocks
//     of the same query range and read the same query blocks.  Per query block it recomputes, for every (row, key)
//     pair of the block, S = Q K^T and dP = dO V^T (32x32x16 MFMA, rows as
//     M, keys as N), P = 2^(S scale log2e - lse2) and dS = P (dP - δ) masked
//     by the bitmap, and accumulates dV^T += dO^T P and dK^T += Q^T dS in
//     AGPRs (the C layout of S is the B layout of these products; the A
//     operands are transposing LDS reads of 4-row runs in the matching
//     order).  Pairs that are not selected get P = 0, so a block costs the
//     same whatever its density.
//  3. Reduction.  The chunks of a key block write fp32 partials; a reduction
//     kernel adds them in chunk order into the per-key accumulators.

#include "sfa_common.h"
#include "sfa_lds.h"
#include "sfa_mfma.h"

namespace sfa {
namespace {

constexpr int kKeyBlock = 128;          // keys per key block (4 waves x 32)
constexpr int kRowBlock = 128;          // query-head rows per query block
constexpr int kChunk = 128;             // query blocks per workgroup (64 measured slower)
constexpr int kD = 128;                 // head dim (d_qk = d_v)
constexpr int kCH = kD / 8;             // 16-byte chunks per row
constexpr int kTB = kRowBlock * kCH;    // slots per Q or dO block buffer
static_assert(kTB % 64 == 0 && kCH == 16, "block buffers: 4 rows per DMA instruction");

// Q / dO block rows are stored unpadded (16 slots) with chunk c of row r at
// slot c ^ blk_swz(r).  Both operand read patterns are then bank-conflict
// free (64 banks x 4 bytes, 256 bytes per pass):
//  * b128 reads of one chunk of 16 consecutive rows (S / dP A operands):
//    blk_swz is a bijection on every 16 consecutive rows;
//  * transposing reads of 4 consecutive rows x an aligned group of 4 chunks
//    (dV / dK A operands): blk_swz(4m + i) = 4 i + (m & 3) sends the group of
//    each of the 4 rows to a different group.
__device__ __forceinline__ int blk_swz(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }

// A pointer that is the same in every lane, read from the first lane (a
// buffer descriptor built from it then stays scalar)
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* ptr) {
  const uint64_t v = reinterpret_cast<uint64_t>(ptr);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// ---- 1a. membership bitmap and repeated-slot flags ------------------------
// One workgroup per index row (b, t, g): the row's bitmap is built with LDS
// atomics, then written out whole (no global atomics, no separate clearing).
constexpr int kMaxMapWords = 8192;  // LDS words per bitmap row: Skv <= 262144
__global__ __launch_bounds__(256) void csr_scatter_kernel(Params p) {
  __shared__ uint32_t s_map[kMaxMapWords];
  int wi = blockIdx.x;
  const int g = wi % p.Hkv;
  wi /= p.Hkv;
  const int t = wi % p.Sq;
  const int b = wi / p.Sq;
  const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh;
  uint32_t* mrow = p.kmap + (((int64_t)b * p.Hkv + g) * p.Sq + t) * p.kmap_w;
  uint8_t* drow = p.dup + (((int64_t)b * p.Sq + t) * p.Hkv + g) * p.topk;
  const int bound = bound_of(p, b);
  for (int w = threadIdx.x; w < p.kmap_w; w += 256) s_map[w] = 0u;
  __syncthreads();
  for (int s = threadIdx.x; s < p.topk; s += 256) {
    const int id = irow[s];
    uint8_t rep = 0;
    if (id >= 0 && id < bound) {
      const uint32_t bit = 1u << (id & 31);
      rep = (atomicOr(&s_map[id >> 5], bit) & bit) ? 1 : 0;
    }
    drow[s] = rep;
  }
  __syncthreads();
  for (int w = threadIdx.x; w < p.kmap_w; w += 256) mrow[w] = s_map[w];
}

// ---- 1b. per key block: ascending list of non-empty query blocks -----------
__global__ __launch_bounds__(256) void csr_blocklist_kernel(Params p) {
  __shared__ int s_cnt[4];
  int wi = blockIdx.x;
  const int kb = wi % p.nkb;
  wi /= p.nkb;
  const int g = wi % p.Hkv;
  const int b = wi / p.Hkv;
  const int nq = kRowBlock >> p.lg_g;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t* mrow = p.kmap + ((int64_t)b * p.Hkv + g) * p.Sq * p.kmap_w + kb * 4;
  const int64_t bgk = ((int64_t)b * p.Hkv + g) * p.nkb + kb;
  int* list = p.blist + bgk * p.nqb;
  int* start = p.bstart + bgk * (p.max_chunks + 1);
  constexpr int kCPI = 256 / kChunk;  // chunks per iteration
  constexpr int kWPC = kChunk / 64;   // waves per chunk
  static_assert(kCPI * kChunk == 256 && kWPC * 64 == kChunk, "an iteration covers whole chunks of whole waves");
  int total = 0;
  for (int q0 = 0; q0 < p.nqb; q0 += 256) {
    const int qb = q0 + tid;
    bool any = false;
    if (qb < p.nqb) {
      const int t0 = qb * nq;
      const int t1 = min(p.Sq, t0 + nq);
      for (int t = t0; t < t1 && !any; ++t) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(mrow + (int64_t)t * p.kmap_w);
        any = (w.x | w.y | w.z | w.w) != 0u;
      }
    }
    const uint64_t m = __ballot(any);
    if (lane == 0) s_cnt[wave] = __popcll(m);
    __syncthreads();
    int pos = total + __popcll(m & ((1ull << lane) - 1ull));
    for (int w = 0; w < wave; ++w) pos += s_cnt[w];
    if (any) list[pos] = qb;
    // chunk starts: the kChunk query blocks of chunk c0 + i are those of
    // waves kWPC i .. kWPC (i + 1) - 1 of this iteration
    const int c0 = q0 / kChunk;
    if (tid == 0) {
      int acc = total;
#pragma unroll
      for (int i = 0; i < kCPI; ++i) {
        if (c0 + i <= p.max_chunks) start[c0 + i] = acc;
#pragma unroll
        for (int w = 0; w < kWPC; ++w) acc += s_cnt[kWPC * i + w];
      }
    }
    total += s_cnt[0] + s_cnt[1] + s_cnt[2] + s_cnt[3];
    __syncthreads();
  }
  if (tid == 0) start[p.max_chunks] = total;
}

// The same per index row, one wave per row (4 rows per workgroup, no block
// barrier): for bitmap rows of at most kWaveMapWords words.  A wave's LDS
// operations complete in program order, so its zeroing, its atomics and its
// final reads need no barrier between them.
constexpr int kWaveMapWords = 1024;  // Skv <= 32768
__global__ __launch_bounds__(256) void csr_scatter_wave_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) uint32_t s_map[4][kWaveMapWords];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t nrows = (int64_t)p.B * p.Sq * p.Hkv;
  const int64_t wi = (int64_t)blockIdx.x * 4 + wave;
  if (wi >= nrows) return;  // the whole wave
  const int g = (int)(wi % p.Hkv);
  const int t = (int)((wi / p.Hkv) % p.Sq);
  const int b = (int)(wi / ((int64_t)p.Hkv * p.Sq));
  const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh;
  uint32_t* mrow = p.kmap + (((int64_t)b * p.Hkv + g) * p.Sq + t) * p.kmap_w;
  uint8_t* drow = p.dup + (((int64_t)b * p.Sq + t) * p.Hkv + g) * p.topk;
  const int bound = bound_of(p, b);
  uint32_t* map = s_map[wave];
  for (int w = lane; w < p.kmap_w; w += 64) map[w] = 0u;
  __builtin_amdgcn_wave_barrier();
  for (int s = lane; s < p.topk; s += 64) {
    const int id = irow[s];
    uint8_t rep = 0;
    if (id >= 0 && id < bound) {
      const uint32_t bit = 1u << (id & 31);
      rep = (atomicOr(&map[id >> 5], bit) & bit) ? 1 : 0;
    }
    drow[s] = rep;
  }
  __builtin_amdgcn_wave_barrier();
  // kmap_w is a multiple of 4: 16-byte stores
  for (int w = 4 * lane; w < p.kmap_w; w += 256)
    *reinterpret_cast<u32x4*>(mrow + w) = *reinterpret_cast<const u32x4*>(map + w);
}

// ---- 1c. the key-major kernel's claim order --------------------------------
// Units u = (chunk, key block, (b, g)) in base order: chunk-descending, then
// key block, then (b, g).  The non-empty units are listed longest first, in
// classes of 16 query blocks (a unit of n listed query blocks is in class
// (kChunk - n) / 16), each class in base order: the full units keep their
// grouping by query range (the units that run together share their query
// blocks in L2), and the short ones, claimed last, fill the end of the
// key-major kernel.  One workgroup: a unit's position is its class's start
// plus the count of earlier units of its class (ballots, then a prefix over
// the waves of the tile and the tiles before it).
constexpr int kClasses = kChunk / 16;
__global__ __launch_bounds__(1024) void unit_order_kernel(Params p) {
  __shared__ int s_cnt[16][kClasses];
  __shared__ int s_start[kClasses];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nbg = p.B * p.Hkv, per_chunk = nbg * p.nkb, nunits = per_chunk * p.max_chunks;
  auto cls = [&](int u) -> int {  // class of unit u, -1 if it has no query block
    const int c = p.max_chunks - 1 - u / per_chunk;
    const int kb = (u % per_chunk) / nbg, bg = (u % per_chunk) % nbg;
    const int* start = p.bstart + ((int64_t)bg * p.nkb + kb) * (p.max_chunks + 1);
    const int n = start[c + 1] - start[c];
    return n > 0 ? (kChunk - n) / 16 : -1;
  };
  // class sizes
  int cnt[kClasses] = {};
  for (int u = tid; u < nunits; u += 1024) {
    const int k = cls(u);
#pragma unroll
    for (int j = 0; j < kClasses; ++j) cnt[j] += k == j;
  }
#pragma unroll
  for (int j = 0; j < kClasses; ++j) {
    const int w = wave_sum_int(cnt[j]);
    if (lane == 0) s_cnt[wave][j] = w;
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int j = 0; j < kClasses; ++j) {
      s_start[j] = acc;
      for (int w = 0; w < 16; ++w) acc += s_cnt[w][j];
    }
    p.kctr[0] = 0;
    p.kctr[1] = acc;
  }
  __syncthreads();
  // positions, tile by tile in base order
  for (int u0 = 0; u0 < nunits; u0 += 1024) {
    const int u = u0 + tid;
    const int k = u < nunits ? cls(u) : -1;
    int rank = 0;
#pragma unroll
    for (int j = 0; j < kClasses; ++j) {
      const uint64_t m = __ballot(k == j);
      if (lane == 0) s_cnt[wave][j] = __popcll(m);
      if (k == j) rank = __popcll(m & ((1ull << lane) - 1ull));
    }
    __syncthreads();
    if (k >= 0) {
      int pos = s_start[k] + rank;
      for (int w = 0; w < wave; ++w) pos += s_cnt[w][k];
      p.uorder[pos] = u;
    }
    __syncthreads();
    if (tid < kClasses) {
      int t = 0;
      for (int w = 0; w < 16; ++w) t += s_cnt[w][tid];
      s_start[tid] += t;
    }
    __syncthreads();
  }
}

// ---- 2. key-major dK / dV ---------------------------------------------------
// LDS: Q and dO blocks double buffered (row r = query (r >> lg_g), head
// (r & (G - 1)); swizzled, see blk_swz), each row's lse and δ, and per wave the
// bitmap word of its 32 keys for each row.  Buffers are separate arrays so
// reads of one are not made to wait for DMA into the other.
__global__ __launch_bounds__(256, 1) void dkv_keymajor_kernel(Params p_arg) {
  typedef Mfma<32> M;
  typedef M::acc_t acc_t;
  __shared__ u32x4 s_q0[kTB];
  __shared__ u32x4 s_q1[kTB];
  __shared__ u32x4 s_d0[kTB];
  __shared__ u32x4 s_d1[kTB];
  __shared__ __attribute__((aligned(16))) float s_lse0[kRowBlock];
  __shared__ __attribute__((aligned(16))) float s_lse1[kRowBlock];
  __shared__ __attribute__((aligned(16))) float s_dlt0[kRowBlock];
  __shared__ __attribute__((aligned(16))) float s_dlt1[kRowBlock];
  __shared__ __attribute__((aligned(16))) uint32_t s_msk0[4][kRowBlock];
  __shared__ __attribute__((aligned(16))) uint32_t s_msk1[4][kRowBlock];
  __shared__ int s_list[kChunk];
  // claimed units by parity: unit i's successor is claimed during unit i and
  // published in the other slot behind unit i's barriers
  __shared__ int s_unit[2];

  // Units are claimed from one counter in the order unit_order_kernel lists
  // them (the full ones first, grouped by query range; the short ones last).
  // Claiming balances the CUs however unequal the units are (a fixed unit ->
  // workgroup mapping leaves CUs idle: workgroups are dispatched to the XCDs
  // in turn, so an XCD whose units are longer holds back the dispatch to the
  // others).  A claim is published as the unit itself, or -1 past the list.
  const int nbg = p_arg.B * p_arg.Hkv;
  const int per_chunk = nbg * p_arg.nkb;
  // (an offset the compiler cannot prove uniform keeps the atomic a single
  // lane's: for a uniform address it is rewritten into a wave reduction that
  // waits for every load in flight)
  auto claim = [](const Params& q) {
    int o = 0;
    asm volatile("" : "+v"(o));
    const int i = atomicAdd(q.kctr + o, 1);
    return i < q.kctr[1] ? q.uorder[i] : -1;
  };
  if (threadIdx.x == 0) s_unit[0] = claim(p_arg);
  __syncthreads();
  int par = 0;
  for (;;) {
  const Params& p = p_arg;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // (read as uniform: a value loaded from LDS is a per-lane value to the
  // compiler, and every address derived from it would be built per lane)
  const int u = __builtin_amdgcn_readfirstlane(s_unit[par]);
  if (u < 0) break;
  // the successor's claim: the atomic goes out now and its result is read at
  // the end of the unit (waiting for it here would also wait for this
  // workgroup's partial stores of the previous unit, still in flight)
  int claim_i = 0;
  if (tid == 0) {
    int o = 0;
    asm volatile("" : "+v"(o));
    claim_i = atomicAdd(p.kctr + o, 1);
  }
  const int c = p.max_chunks - 1 - u / per_chunk;
  const int kb = (u % per_chunk) / nbg;
  const int bg = (u % per_chunk) % nbg;
  const int g = bg % p.Hkv;
  const int b = bg / p.Hkv;
  const int64_t bgk = ((int64_t)b * p.Hkv + g) * p.nkb + kb;
  const int* start = p.bstart + bgk * (p.max_chunks + 1);
  const int e0 = __builtin_amdgcn_readfirstlane(start[c]);
  const int nblk = __builtin_amdgcn_readfirstlane(start[c + 1]) - e0;
  if (nblk <= 0) {  // no query block of this chunk selects the key block
    if (tid == 0) s_unit[par ^ 1] = claim_i < p.kctr[1] ? p.uorder[claim_i] : -1;
    par ^= 1;
    __syncthreads();
    continue;
  }
  for (int i = tid; i < nblk; i += 256) s_list[i] = p.blist[bgk * p.nqb + e0 + i];

  const int G = p.G, lg = p.lg_g;
  const int nq = kRowBlock >> lg;
  const int n = lane & 31, g2 = lane >> 5;
  const int key = kb * kKeyBlock + wave * 32 + n;

  // K and V rows of the lane's key as the B operands of S = Q K^T and
  // dP = dO V^T: step s holds dims 16 s + 8 g2 .. +7 (keys past Skv: zeros)
  bf16x8 kB[kD / 16], vB[kD / 16];
  {
    const bool ok = key < p.Skv;
    const bf16* kr = reinterpret_cast<const bf16*>(p.k) + b * p.k_sb + (int64_t)(ok ? key : 0) * p.k_ss +
                     g * p.k_sh + 8 * g2;
    const bf16* vr = reinterpret_cast<const bf16*>(p.v) + b * p.v_sb + (int64_t)(ok ? key : 0) * p.v_ss +
                     g * p.v_sh + 8 * g2;
#pragma unroll
    for (int s = 0; s < kD / 16; ++s) {
      kB[s] = ok ? *reinterpret_cast<const bf16x8*>(kr + 16 * s) : bf16x8{};
      vB[s] = ok ? *reinterpret_cast<const bf16x8*>(vr + 16 * s) : bf16x8{};
    }
  }

  // buffer resources (ranges checked on the host to fit 31 bits; the bases
  // are the unit's, the same in every lane, and are read as such so that no
  // load waits on a loop over distinct descriptors)
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(
      uniform_ptr(reinterpret_cast<const bf16*>(p.q) + b * p.q_sb + (int64_t)(g * G) * p.q_sh),
      (uint32_t)(2 * ((int64_t)(p.Sq - 1) * p.q_ss + (int64_t)(G - 1) * p.q_sh + kD)));
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(
      uniform_ptr(reinterpret_cast<const bf16*>(p.dout) + b * p.do_sb + (int64_t)(g * G) * p.do_sh),
      (uint32_t)(2 * ((int64_t)(p.Sq - 1) * p.do_ss + (int64_t)(G - 1) * p.do_sh + kD)));
  // per-row start values of the S and dP accumulators (-lse / scale, -δ)
  const int64_t nrows = (int64_t)p.B * p.Sq * p.Hq;
  const uint32_t rc_bytes = (uint32_t)(4 * ((int64_t)(p.Sq - 1) * p.Hq + G));
  const __amdgpu_buffer_rsrc_t rl = make_rsrc(uniform_ptr(p.rowc + (int64_t)b * p.Sq * p.Hq + g * G), rc_bytes);
  const __amdgpu_buffer_rsrc_t rdl = make_rsrc(uniform_ptr(p.rowc + nrows + (int64_t)b * p.Sq * p.Hq + g * G), rc_bytes);
  const __amdgpu_buffer_rsrc_t rm = make_rsrc(
      uniform_ptr(p.kmap + ((int64_t)b * p.Hkv + g) * p.Sq * p.kmap_w + kb * 4),
      (uint32_t)(4 * ((int64_t)(p.Sq - 1) * p.kmap_w + 4)));

  // Query block qb into one set of buffers: Q / dO rows (32 instructions
  // each, 4 rows per instruction, wave w issues instructions w, w + 4, ...),
  // lse (wave 0), δ (wave 1), each wave its bitmap words.  Rows of queries
  // >= Sq read out of range (zeros); such rows have an all-zero mask, so they
  // contribute nothing.
  // A block load in steps: step k < 8 issues Q and dO instruction 4 k + wave,
  // steps 8 and 9 the lse / δ / mask rows 64 (k - 8) .. +63.  (Spreading the
  // steps over the previous block's MFMA stream measured slower than the
  // burst.)
  constexpr int kLoadSteps = kTB / 64 / 4 + kRowBlock / 64;
  auto load_step = [&](int step, int qb, u32x4* qd, u32x4* dd, float* ls, float* dl, uint32_t (*mk)[kRowBlock]) {
    const int t0 = qb * nq;
    if (step < kTB / 64 / 4) {
      const int ki = 4 * step + wave;
      const int r = 4 * ki + (lane >> 4);
      const int cc = (lane & 15) ^ blk_swz(r);  // slot lane & 15 of row r holds chunk cc
      const int t = t0 + (r >> lg), h = r & (G - 1);
      const bool ok = t < p.Sq;
      const uint32_t oq = ok ? (uint32_t)(2 * (t * p.q_ss + h * p.q_sh) + 16 * cc) : kOOB;
      const uint32_t od = ok ? (uint32_t)(2 * (t * p.do_ss + h * p.do_sh) + 16 * cc) : kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void*)(qd + 64 * ki), 16, oq, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rd, (lds_void*)(dd + 64 * ki), 16, od, 0, 0, 0);
    } else {
      const int k2 = step - kTB / 64 / 4;
      const int r = 64 * k2 + lane;
      const int t = t0 + (r >> lg), h = r & (G - 1);
      const bool ok = t < p.Sq;
      const uint32_t o = ok ? (uint32_t)(4 * (t * p.Hq + h)) : kOOB;
      if (wave == 0)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rl, (lds_void*)(ls + 64 * k2), 4, o, 0, 0, 0);
      else if (wave == 1)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rdl, (lds_void*)(dl + 64 * k2), 4, o, 0, 0, 0);
      const uint32_t om = ok ? (uint32_t)(4 * (t * p.kmap_w + wave)) : kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (lds_void*)(&mk[wave][64 * k2]), 4, om, 0, 0, 0);
    }
  };
  auto load_block = [&](int qb, u32x4* qd, u32x4* dd, float* ls, float* dl, uint32_t (*mk)[kRowBlock]) {
#pragma unroll
    for (int k = 0; k < kLoadSteps; ++k) load_step(k, qb, qd, dd, ls, dl, mk);
  };

  acc_t dkacc[kD / 32], dvacc[kD / 32];
#pragma unroll
  for (int d = 0; d < kD / 32; ++d) {
    dkacc[d] = acc_t{};
    dvacc[d] = acc_t{};
  }

  // Per-lane LDS byte offsets (tile row 0; rows of the tile add immediates).
  // S / dP A operand of step s: row n, chunk 2 s + g2.
  uint32_t aofs[kD / 16];
#pragma unroll
  for (int st = 0; st < kD / 16; ++st) aofs[st] = (uint32_t)(n * kCH + ((2 * st + g2) ^ blk_swz(n))) * 16u;
  // dV / dK A operands (transposing reads): lane group gi of each 16 lanes
  // loads row run + (gi >> 2), dims 32 d + mgrp + 4 (gi & 3) .. +3, i.e. chunk
  // 4 d + cl with cl = mgrp / 8 + (gi & 3) / 2, bytes 8 (gi & 1) on; the runs
  // are rows 4 g2 + rr and 4 g2 + rr + 8 (plus 32 mt + 16 kk, which leave
  // blk_swz unchanged)
  uint32_t vofs[2][kD / 32];
  {
    const int gi = lane & 15, rr = gi >> 2, cc4 = gi & 3, mgrp = (n >> 4) << 4;
    const int cl = mgrp / 8 + cc4 / 2;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int row = 4 * g2 + rr + 8 * hh;
#pragma unroll
      for (int d = 0; d < kD / 32; ++d)
        vofs[hh][d] = (uint32_t)(row * kCH + ((4 * d + cl) ^ blk_swz(row))) * 16u + (uint32_t)(cc4 & 1) * 8u;
    }
  }
  // One query block = 4 tiles of 32 rows.  Tile t: S, dP (16 MFMAs), then P,
  // dS (VALU), then dV, dK (16 MFMAs).  Software pipelined at one wave per
  // SIMD: the P/dS arithmetic of tile t runs between the S/dP MFMAs of tile
  // t + 1 (two sets of S/dP accumulators), so the VALU works while the MFMA
  // pipe is busy.  Fully unrolled: the tile offsets fold into the LDS read
  // immediates.
  constexpr int kTiles = kRowBlock / 32;
  auto compute = [&](const u32x4* qt, const u32x4* dt, const float* ls, const float* dl,
                     const uint32_t (*mk)[kRowBlock]) {
    const uint32_t* msk = mk[wave];
    bf16x8 prev_a = {}, prev_b = {};
    acc_t sacc[2], dpacc[2];
    bf16x8 pb[2][2], db[2][2];  // [tile == last][16-row step]
    // S, dP for rows 32 t .. +31 into (sa, dpa): two interleaved VGPR chains
    // (inline-asm MFMAs, so the operand reads of step st + PDK stay ahead of
    // the MFMAs of step st); mid(st) runs after step st's two MFMAs.
    auto sdp = [&](int t, acc_t& sa, acc_t& dpa, auto&& mid) {
      constexpr int NS = kD / 16, PDK = 4;
      const uint32_t mrow = (uint32_t)(32 * t * kCH) * 16u;
      // start values: S - lse / scale and dP - δ accumulate directly (C-layout
      // element e is row 32 t + 8 (e / 4) + 4 g2 + e % 4)
      acc_t s0, d0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r0 = 32 * t + 8 * q + 4 * g2;
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(ls + r0);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(dl + r0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          s0[4 * q + j] = l4[j];
          d0[4 * q + j] = d4[j];
        }
      }
      bf16x8 qa[PDK], da[PDK];
#pragma unroll
      for (int i = 0; i < PDK; ++i) {
        qa[i] = lds_read_b128(qt, aofs[i] + mrow);
        da[i] = lds_read_b128(dt, aofs[i] + mrow);
      }
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        const bf16x8 aq = qa[st % PDK], ad = da[st % PDK];
        if (st + PDK < NS) {
          qa[st % PDK] = lds_read_b128(qt, aofs[st + PDK] + mrow);
          da[st % PDK] = lds_read_b128(dt, aofs[st + PDK] + mrow);
        }
        if (st == 0) {
          sa = s0;
          dpa = d0;
          M::mma_vn(aq, kB[0], sa, prev_a, prev_b);
          M::mma_vn(ad, vB[0], dpa, aq, kB[0]);
        } else {
          M::mma_v(aq, kB[st], sa, prev_a, prev_b);
          M::mma_v(ad, vB[st], dpa, aq, kB[st]);
        }
        prev_a = ad;
        prev_b = vB[st];
        mid(st);
        // keep mid(st) between these MFMAs and the next step's (the
        // scheduler otherwise sinks all of it below the chain)
        __builtin_amdgcn_sched_barrier(0);
      }
      M::drain_v2(sa, dpa, prev_a, prev_b);
    };
    // P and dS of tile t in 8 pieces; piece st covers C-layout elements
    // e = 4 q + j, q = st / 2, j = 2 (st % 2) + {0, 1}.  The mask words of
    // row group q + 1 are read at piece 2 q, two MFMA steps before their use.
    u32x4 m4[2];
    auto pds_load = [&](int t, int q) {
      m4[q & 1] = *reinterpret_cast<const u32x4*>(msk + 32 * t + 8 * q + 4 * g2);
    };
    auto pds = [&](int t, int st, const acc_t& sa, const acc_t& dpa) {
      const int set = t == kTiles - 1;
      const int q = st >> 1;
      if ((st & 1) == 0 && q + 1 < 4) pds_load(t, q + 1);
      bf16x2 pp, dd;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int j = 2 * (st & 1) + jj, e = 4 * q + j;
        // all ones if the pair (row, key n) is selected, else zero
        const uint32_t keep = (uint32_t)__builtin_amdgcn_sbfe((int)m4[q & 1][j], n, 1);
        // sa = S - lse / scale, dpa = dP - δ
        const float ex = __builtin_amdgcn_exp2f(sa[e] * p.scale_log2);
        const float pr = __uint_as_float(__float_as_uint(ex) & keep);
        const float ds = pr * dpa[e];
        pp[jj] = (bf16)pr;
        dd[jj] = (bf16)ds;
      }
      // materialise the piece here: the empty volatile asm stays between the
      // surrounding MFMA asm statements, and so does the arithmetic feeding it
      asm volatile("" : "+v"(pp), "+v"(dd));
      const int e0 = 4 * q + 2 * (st & 1);
      pb[set][e0 / 8][e0 % 8] = pp[0];
      pb[set][e0 / 8][e0 % 8 + 1] = pp[1];
      db[set][e0 / 8][e0 % 8] = dd[0];
      db[set][e0 / 8][e0 % 8 + 1] = dd[1];
    };
    // dV^T += dO^T P, dK^T += Q^T dS over tile t's rows in two 16-row steps
    // kk; step kk's B operand (lane group g2) holds rows 32 t + 16 kk + 4 g2 +
    // {0..3} and the same + 8, which the A operand gets from two transposing
    // reads of those 4-row runs.  Operand i = 8 kk + 2 d + w (w = 0: dO for
    // dV, 1: Q for dK); the reads of operand i + PD are issued before MFMA i.
    // mid(i) runs after MFMA i.
    auto dvdk = [&](int t, auto&& mid) {
      const int set = t == kTiles - 1;
      const uint32_t mrow = (uint32_t)(32 * t * kCH) * 16u;
      auto load_a = [&](int i) -> bf16x8 {
        const int kk = i / 8, d = (i / 2) % 4, w = i % 2;
        const uint32_t rb = mrow + (uint32_t)(16 * kk * kCH) * 16u;
        const u32x4* src = w ? qt : dt;
        const bf16x4 lo = lds_read_tr16(src, vofs[0][d] + rb);
        const bf16x4 hi = lds_read_tr16(src, vofs[1][d] + rb);
        return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      };
      constexpr int NA = 16, PD = 4;
      bf16x8 abuf[PD];
#pragma unroll
      for (int i = 0; i < PD; ++i) abuf[i] = load_a(i);
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int kk = i / 8, d = (i / 2) % 4, w = i % 2;
        const bf16x8 a = abuf[i % PD];
        if (i + PD < NA) abuf[i % PD] = load_a(i + PD);
        const bf16x8 bop = w ? db[set][kk] : pb[set][kk];
        acc_t& acc = w ? dkacc[d] : dvacc[d];
        if (i % 8 < 2)  // first use of pb[kk] / db[kk], written by VALU
          M::template mma_agpr<true>(a, bop, acc, prev_a, prev_b);
        else
          M::template mma_agpr<false>(a, bop, acc, prev_a, prev_b);
        prev_a = a;
        prev_b = bop;
        mid(i);
      }
    };
    sdp(0, sacc[0], dpacc[0], [](int) {});
#pragma unroll
    for (int mt = 0; mt < kTiles; ++mt) {
      const acc_t& sc = sacc[mt & 1];
      const acc_t& dc = dpacc[mt & 1];
      if (mt + 1 < kTiles) {
        pds_load(mt, 0);
        sdp(mt + 1, sacc[(mt + 1) & 1], dpacc[(mt + 1) & 1], [&](int st) { pds(mt, st, sc, dc); });
      }
      if (mt + 2 == kTiles) {
        // no S/dP chain follows: the last tile's P/dS pieces run between this
        // tile's dV/dK MFMAs instead, into their own P/dS operand set
        const acc_t& sn = sacc[(mt + 1) & 1];
        const acc_t& dn = dpacc[(mt + 1) & 1];
        pds_load(mt + 1, 0);
        dvdk(mt, [&](int i) {
          if (i & 1) {
            pds(mt + 1, i / 2, sn, dn);
            __builtin_amdgcn_sched_barrier(0);
          }
        });
      } else {
        dvdk(mt, [](int) {});
      }
    }
    M::tail(prev_a, prev_b);
  };

  __syncthreads();  // list staged
  load_block(s_list[0], s_q0, s_d0, s_lse0, s_dlt0, s_msk0);
  __syncthreads();
  for (int j = 0; j < nblk; j += 2) {
    if (j + 1 < nblk) load_block(s_list[j + 1], s_q1, s_d1, s_lse1, s_dlt1, s_msk1);
    compute(s_q0, s_d0, s_lse0, s_dlt0, s_msk0);
    __syncthreads();
    if (j + 1 < nblk) {
      if (j + 2 < nblk) load_block(s_list[j + 2], s_q0, s_d0, s_lse0, s_dlt0, s_msk0);
      compute(s_q1, s_d1, s_lse1, s_dlt1, s_msk1);
      __syncthreads();
    }
  }

#pragma unroll
  for (int d = 0; d < kD / 32; ++d) {
    M::drain(dkacc[d]);
    M::drain(dvacc[d]);
  }
  // partial [key][dK 128 | dV 128] of this chunk; C layout: lane (key n,
  // group g2), element e = dim 32 d + 8 (e / 4) + 4 g2 + e % 4
  float* part = p.dkv_part + ((bgk * p.max_chunks + c) * kKeyBlock + wave * 32 + n) * (2 * kD);
#pragma unroll
  for (int d = 0; d < kD / 32; ++d) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int dim = 32 * d + 8 * q + 4 * g2;
      const f32x4 k4 = {dkacc[d][4 * q] * p.scale, dkacc[d][4 * q + 1] * p.scale, dkacc[d][4 * q + 2] * p.scale,
                        dkacc[d][4 * q + 3] * p.scale};
      const f32x4 v4 = {dvacc[d][4 * q], dvacc[d][4 * q + 1], dvacc[d][4 * q + 2], dvacc[d][4 * q + 3]};
      *reinterpret_cast<f32x4*>(part + dim) = k4;
      *reinterpret_cast<f32x4*>(part + kD + dim) = v4;
    }
  }
  if (tid == 0) s_unit[par ^ 1] = claim_i < p.kctr[1] ? p.uorder[claim_i] : -1;
  par ^= 1;
  __syncthreads();  // the next unit's list and blocks overwrite the LDS; its claim is published
  }  // units
}

// ---- 3. chunk partials -> per-key accumulators (chunk order) --------------
__global__ __launch_bounds__(256) void dkv_reduce_kernel(Params p) {
  constexpr int Q4 = 2 * kD / 4;
  const int64_t n4 = (int64_t)p.B * p.Skv * p.Hkv * Q4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
    const int q4 = (int)(i % Q4);
    int64_t r = i / Q4;
    const int g = (int)(r % p.Hkv);
    r /= p.Hkv;
    const int key = (int)(r % p.Skv);
    const int b = (int)(r / p.Skv);
    const int kb = key / kKeyBlock;
    const int64_t bgk = ((int64_t)b * p.Hkv + g) * p.nkb + kb;
    const int* start = p.bstart + bgk * (p.max_chunks + 1);
    const float* src = p.dkv_part + (bgk * p.max_chunks * kKeyBlock + (key % kKeyBlock)) * (2 * kD) + 4 * q4;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int ch = 0; ch < p.max_chunks; ++ch)  // chunks with entries wrote a partial
      if (start[ch + 1] > start[ch]) acc += *reinterpret_cast<const f32x4*>(src + (int64_t)ch * kKeyBlock * (2 * kD));
    const int64_t row = (((int64_t)b * p.Skv + key) * p.Hkv + g) * kD;
    float* dst = (4 * q4 < kD) ? p.dk_acc + row + 4 * q4 : p.dv_acc + row + 4 * q4 - kD;
    *reinterpret_cast<f32x4*>(dst) += acc;
  }
}

inline unsigned grid_stride_blocks(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return (unsigned)(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

bool fits31(int64_t bytes) { return bytes > 0 && bytes < (int64_t)kOOB; }

}  // namespace

bool bwd_csr_supported(const Params& p) {
  if (!bwd_mfma_supported(p)) return false;  // the query-major dQ kernel
  if (p.Dqk != kD || p.Dv != kD) return false;
  if (p.G < 1 || p.G > kRowBlock || (p.G & (p.G - 1)) != 0) return false;  // a query block holds whole queries
  const int nkb = (p.Skv + kKeyBlock - 1) / kKeyBlock;
  const int64_t w = 4 * (int64_t)nkb;
  if (w > kMaxMapWords) return false;
  return fits31(2 * ((int64_t)(p.Sq - 1) * p.q_ss + (int64_t)(p.G - 1) * p.q_sh + kD)) &&
         fits31(2 * ((int64_t)(p.Sq - 1) * p.do_ss + (int64_t)(p.G - 1) * p.do_sh + kD)) &&
         fits31(4 * ((int64_t)(p.Sq - 1) * p.l_ss + (int64_t)(p.G - 1) * p.l_sh + 1)) &&
         fits31(4 * ((int64_t)(p.Sq - 1) * p.Hq + p.G)) && fits31(4 * ((int64_t)(p.Sq - 1) * w + 4));
}

void csr_geometry(Params& p) {
  p.nkb = (p.Skv + kKeyBlock - 1) / kKeyBlock;
  p.kmap_w = 4 * p.nkb;
  p.lg_g = 0;
  while ((1 << p.lg_g) < p.G) ++p.lg_g;  // G is a power of two <= 128
  const int nq = kRowBlock >> p.lg_g;
  p.nqb = (p.Sq + nq - 1) / nq;
  p.max_chunks = (p.nqb + kChunk - 1) / kChunk;
}

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t csr_workspace_bytes(const Params& p) {
  const size_t bg = (size_t)p.B * p.Hkv;
  return al256(bg * p.Sq * p.kmap_w * 4) + al256((size_t)p.B * p.Sq * p.Hkv * p.topk) +
         al256(bg * p.nkb * p.nqb * 4) + al256(bg * p.nkb * (p.max_chunks + 1) * 4) +
         al256(bg * p.nkb * p.max_chunks * kKeyBlock * 2 * kD * 4) + al256((size_t)2 * p.B * p.Sq * p.Hq * 4) + 256 +
         al256(bg * p.nkb * p.max_chunks * 4);
}

void csr_bind_workspace(Params& p, void* ws) {
  const size_t bg = (size_t)p.B * p.Hkv;
  char* c = static_cast<char*>(ws);
  p.kmap = reinterpret_cast<uint32_t*>(c);
  c += al256(bg * p.Sq * p.kmap_w * 4);
  p.dup = reinterpret_cast<uint8_t*>(c);
  c += al256((size_t)p.B * p.Sq * p.Hkv * p.topk);
  p.blist = reinterpret_cast<int*>(c);
  c += al256(bg * p.nkb * p.nqb * 4);
  p.bstart = reinterpret_cast<int*>(c);
  c += al256(bg * p.nkb * (p.max_chunks + 1) * 4);
  p.dkv_part = reinterpret_cast<float*>(c);
  c += al256(bg * p.nkb * p.max_chunks * kKeyBlock * 2 * kD * 4);
  p.rowc = reinterpret_cast<float*>(c);
  c += al256((size_t)2 * p.B * p.Sq * p.Hq * 4);
  p.kctr = reinterpret_cast<int*>(c);
  c += 256;
  p.uorder = reinterpret_cast<int*>(c);
}

hipError_t launch_csr_index(const Params& p, hipStream_t s) {
  const int64_t rows = (int64_t)p.B * p.Sq * p.Hkv;
  if (p.kmap_w <= kWaveMapWords)
    hipLaunchKernelGGL(csr_scatter_wave_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(csr_scatter_kernel, dim3((unsigned)rows), dim3(256), 0, s, p);
  hipLaunchKernelGGL(csr_blocklist_kernel, dim3((unsigned)((int64_t)p.B * p.Hkv * p.nkb)), dim3(256), 0, s, p);
  hipLaunchKernelGGL(unit_order_kernel, dim3(1), dim3(1024), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_csr_dkv(const Params& p, hipStream_t s) {
  // persistent: one workgroup per CU (its LDS use allows one)
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  const int64_t units = (int64_t)p.B * p.Hkv * p.nkb * p.max_chunks;
  const int64_t wgs = units < cus ? units : cus;
  hipLaunchKernelGGL(dkv_keymajor_kernel, dim3((unsigned)wgs), dim3(256), 0, s, p);
  const int64_t n4 = (int64_t)p.B * p.Skv * p.Hkv * (2 * kD / 4);
  hipLaunchKernelGGL(dkv_reduce_kernel, dim3(grid_stride_blocks(n4)), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace sfa

// gfx950 MFMA backward of top-k sparse flash attention for DeepSeek MLA: one
// latent KV head whose 576-dim rows serve as K and whose first 512 dims are
// V, G = 65..128 query heads, bf16 in, fp32 accumulate.  The gradient of the
// shared rows is dK + dV (the reference sums both into one buffer,
// SFA.py:849-853), written to dk.
//
// Reference: `_attn_bwd_dq_dsink` / `_inner_dq` (SFA.py:856-1002, 613-716) and
// `_attn_bwd_dk_dv` / `_inner_dkv` (SFA.py:1005-1145, 719-853).  The shape
// decides the schedule here: per query, Q and dO of the 128 heads (278 KB)
// and the dQ accumulators (295 KB fp32) together exceed what one CU holds, so
// the work is split in two passes over a chunk of queries:
//
//  * dQ pass (mla_bwd_dq_kernel): a workgroup owns (query, 64 heads), 4 waves
//    x 16 heads.  The query's top-k K rows are gathered into LDS 32 at a time
//    (the forward's RowGather and swizzled tile).  Per 32-key tile a wave
//    computes S^T = K Q^T and dP^T = V dO^T (16x16x32, keys as rows; each K
//    operand read serves both; Q^T and dO^T are B operands held in AGPRs),
//    P = 2^(S scale log2e - lse2) and dS = P (dP - delta), then
//    dQ^T += K^T dS^T (K^T by transposing LDS reads; the S^T accumulator
//    layout already is dS^T's B layout) into 144 VGPR accumulators.  P and
//    scale * dS leave as bf16 in the wave's register layout: one 16-byte
//    store per lane and matrix.
//  * dK/dV pass (mla_bwd_dkv_kernel): a workgroup owns one query with all its
//    heads, so the contraction over heads is complete inside it.  Q and dO,
//    staged once per query through LDS and read transposed, sit in registers
//    as operands of dKV^T = Q^T (scale dS) + dO^T P (16x16x32, heads as the
//    contraction; wave w owns dims 144 w .. 144 w + 143).  Per 32-key tile
//    the P / dS tile of the dQ pass is DMA'd into LDS and read back
//    transposed.  The 32 x 576 result of the query is then either
//    - (deterministic, default) rounded to bf16 and stored as one row per
//      (query, distinct key) into the chunk's contribution rows, which
//      mla_bwd_reduce_kernel sums per key in query order into the fp32
//      accumulators (mla_map_kernel first ranks each query's keys; a slot
//      repeating a key of its row adds with fp32 atomics), or
//    - (SFA_DKV_ATOMIC) added to the key rows with fp32 atomics, the
//      reference's scheme (SFA.py:853).
//    An inverted index (key-major pass) does not fit this density: ~2000
//    queries select each key, and each would re-read its 278 KB of Q and dO
//    per key block.
//
// MFMA layouts (16x16x32 bf16, gfx950):
//   A[m][k]: lane l holds m = l % 16, k = 8 (l / 16) + j        (j = 0..7)
//   B[k][n]: lane l holds n = l % 16, k = 8 (l / 16) + j
//   C[m][n]: lane l holds n = l % 16, m = 4 (l / 16) + i        (i = 0..3)

#include "sfa_common.h"
#include "sfa_lds.h"
#include "sfa_mfma.h"

namespace sfa {
namespace {

constexpr int kMT = 32;           // keys per tile
constexpr int kMCH = 72;          // 16-byte chunks of a 576-dim row
constexpr int kMQS = 18;          // 32-dim contraction steps over d_qk = 576
constexpr int kMVS = 16;          // over d_v = 512
constexpr int kMDT = 36;          // 16-dim tiles of d_qk
constexpr int kMHG = 64;          // heads per dQ-pass workgroup
constexpr int kMIdxCap = 2048;    // index slots staged per query
constexpr int kMThreads = 256;
typedef RowGather<kMT, kMCH, 4, true, BufRows> MRG;
static_assert(MRG::PITCH == kMCH, "swizzled tile rows have no pad slot");

// P / dS export of the dQ pass, per (query of the chunk, tile, matrix, head
// group, wave): 64 lanes x 8 bf16.  Lane l = 16 r + h (key run r, head h of
// the wave) holds the values of keys {4 r + i, 16 + 4 r + i}, i = 0..3; it is
// stored at position 16 r + (h ^ 4 r) so the dK/dV pass's transposing reads
// (4 heads x 4 key runs per 16-lane group) are bank-conflict free.
__host__ __device__ constexpr int64_t pd_block_elems() { return 64 * 8; }
__device__ __forceinline__ int pd_pos(int lane) { return (lane & 48) | ((lane & 15) ^ ((lane >> 2) & 12)); }

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// dQ pass
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kMThreads, 1) void mla_bwd_dq_kernel(Params p, int64_t item0, int nitems, bf16* pd) {
  __shared__ int s_idx[kMIdxCap];
  __shared__ u32x4 s_k0[kMT * kMCH];
  __shared__ u32x4 s_k1[kMT * kMCH];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lt = lane & 15, hq = lane >> 4;
  const int nhg = (p.G + kMHG - 1) / kMHG;

  // (item, head group): the head groups of one item go to the same XCD
  // (blockIdx % 8) when the chunk allows it, so its L2 serves the gathered
  // rows to both
  int li, hg;
  {
    const int bi = blockIdx.x;
    if (nitems % 8 == 0) {
      const int x = bi % 8, r = bi / 8;
      hg = r % nhg;
      li = (r / nhg) * 8 + x;
    } else {
      hg = bi % nhg;
      li = bi / nhg;
    }
  }
  const int64_t item = item0 + li;
  const int g = (int)(item % p.Hkv);
  const int t = (int)((item / p.Hkv) % p.Sq);
  const int b = (int)(item / ((int64_t)p.Hkv * p.Sq));
  const int nslots = p.topk;
  const int ntiles = (nslots + kMT - 1) / kMT;

  BufRows ksrc;
  {
    const char* kbase = reinterpret_cast<const char*>(p.k) + 2 * (b * p.k_sb + g * p.k_sh);
    ksrc.rs = make_rsrc(kbase, (uint32_t)(2 * ((int64_t)(p.Skv - 1) * p.k_ss + 576)));
    ksrc.row_bytes = (uint32_t)(2 * p.k_ss);
  }
  const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh;
  const int bound = bound_of(p, b);

  // this lane's head
  const int hl = hg * kMHG + wave * 16 + lt;  // head within the group
  const bool hvalid = hl < p.G;
  const int h = g * p.G + (hvalid ? hl : 0);
  const int64_t row = ((int64_t)b * p.Sq + t) * p.Hq + h;

  // Every load of the prologue goes out before the first wait, oldest first
  // in the order they are needed (loads complete in order, so each wait below
  // covers only what was issued before it): the index row and tile 0's row
  // ids, the row's lse (and LSE gradient), then the Q, dO and O rows of the
  // lane's head (dims 32 s + 8 hq .. +7).  Waiting on each group before
  // issuing the next made the prologue a chain of round trips.
  IdxStage<kMIdxCap, kMThreads> istage;
  istage.load(irow, nslots, tid);
  int raw[MRG::RPW];
#pragma unroll
  for (int r = 0; r < MRG::RPW; ++r) raw[r] = irow[min(wave * MRG::RPW + r, nslots - 1)];
  const float lse = p.lse[b * p.l_sb + t * p.l_ss + (int64_t)h * p.l_sh];
  const float dlse = p.dlse ? p.dlse[b * p.l_sb + t * p.l_ss + (int64_t)h * p.l_sh] : 0.f;
  const bf16* qrow = reinterpret_cast<const bf16*>(p.q) + b * p.q_sb + t * p.q_ss + (int64_t)h * p.q_sh + 8 * hq;
  const bf16* dorow = reinterpret_cast<const bf16*>(p.dout) + b * p.do_sb + t * p.do_ss + (int64_t)h * p.do_sh + 8 * hq;
  const bf16* orow = reinterpret_cast<const bf16*>(p.out) + b * p.o_sb + t * p.o_ss + (int64_t)h * p.o_sh + 8 * hq;
  bf16x8 xq[kMQS], xd[kMVS], xo[kMVS];
#pragma unroll
  for (int s = 0; s < kMQS; ++s) xq[s] = *reinterpret_cast<const bf16x8*>(qrow + 32 * s);
#pragma unroll
  for (int s = 0; s < kMVS; ++s) {
    xd[s] = *reinterpret_cast<const bf16x8*>(dorow + 32 * s);
    xo[s] = *reinterpret_cast<const bf16x8*>(orow + 32 * s);
  }

  // tile 0's gather, from the ids
  {
    MRG rg0;
#pragma unroll
    for (int r = 0; r < MRG::RPW; ++r)
      rg0.set_row(r, (wave * MRG::RPW + r < nslots) ? staged_id<false>(p, b, raw[r], bound) : -1, true, ksrc);
#pragma unroll
    for (int k = 0; k < MRG::NI; ++k) rg0.issue(k, ksrc, s_k0, wave, lane);
  }

  // the row's softmax statistics
  const bool live = hvalid && lse != kNegInf;  // rows with no valid slot contribute nothing
  const float lse2 = live ? lse * kLog2e : 0.f;

  // B operands over the head dims (AGPRs: the VGPR file holds the dQ^T
  // accumulators), and δ = Σ O·dO over the row (SFA.py:590-610's
  // _get_delta_split) from the dO values and the same lane's pieces of the O
  // row: 128 dims per lane, then the 4 lanes of a head (lane groups hq)
  bf16x8 qb[kMQS], dob[kMVS];
#pragma unroll
  for (int s = 0; s < kMQS; ++s) qb[s] = Mfma16A::to_agpr(hvalid ? xq[s] : bf16x8{});  // B operands read from AGPRs
  float delta_h;  // δ of the lane's row, less the LSE gradient
  {
    float acc = 0.f;
#pragma unroll
    for (int s = 0; s < kMVS; ++s)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = fmaf((float)xo[s][j], (float)xd[s][j], acc);
    acc += __shfl_xor(acc, 16, 64);
    acc += __shfl_xor(acc, 32, 64);
    delta_h = acc - dlse;
  }
#pragma unroll
  for (int s = 0; s < kMVS; ++s) dob[s] = Mfma16A::to_agpr(hvalid ? xd[s] : bf16x8{});
  // (δ of every row goes to the workspace for the sink's gradient, reduced
  // after the last chunk)
  if (hvalid && hq == 0) p.delta[row] = delta_h;
  const float delta = live ? delta_h : 0.f;
  istage.store<false>(p, b, bound, nslots, ntiles * kMT, s_idx, tid);

  // Per-lane LDS byte offsets.  S^T / dP^T A operand of M-tile mt, step s:
  // row 16 mt + lt, chunk c = 4 s + hq at slot 8 (c >> 3) + ((c & 7) ^ swz);
  // c & 7 = 4 (s & 1) + hq, so one base per (mt, s & 1) plus (s >> 1) * 128.
  uint32_t ka[2][2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int r = 16 * mt + lt;
      ka[mt][par] = (uint32_t)(r * kMCH + ((4 * par + hq) ^ tile_swz(r))) * 16u;
    }
  // K^T A operand of dQ^T tile m (dims 16 m .. 16 m + 15; keys 4 hq .. +3
  // and 16 + 4 hq .. +3): the 16-lane group of lane group hq reads rows
  // 4 hq + rr (+ 16), dims 16 m + 4 cc .. +3, i.e. chunk 2 m + (cc >> 1) at
  // byte 8 (cc & 1); c & 7 = 2 (m & 3) + (cc >> 1): one base per (m & 3, row
  // run) plus (m >> 2) * 128.  Rows r and r + 16 share their swizzle.
  uint32_t kt_off[4][2];
  {
    const int rr = lt >> 2, cc = lt & 3;
    const int r0 = 4 * hq + rr;
    const int sw = tile_swz(r0);
#pragma unroll
    for (int m4 = 0; m4 < 4; ++m4)
#pragma unroll
      for (int run = 0; run < 2; ++run) {
        const int r = r0 + 16 * run;
        kt_off[m4][run] = (uint32_t)(r * kMCH + ((2 * m4 + (cc >> 1)) ^ sw)) * 16u + (uint32_t)(cc & 1) * 8u;
      }
  }

  f32x4 dq[kMDT];  // dQ^T accumulators (VGPRs)
#pragma unroll
  for (int i = 0; i < kMDT; ++i) dq[i] = f32x4{};

  bf16* const pd_item = pd + (int64_t)li * ntiles * 2 * nhg * 4 * pd_block_elems();
  const int ppos = pd_pos(lane);
  const float scale = p.scale;

  // the gather of the next tile is issued from inside this tile's S^T / dP^T
  // MFMA stream (instruction k after MFMA pair 2 k + 1)
  auto compute = [&](int tile, const u32x4* kt, MRG& rg, u32x4* ndst, uint32_t& vmask_io) {
    const uint32_t vmask = vmask_io;
    // S^T and dP^T, the K operands of step s + PDK read before step s's
    // MFMAs (inline-asm MFMAs with a memory clobber keep that order)
    f32x4 sacc[2], dpacc[2];
    constexpr int PDK = 4;
    auto load_k = [&](int s, int mt) { return lds_read_b128(kt, ka[mt][s & 1] + (uint32_t)(s >> 1) * 128u); };
    bf16x8 kbuf[PDK][2];
#pragma unroll
    for (int i = 0; i < PDK; ++i) {
      kbuf[i][0] = load_k(i, 0);
      kbuf[i][1] = load_k(i, 1);
    }
    bf16x8 prev = {};
#pragma unroll
    for (int s = 0; s < kMQS; ++s) {
      const bf16x8 a0 = kbuf[s % PDK][0], a1 = kbuf[s % PDK][1];
      if (s + PDK < kMQS) {
        kbuf[s % PDK][0] = load_k(s + PDK, 0);
        kbuf[s % PDK][1] = load_k(s + PDK, 1);
      }
      if (s == 0) {
        Mfma16A::mma_v0_ba(a0, qb[0], sacc[0], prev);
        Mfma16A::mma_v0_ba(a1, qb[0], sacc[1], a0);
        Mfma16A::mma_v0_ba(a0, dob[0], dpacc[0], a1);
        Mfma16A::mma_v0_ba(a1, dob[0], dpacc[1], a0);
      } else {
        Mfma16A::mma_v_ba(a0, qb[s], sacc[0], prev);
        Mfma16A::mma_v_ba(a1, qb[s], sacc[1], a0);
        if (s < kMVS) {
          Mfma16A::mma_v_ba(a0, dob[s < kMVS ? s : 0], dpacc[0], a1);
          Mfma16A::mma_v_ba(a1, dob[s < kMVS ? s : 0], dpacc[1], a0);
        }
      }
      prev = a1;
      if ((s & 1) && (s >> 1) < MRG::NI) rg.issue(s >> 1, ksrc, ndst, wave, lane);
    }
    Mfma16A::tail1(prev);
    Mfma16A::drain_v4(sacc[0], sacc[1], dpacc[0], dpacc[1]);
    // row ids of tile + 2 (gathered during the next tile) and the validity
    // of tile + 1's keys
    const bool next2 = tile + 2 < ntiles;
    rg.load_ids(s_idx + (next2 ? tile + 2 : 0) * kMT, next2, wave, ksrc);
    vmask_io = (uint32_t)__ballot(s_idx[(tile + 1 < ntiles ? tile + 1 : 0) * kMT + (lane & 31)] >= 0);

    // P and dS of this lane's head, keys 16 mt + 4 hq + i
    bf16x8 pb, dsb, dse;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = 16 * mt + 4 * hq + i;
        const bool valid = live && ((vmask >> key) & 1u);
        const float pr = valid ? __builtin_amdgcn_exp2f(fmaf(sacc[mt][i], p.scale_log2, -lse2)) : 0.f;
        const float ds = pr * (dpacc[mt][i] - delta);
        pb[4 * mt + i] = (bf16)pr;
        dsb[4 * mt + i] = (bf16)ds;
        dse[4 * mt + i] = (bf16)(ds * scale);
      }
    {
      bf16* blk = pd_item + ((int64_t)((tile * 2 + 0) * nhg + hg) * 4 + wave) * pd_block_elems();
      // (non-temporal: the dK/dV pass reads each block once)
      __builtin_nontemporal_store(pb, reinterpret_cast<bf16x8*>(blk + 8 * ppos));
      __builtin_nontemporal_store(dse, reinterpret_cast<bf16x8*>(blk + (int64_t)nhg * 4 * pd_block_elems() + 8 * ppos));
    }
    // dQ^T += K^T dS^T
    constexpr int PD = 3;
    bf16x8 abuf[PD];
    auto load_kt = [&](int m) -> bf16x8 {
      const uint32_t o = (uint32_t)(m >> 2) * 128u;
      const bf16x4 lo = lds_read_tr16(kt, kt_off[m & 3][0] + o);
      const bf16x4 hi = lds_read_tr16(kt, kt_off[m & 3][1] + o);
      return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
#pragma unroll
    for (int i = 0; i < PD; ++i) abuf[i] = load_kt(i);
    bf16x8 pa = {};
#pragma unroll
    for (int m = 0; m < kMDT; ++m) {
      const bf16x8 a = abuf[m % PD];
      if (m + PD < kMDT) abuf[m % PD] = load_kt(m + PD);
      if (m == 0)
        Mfma16A::mma_vn(a, dsb, dq[m], pa);
      else
        Mfma16A::mma_v(a, dsb, dq[m], pa);
      pa = a;
    }
    Mfma16A::tail(pa, dsb);
  };

  __syncthreads();  // indices staged, first tile in place
  MRG rg;
  rg.load_ids(s_idx + (ntiles > 1 ? kMT : 0), ntiles > 1, wave, ksrc);
  uint32_t vmask = (uint32_t)__ballot(s_idx[lane & 31] >= 0);
  for (int j = 0; j < ntiles; j += 2) {
    compute(j, s_k0, rg, s_k1, vmask);
    __syncthreads();
    if (j + 1 < ntiles) {
      compute(j + 1, s_k1, rg, s_k0, vmask);
      __syncthreads();
    }
  }

  // dQ = scale * dQ^T (lane: head h, dims 16 m + 4 hq .. +3)
#pragma unroll
  for (int m = 0; m < kMDT; ++m) Mfma16A::drain_v1(dq[m]);
  if (!hvalid) return;
  bf16* dqrow = reinterpret_cast<bf16*>(p.dq) + b * p.dq_sb + t * p.dq_ss + (int64_t)h * p.dq_sh + 4 * hq;
#pragma unroll
  for (int m = 0; m < kMDT; ++m) {
    const bf16x4 v = {(bf16)(dq[m][0] * scale), (bf16)(dq[m][1] * scale), (bf16)(dq[m][2] * scale),
                      (bf16)(dq[m][3] * scale)};
    *reinterpret_cast<bf16x4*>(dqrow + 16 * m) = v;
  }
}

// ---------------------------------------------------------------------------
// Index maps of a chunk (deterministic dK/dV): per work item, the membership
// bitmap of its valid keys (bit k of word k >> 5), the number of set bits in
// the words before each word (so a key's rank among the item's distinct keys
// in ascending order is prefix[w] + popc(word & below)), and a flag per slot
// that repeats a key an earlier slot of the row already selected.
// ---------------------------------------------------------------------------
constexpr int kMaxMapW = 2048;  // bitmap words per item: Skv <= 65536

__global__ __launch_bounds__(256) void mla_map_kernel(Params p, int64_t item0, int nitems, int W, uint32_t* kmap,
                                                      uint16_t* prefix, uint8_t* dup) {
  __shared__ uint32_t s_map[4][kMaxMapW];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = blockIdx.x * 4 + wave;
  if (li >= nitems) return;  // the whole wave
  const int64_t item = item0 + li;
  const int g = (int)(item % p.Hkv);
  const int t = (int)((item / p.Hkv) % p.Sq);
  const int b = (int)(item / ((int64_t)p.Hkv * p.Sq));
  const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh;
  const int bound = bound_of(p, b);
  uint32_t* map = s_map[wave];
  for (int w = lane; w < W; w += 64) map[w] = 0u;
  __builtin_amdgcn_wave_barrier();
  uint8_t* drow = dup + (int64_t)li * p.topk;
  // the lane's slots s = 64 j + lane are loaded first, all in flight together
  // (buffer loads over the row's topk ids: slots past it read 0 and are
  // dropped by the slot test below; a load used where it is issued would
  // cost one memory round trip per 64 slots)
  constexpr int J = kMIdxCap / 64;
  const __amdgpu_buffer_rsrc_t rrow = make_rsrc(irow, 4u * (uint32_t)p.topk);
  int ids[J];
#pragma unroll
  for (int j = 0; j < J; ++j) ids[j] = (int)__builtin_amdgcn_raw_buffer_load_b32(rrow, 4u * (uint32_t)(64 * j + lane), 0, 0);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int s = 64 * j + lane;
    const int id = ids[j];
    // exactly one slot of each distinct key finds its bit clear (the first
    // atomicOr to set it); every other slot of that key is a repeat
    uint8_t rep = 0;
    if (s < p.topk && id >= 0 && id < bound) {
      const uint32_t bit = 1u << (id & 31);
      rep = (atomicOr(&map[id >> 5], bit) & bit) ? 1 : 0;
    }
    if (s < p.topk) drow[s] = rep;
  }
  __builtin_amdgcn_wave_barrier();
  // prefix popcounts: lane l sums words [l W/64, (l + 1) W/64), then a wave scan
  const int per = W / 64;  // W is a multiple of 64
  int cnt = 0;
  for (int i = 0; i < per; ++i) cnt += __builtin_popcount(map[lane * per + i]);
  int incl = cnt;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  int run = incl - cnt;
  uint32_t* mrow = kmap + (int64_t)li * W;
  uint16_t* prow = prefix + (int64_t)li * W;
  for (int i = 0; i < per; ++i) {
    const uint32_t x = map[lane * per + i];
    mrow[lane * per + i] = x;
    prow[lane * per + i] = (uint16_t)run;
    run += __builtin_popcount(x);
  }
}

// ---------------------------------------------------------------------------
// dK/dV pass
// ---------------------------------------------------------------------------
constexpr int kQP = 73;   // LDS row pitch (16-byte slots) of the staged Q rows: conflict-free transposing reads
constexpr int kDP = 66;   // of the staged dO rows
constexpr int kCP = 73;   // of the staged contribution rows (576 bf16)
constexpr int kMaxG = 128;
constexpr int kDN = 9;    // 16-dim tiles per wave (dims 144 w .. 144 w + 143)
constexpr int kHS = 4;    // 32-head contraction steps over 128 heads
constexpr int kRankRepeat = -2;  // a slot repeating an earlier slot's key (fp32 atomics)

// Per 32-key tile the product dKV^T = Q^T (scale dS) + dO^T P (dims as MFMA
// rows, keys as columns, heads as the contraction) leaves each lane 4
// consecutive dims of one key.
//  * DET: the bf16 rows go through a double-buffered LDS stage into the
//    chunk's contribution rows, row rank(key) of the item (the key's place
//    among the item's distinct valid keys, ascending); slots that repeat a key
//    add fp32 atomics into the accumulators instead.  mla_bwd_reduce_kernel
//    then sums the rows of each key in item order.
//  * !DET: every slot's fp32 row is added with atomics.
template <bool DET>
__global__ __launch_bounds__(kMThreads, 1) void mla_bwd_dkv_kernel(Params p, int64_t item0, const bf16* pd,
                                                                   bf16* contrib, const uint32_t* kmap,
                                                                   const uint16_t* prefix, const uint8_t* dup,
                                                                   int W) {
  constexpr int kStage = kMaxG * kQP;  // 16-byte slots: Q rows, then dO rows, then P / dS tiles and output rows
  __shared__ u32x4 s_stage[kStage];
  __shared__ int s_idx[kMIdxCap];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lt = lane & 15, hq = lane >> 4;
  const int nhg = (p.G + kMHG - 1) / kMHG;

  const int li = blockIdx.x;
  const int64_t item = item0 + li;
  const int g = (int)(item % p.Hkv);
  const int t = (int)((item / p.Hkv) % p.Sq);
  const int b = (int)(item / ((int64_t)p.Hkv * p.Sq));
  const int nslots = p.topk;
  const int ntiles = (nslots + kMT - 1) / kMT;
  const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh;
  const int bound = bound_of(p, b);
  IdxStage<kMIdxCap, kMThreads> istage;
  istage.load(irow, nslots, tid);

  // ---- Q and dO of the query's heads, as A operands over heads ----------
  // (lane: dim 144 w + 16 n + lt, heads 32 ks + 8 hq .. +7; read from the
  // staged [head][dim] rows with two transposing reads of 4 heads each)
  const bf16* q0 = reinterpret_cast<const bf16*>(p.q) + b * p.q_sb + t * p.q_ss + (int64_t)(g * p.G) * p.q_sh;
  const bf16* d0 = reinterpret_cast<const bf16*>(p.dout) + b * p.do_sb + t * p.do_ss + (int64_t)(g * p.G) * p.do_sh;
  bf16x8 qB[kDN][kHS];
  bf16x8 dB[kDN][kHS];
  const int dim0 = 144 * wave;
  const int ndv = wave < 3 ? kDN : 5;  // dim tiles below 512
  // rows [G][nch 16-byte chunks] (row stride sh elements) into LDS rows of
  // `pitch` slots by DMA (all in flight at once); pad slots and rows >= G
  // read an out-of-range offset and get zeros
  auto stage_rows = [&](const bf16* src, int64_t sh, int nch, int pitch) {
    const uint32_t rb = (uint32_t)(2 * sh);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, (uint32_t)((p.G - 1) * rb + 16u * (uint32_t)nch));
    const int nslot = kMaxG * pitch;  // a multiple of 64 for both pitches
    for (int u0 = wave * 64; u0 < nslot; u0 += kMThreads) {
      const int u = u0 + lane;
      const int hh = u / pitch, c = u - hh * pitch;
      const uint32_t off = (hh < p.G && c < nch) ? (uint32_t)hh * rb + 16u * (uint32_t)c : kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(s_stage + u0), 16, off, 0, 0, 0);
    }
  };
  static_assert((kMaxG * kQP) % 64 == 0 && (kMaxG * kDP) % 64 == 0, "whole DMA instructions");
  auto read_b = [&](int pitch, int n, int ks) -> bf16x8 {
    const int rr = lt >> 2, cc = lt & 3;
    const int hh = 32 * ks + 8 * hq + rr;
    const int d = dim0 + 16 * n + 4 * cc;
    const uint32_t o0 = (uint32_t)(hh * pitch) * 16u + (uint32_t)d * 2u;
    const uint32_t o1 = o0 + (uint32_t)(4 * pitch) * 16u;
    const bf16x4 lo = lds_read_tr16(s_stage, o0);
    const bf16x4 hi = lds_read_tr16(s_stage, o1);
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };
  stage_rows(q0, p.q_sh, kMCH, kQP);
  istage.store<false>(p, b, bound, nslots, ntiles * kMT, s_idx, tid);
  __syncthreads();
#pragma unroll
  for (int n = 0; n < kDN; ++n)
#pragma unroll
    for (int ks = 0; ks < kHS; ++ks) qB[n][ks] = read_b(kQP, n, ks);
  __syncthreads();
  stage_rows(d0, p.do_sh, 64, kDP);
  __syncthreads();
#pragma unroll
  for (int n = 0; n < kDN; ++n)
#pragma unroll
    for (int ks = 0; ks < kHS; ++ks) dB[n][ks] = Mfma16A::to_agpr(n < ndv ? read_b(kDP, n, ks) : bf16x8{});
  __syncthreads();  // the stage area now holds P / dS tiles, output rows and ranks

  // ---- LDS layout of the tile loop (16-byte slots of s_stage) -------------
  // [0, 2048): P / dS tiles 0 and 1; [2048, 2048 + 2 * 32 * kCP): output rows
  // (2 x 32 rows); then the ranks of the item's slots (DET); then P / dS tile 2
  constexpr int kOutBase = 2048;
  constexpr int kRankBase = kOutBase + 2 * kMT * kCP;
  constexpr int kPd2Base = kRankBase + kMIdxCap / 4;
  static_assert(kPd2Base + 1024 <= kStage, "tile-loop LDS fits the stage area");
  int* s_rank = reinterpret_cast<int*>(s_stage + kRankBase);
  if constexpr (DET) {
    // rank of each slot's key among the item's distinct keys (ascending),
    // -1 for an invalid slot, kRankRepeat for a repeat
    const uint32_t* mrow = kmap + (int64_t)li * W;
    const uint16_t* prow = prefix + (int64_t)li * W;
    const uint8_t* drow = dup + (int64_t)li * p.topk;
    constexpr int IPT = kMIdxCap / kMThreads;
    int ids[IPT];
    uint32_t words[IPT];
    int pre[IPT];
    uint8_t rep[IPT];
    // the repeat flags by buffer loads (slots >= nslots read 0): a load under
    // the slot test would be waited for where it is issued, one memory round
    // trip per j
    const __amdgpu_buffer_rsrc_t rdup = make_rsrc(drow, (uint32_t)nslots);
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const int sl = tid + j * kMThreads;
      ids[j] = sl < ntiles * kMT ? s_idx[sl] : -1;
    }
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const int id = ids[j] >= 0 ? ids[j] : 0;
      words[j] = mrow[id >> 5];
      pre[j] = prow[id >> 5];
      rep[j] = __builtin_amdgcn_raw_buffer_load_b8(rdup, (uint32_t)(tid + j * kMThreads), 0, 0);
    }
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const int id = ids[j];
      int r = -1;
      if (id >= 0) r = rep[j] ? kRankRepeat : pre[j] + __builtin_popcount(words[j] & ((1u << (id & 31)) - 1u));
      s_rank[tid + j * kMThreads] = r;
    }
  }

  // ---- P / dS tiles: DMA of the dQ pass's blocks into LDS, two tiles ahead -
  const int tile_slots = 2 * nhg * 4 * 64;  // 16-byte slots per tile (<= 1024)
  auto buf = [&](int k) -> u32x4* { return s_stage + (k == 0 ? 0 : k == 1 ? 1024 : kPd2Base); };
  const char* pd_item = reinterpret_cast<const char*>(pd + (int64_t)li * ntiles * 2 * nhg * 4 * pd_block_elems());
  // The DMA is issued as inline asm (global_load_lds_dwordx4: M0 = the wave's
  // LDS destination, lane l writes 16 bytes at M0 + 16 l), which the compiler
  // does not see: with both tile buffers in one LDS array it cannot tell the
  // current tile's operand reads from the next tile's DMA target, and for the
  // builtin form it waited for the DMA (and the previous tile's row stores)
  // before the first MFMA of every tile.  The loop waits for vmcnt(0) itself
  // before the barrier that publishes a tile.  (nt: each block is read once;
  // with the other single-use streams of the backward marked non-temporal,
  // the whole backward runs about 3 % faster: fewer of the dQ pass's gathered
  // rows are evicted from the caches.)
  auto load_tile = [&](int tile, u32x4* dst) {
    for (int i = wave * 64; i < tile_slots; i += kMThreads) {
      const char* src = pd_item + ((int64_t)tile * tile_slots + i + lane) * 16;
      const uint32_t lds = (uint32_t)(uintptr_t)(lds_void*)(dst + i);
      asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off nt" ::"s"(lds), "v"(src) : "memory", "m0");
    }
  };
  auto dma_done = [&]() { __builtin_amdgcn_s_waitcnt(0x0F70); };  // vmcnt(0)
  // DET: tile j's barrier needs tile j + 1's DMA, issued at the top of tile
  // j - 1.  Issued after it: the 9 row stores of tile j - 1 per wave (buffer
  // stores, unconditional: a row without a rank goes to an out-of-range
  // offset and is dropped), tile j + 2's DMA, and repeat atomics, so at most
  // 9 newer operations may still be outstanding: vmcnt(9).
  auto dma_next_done = [&]() { __builtin_amdgcn_s_waitcnt(0x0F70 | 9); };  // vmcnt(9)
  static_assert(kMT * kMCH == 9 * kMThreads, "9 row stores per thread and tile");


  float* const dkv = p.dk_acc + ((int64_t)b * p.Skv * p.Hkv + g) * 576;
  const int64_t acc_row = (int64_t)p.Hkv * 576;
  bf16* const crow0 = DET ? contrib + (int64_t)li * p.topk * 576 : nullptr;
  const __amdgpu_buffer_rsrc_t rcon = make_rsrc(crow0, DET ? (uint32_t)p.topk * 1152u : 0u);

  // B operands (keys 16 nt + lt, heads 32 ks + 8 hq .. +7) of matrix mat:
  // heads 32 ks + 8 hq + 4 half + rr live in head group (32 ks + 8 hq) / 64,
  // wave ((32 ks + 8 hq) % 64) / 16, head 8 (hq & 1) + 4 half + rr of it
  auto read_pd = [&](const u32x4* tb, int mat, int nt, int ks) -> bf16x8 {
    const int rr = lt >> 2, cc = lt & 3;
    const int hh = 32 * ks + 8 * hq;
    const int blk = (mat * nhg + hh / 64) * 4 + (hh % 64) / 16;
    bf16x4 part[2];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int src_lane = 16 * cc + 8 * (hq & 1) + 4 * half + rr;
      const uint32_t o = (uint32_t)(blk * 64 + pd_pos(src_lane)) * 16u + (uint32_t)nt * 8u;
      part[half] = lds_read_tr16(tb, o);
    }
    return bf16x8{part[0][0], part[0][1], part[0][2], part[0][3], part[1][0], part[1][1], part[1][2], part[1][3]};
  };

  if (ntiles > 0) load_tile(0, buf(0));
  if (ntiles > 1) load_tile(1, buf(1));
  dma_done();
  __syncthreads();
  for (int j = 0; j < ntiles; ++j) {
    const u32x4* tb = buf(j % 3);
    // (tile j - 1's buffer: its reads ended before the last barrier)
    if (j + 2 < ntiles) load_tile(j + 2, buf((j + 2) % 3));
    // (the first contraction step starts each accumulator from 0 inside the
    // MFMA: no VALU write of an accumulator precedes its MFMA)
    // DET: dims as MFMA rows (lane: dims dim0 + 16 n + 4 hq .. +3 of key
    // 16 nt + lt: 8-byte row pieces for the staged rows); atomics: keys as
    // rows (lane: keys 16 nt + 4 hq + i of dim dim0 + 16 n + lt: each atomic
    // instruction covers 4 keys x 16 contiguous dims)
    // The B operands (P and dS of a (key half, head step)) of step st + 1 are
    // read into the other register set after the second MFMA of step st, so
    // their LDS latency runs under step st's MFMAs; the first two MFMAs take
    // the other set (step st - 1's operands) as keep-alive inputs, so at
    // least two MFMAs issue between the last one reading them and the reads
    // that overwrite them (the old per-step s_nop 7 kept that distance).
    // The dO^T operands of dims >= 512 (wave 3) are zeros: their MFMAs run
    // too, which keeps the stream free of branches (wave 3 then does as
    // many MFMAs per step as the others, which the barrier waits for anyway).
    Mfma16A::acc_t acc[kDN][2];
    constexpr int kSteps = 2 * kHS;
    bf16x8 bsv[2], bpv[2];
    bsv[0] = read_pd(tb, 1, 0, 0);
    bpv[0] = read_pd(tb, 0, 0, 0);
    bsv[1] = bf16x8{};
    bpv[1] = bf16x8{};
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      const int nt = st / kHS, ks = st % kHS, cur = st & 1, nxt = cur ^ 1;
      const bf16x8 bs = bsv[cur], bp = bpv[cur];
#pragma unroll
      for (int n = 0; n < kDN; ++n) {
        // (n < 2: keep the other set alive up to here; then read step st + 1 into it)
        const bf16x8& ka = n < 2 ? bpv[nxt] : bp;
        const bf16x8& kb = n < 2 ? bsv[nxt] : bs;
        if constexpr (DET) {
          if (ks == 0)
            Mfma16A::mma0(qB[n][ks], bs, acc[n][nt], ka, kb);
          else
            Mfma16A::mma<false>(qB[n][ks], bs, acc[n][nt], ka, kb);
        } else {
          if (ks == 0)
            Mfma16A::mma0(bs, qB[n][ks], acc[n][nt], ka, kb);
          else
            Mfma16A::mma<false>(bs, qB[n][ks], acc[n][nt], ka, kb);
        }
        if (n == 1 && st + 1 < kSteps) {
          bsv[nxt] = read_pd(tb, 1, (st + 1) / kHS, (st + 1) % kHS);
          bpv[nxt] = read_pd(tb, 0, (st + 1) / kHS, (st + 1) % kHS);
        }
      }
#pragma unroll
      for (int n = 0; n < kDN; ++n) {
        if constexpr (DET)
          Mfma16A::mma_a_agpr(dB[n][ks], bp, acc[n][nt], bs);
        else
          Mfma16A::mma_b_agpr(bp, dB[n][ks], acc[n][nt], bs);
      }
      if (st + 1 == kSteps) Mfma16A::tail(bs, bp);
    }
#pragma unroll
    for (int n = 0; n < kDN; ++n)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) Mfma16A::drain(acc[n][nt]);
    if constexpr (DET) {
      u32x4* orow = s_stage + kOutBase + (j & 1) * kMT * kCP;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int key = 16 * nt + lt;
        const int rk = s_rank[j * kMT + key];
        bf16* r = reinterpret_cast<bf16*>(orow + key * kCP);
#pragma unroll
        for (int n = 0; n < kDN; ++n) {
          const bf16x4 v = {(bf16)acc[n][nt][0], (bf16)acc[n][nt][1], (bf16)acc[n][nt][2], (bf16)acc[n][nt][3]};
          *reinterpret_cast<bf16x4*>(r + dim0 + 16 * n + 4 * hq) = v;
        }
        if (rk == kRankRepeat) {  // rare: a key repeated in the row
          float* dst = dkv + (int64_t)s_idx[j * kMT + key] * acc_row + dim0 + 4 * hq;
#pragma unroll
          for (int n = 0; n < kDN; ++n)
#pragma unroll
            for (int i = 0; i < 4; ++i) atomicAdd(dst + 16 * n + i, acc[n][nt][i]);
        }
      }
      dma_next_done();
      __syncthreads();  // output rows staged; the next tile's P / dS landed
      // rows to their rank in the item's contribution block (72 slots a row;
      // non-temporal: the reduction reads each row once)
#pragma unroll
      for (int k = 0; k < 9; ++k) {
        const int u = tid + k * kMThreads;
        const int key = u / kMCH, c = u - key * kMCH;
        const int rk = s_rank[j * kMT + key];
        const uint32_t off = rk >= 0 ? (uint32_t)rk * 1152u + 16u * (uint32_t)c : kOOB;
        __builtin_amdgcn_raw_buffer_store_b128(orow[key * kCP + c], rcon, off, 0, kCpolNT);
      }
    } else {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int id = s_idx[j * kMT + 16 * nt + 4 * hq + i];
          if (id < 0) continue;
          float* dst = dkv + (int64_t)id * acc_row + dim0 + lt;
#pragma unroll
          for (int n = 0; n < kDN; ++n) atomicAdd(dst + 16 * n, acc[n][nt][i]);
        }
      dma_done();
      __syncthreads();  // the next tile's P / dS landed; this tile's buffer is free
    }
  }
}

// Deterministic reduction of a chunk's contributions.  A group is 16 keys,
// half of one membership-bitmap word (b, g, word): its workgroup stages that
// word and its prefix count for each of the chunk's items of (b, g) in LDS
// (one scattered read per item for all 16 keys, instead of one per item and
// key), then each of its 4 waves sums the rows of 4 of the keys, one key at
// a time, into the fp32 accumulator row (each row owned by one wave; chunks
// run in order) in a fixed order: dims 0..511 in item order, the last 64
// dims in 8 item-ordered partial sums combined by a fixed tree (see flush).
// A chunk holds at most kRedItems items (host-side cap).
// The kernel runs on a second stream beside the next chunk's dQ pass, so it
// is persistent (one workgroup per CU, groups strided over the grid) and
// small: its 95 registers per lane fit beside the dQ pass's 392 (256 + 136
// accumulation registers) in the 512 of a SIMD lane (at most 120 would), and
// its 6.4 KB of LDS beside the dQ pass's 80 KB.  Its VALU work competes with
// the dQ pass's on the shared SIMDs, which is why the tail dims are split
// by rows.
constexpr int kRedItems = 1024;
constexpr int kRedThreads = 256;
constexpr int kRedWaves = kRedThreads / 64;
__global__ __launch_bounds__(kRedThreads) void mla_bwd_reduce_kernel(
    Params p, int64_t item0, int nitems, int b0, int64_t groups, const bf16* contrib, const uint32_t* kmap,
    const uint16_t* prefix, int W) {
  __shared__ uint32_t s_word[kRedItems];
  __shared__ uint16_t s_pre[kRedItems];
  __shared__ int2 s_hits[kRedWaves][8];  // per wave: queued hits (item, rank)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = (p.Skv + 31) / 32;
  for (int64_t gi = blockIdx.x; gi < groups; gi += gridDim.x) {
    const int wsel = (int)((gi >> 1) % nw);
    const int half = (int)(gi & 1);
    const int64_t r = (gi >> 1) / nw;
    const int g = (int)(r % p.Hkv);
    const int b = b0 + (int)(r / p.Hkv);
    // this (b, g)'s items of the chunk: item = (b Sq + t) Hkv + g, stride Hkv
    const int64_t first = ((int64_t)b * p.Sq) * p.Hkv + g;
    const int64_t lo = first < item0 ? item0 + ((g - item0 % p.Hkv) + p.Hkv) % p.Hkv : first;
    const int64_t hi_b = ((int64_t)(b + 1) * p.Sq) * p.Hkv;
    const int64_t hi = hi_b < item0 + nitems ? hi_b : item0 + nitems;
    const int nit = lo < hi ? (int)((hi - lo + p.Hkv - 1) / p.Hkv) : 0;  // <= kRedItems
    const int li0 = (int)(lo - item0);
    __syncthreads();  // the previous group's reads of the staged words are done
    for (int i = tid; i < nit; i += kRedThreads) {
      const int li = li0 + i * p.Hkv;
      s_word[i] = kmap[(int64_t)li * W + wsel];
      s_pre[i] = prefix[(int64_t)li * W + wsel];
    }
    __syncthreads();
    const int bound = bound_of(p, b);
    for (int kk = 0; kk < 16 / kRedWaves; ++kk) {
      const int kbit = 16 * half + kRedWaves * kk + wave;
      const int key = 32 * wsel + kbit;
      if (key >= p.Skv) continue;  // the whole wave
      const uint32_t bit = 1u << kbit;
      float a0[8] = {}, a1[8] = {};
      bool any = false;
      // Items in batches of 64 (one per lane).  A key has only a few hits per
      // batch, so the hits are queued across batches (item and rank, in item
      // order, in the wave's LDS list) and their rows are loaded U at a time,
      // then added in item order: full rounds of loads in flight instead of
      // one short round per batch.
      constexpr int U = 8;
      int2* q = s_hits[wave];
      int nq = 0;  // queued hits (wave-uniform)
      // Row dims 0..511 are lane l's dims 8 l .. 8 l + 7 of every row; the
      // 64 dims past them are split by rows: lane group r = l / 8 loads dims
      // 512 + 8 (l % 8) .. of the flush's row r, so a flush of up to 8 rows
      // takes 9 loads instead of 16, and half the conversions and adds.
      // a1 holds group r's partial sums of the tail dims over the rows it
      // took (in item order); they are combined in a fixed order at the end.
      static_assert(U == 8, "8 lane groups take one row each per flush");
      auto flush = [&](int n) {
        u32x4 v0[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (u < n) {
            // (the queue entry is the wave's: its row address is scalar)
            const int2 h = q[u];
            const int hx = __builtin_amdgcn_readfirstlane(h.x), hy = __builtin_amdgcn_readfirstlane(h.y);
            const u32x4* row = reinterpret_cast<const u32x4*>(contrib + ((int64_t)hx * p.topk + hy) * 576);
            // (non-temporal: each row is read once, beside the dQ pass's gathers)
            v0[u] = __builtin_nontemporal_load(row + lane);
          }
        }
        const int r = lane >> 3;
        u32x4 vt = {0u, 0u, 0u, 0u};
        if (r < n) {
          const int2 h = q[r];
          const u32x4* row = reinterpret_cast<const u32x4*>(contrib + ((int64_t)h.x * p.topk + h.y) * 576);
          vt = __builtin_nontemporal_load(row + 64 + (lane & 7));
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (u >= n) continue;
          const bf16x8 x0 = __builtin_bit_cast(bf16x8, v0[u]);
#pragma unroll
          for (int e = 0; e < 8; ++e) a0[e] += (float)x0[e];
        }
        if (r < n) {
          const bf16x8 xt = __builtin_bit_cast(bf16x8, vt);
#pragma unroll
          for (int e = 0; e < 8; ++e) a1[e] += (float)xt[e];
        }
        any = true;
      };
      for (int ib = 0; ib < nit; ib += 64) {
        const int i = ib + lane;
        const uint32_t word = i < nit ? s_word[i] : 0u;
        const int rank = i < nit ? (int)s_pre[i] + __builtin_popcount(word & (bit - 1u)) : 0;
        uint64_t hits = __ballot((word & bit) != 0u);
        while (hits) {
          // queue up to U - nq of this batch's hits (lane order = item order)
          const int take = min(__popcll(hits), U - nq);
          const uint64_t below = ((1ull << lane) - 1ull);
          const bool mine = ((hits >> lane) & 1ull) && __popcll(hits & below) < take;
          if (mine) q[nq + __popcll(hits & below)] = int2{li0 + i * p.Hkv, rank};
          for (int t = 0; t < take; ++t) hits &= hits - 1;
          nq += take;
          __builtin_amdgcn_wave_barrier();
          if (nq == U) {
            flush(U);
            nq = 0;
            __builtin_amdgcn_wave_barrier();
          }
        }
      }
      if (nq > 0) flush(nq);
      __builtin_amdgcn_wave_barrier();  // the queue's last reads before the next key's writes
      if (!any || key >= bound) continue;
      // the tail dims' total over the 8 groups' partials, a fixed tree
      // ((g0 + g1) + (g2 + g3)) + ((g4 + g5) + (g6 + g7)) (the whole wave is
      // active here)
      float tail[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float t = a1[e];
        t += __shfl_xor(t, 8);
        t += __shfl_xor(t, 16);
        t += __shfl_xor(t, 32);
        tail[e] = t;
      }
      float* dst = p.dk_acc + (((int64_t)b * p.Skv + key) * p.Hkv + g) * 576;
#pragma unroll
      for (int e = 0; e < 8; ++e) dst[8 * lane + e] += a0[e];
      if (lane < 8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) dst[512 + 8 * lane + e] += tail[e];
      }
    }
  }
}

}  // namespace

bool bwd_mla_supported(const Params& p) {
  if (p.Dqk != 576 || p.Dv != 512 || p.G > kMaxG || p.G <= 64 || p.topk > kMIdxCap) return false;
  if (!(p.v == p.k && p.v_sb == p.k_sb && p.v_ss == p.k_ss && p.v_sh == p.k_sh)) return false;
  const int64_t kb = 2 * ((int64_t)(p.Skv - 1) * p.k_ss + p.Dqk);
  return kb < (int64_t)kOOB && fits_u24(2 * p.k_ss);
}

bool bwd_mla_det_supported(const Params& p) { return p.Skv <= kMaxMapW * 32; }

int bwd_mla_max_chunk_items(bool det) { return det ? kRedItems : 1 << 30; }

int bwd_mla_map_words(const Params& p) { return (p.Skv + 2047) / 2048 * 64; }

size_t bwd_mla_pd_bytes_per_item(const Params& p) {
  const int64_t ntiles = (p.topk + kMT - 1) / kMT;
  const int64_t nhg = (p.G + kMHG - 1) / kMHG;
  return (size_t)(ntiles * 2 * nhg * 4 * pd_block_elems() * 2);
}

size_t bwd_mla_set_bytes_per_item(const Params& p) {
  return (size_t)p.topk * 576 * 2 + (size_t)bwd_mla_map_words(p) * 6 + (size_t)p.topk;
}

size_t bwd_mla_bytes_per_item(const Params& p, bool det) {
  return bwd_mla_pd_bytes_per_item(p) + (det ? bwd_mla_set_bytes_per_item(p) : 0);
}

namespace {
// a deterministic chunk's buffer set: contributions, bitmaps, prefixes and
// repeat flags of n items, in that order
struct MlaSet {
  bf16* contrib;
  uint32_t* kmap;
  uint16_t* prefix;
  uint8_t* dup;
};
MlaSet mla_set(const Params& p, int n, void* set) {
  char* c = (char*)set;
  const int W = bwd_mla_map_words(p);
  MlaSet m;
  m.contrib = (bf16*)c;
  c += (size_t)n * p.topk * 576 * 2;
  m.kmap = (uint32_t*)c;
  c += (size_t)n * W * 4;
  m.prefix = (uint16_t*)c;
  c += (size_t)n * W * 2;
  m.dup = (uint8_t*)c;
  return m;
}
}  // namespace

// Work items (b, t, kv-head) [item0, item0 + n) of one chunk.  The index
// maps of a deterministic chunk (into its buffer set), read by its dK/dV
// pass and its reduction.
hipError_t launch_bwd_mla_map(const Params& p, int64_t item0, int n, void* set, hipStream_t s) {
  const MlaSet m = mla_set(p, n, set);
  hipLaunchKernelGGL(mla_map_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, p, item0, n,
                     bwd_mla_map_words(p), m.kmap, m.prefix, m.dup);
  return hipGetLastError();
}

// The dQ pass of a chunk: dQ, δ, and the chunk's P / dS blocks into pd.
hipError_t launch_bwd_mla_dq(const Params& p, int64_t item0, int n, void* pd, hipStream_t s) {
  const int nhg = (p.G + kMHG - 1) / kMHG;
  hipLaunchKernelGGL(mla_bwd_dq_kernel, dim3((unsigned)(n * nhg)), dim3(kMThreads), 0, s, p, item0, n, (bf16*)pd);
  return hipGetLastError();
}

// The dK/dV pass of a chunk from its P / dS blocks: det, the contribution
// rows into the chunk's buffer set (its index maps already built); else
// fp32 atomics into p.dk_acc.  p.dk_acc holds [B, Skv, Hkv, 576] fp32.
hipError_t launch_bwd_mla_dkv(const Params& p, int64_t item0, int n, const void* pd, void* set, bool det,
                              hipStream_t s) {
  const int W = bwd_mla_map_words(p);
  if (det) {
    const MlaSet m = mla_set(p, n, set);
    hipLaunchKernelGGL(mla_bwd_dkv_kernel<true>, dim3((unsigned)n), dim3(kMThreads), 0, s, p, item0,
                       (const bf16*)pd, m.contrib, (const uint32_t*)m.kmap, (const uint16_t*)m.prefix,
                       (const uint8_t*)m.dup, W);
  } else {
    hipLaunchKernelGGL(mla_bwd_dkv_kernel<false>, dim3((unsigned)n), dim3(kMThreads), 0, s, p, item0,
                       (const bf16*)pd, nullptr, nullptr, nullptr, nullptr, W);
  }
  return hipGetLastError();
}

// The ordered reduction of a deterministic chunk's buffer set into
// p.dk_acc; chunks must be reduced in order.  One workgroup per CU.
hipError_t launch_bwd_mla_reduce(const Params& p, int64_t item0, int n, void* set, int cus, hipStream_t s) {
  const MlaSet m = mla_set(p, n, set);
  const int W = bwd_mla_map_words(p);
  const int b0 = (int)(item0 / ((int64_t)p.Hkv * p.Sq));
  const int b1 = (int)((item0 + n - 1) / ((int64_t)p.Hkv * p.Sq));
  const int64_t groups = (int64_t)(b1 - b0 + 1) * p.Hkv * ((p.Skv + 31) / 32) * 2;
  const unsigned grid = (unsigned)(groups < cus ? groups : cus);
  hipLaunchKernelGGL(mla_bwd_reduce_kernel, dim3(grid), dim3(kRedThreads), 0, s, p, item0, n, b0, groups,
                     (const bf16*)m.contrib, (const uint32_t*)m.kmap, (const uint16_t*)m.prefix, W);
  return hipGetLastError();
}

}  // namespace sfa

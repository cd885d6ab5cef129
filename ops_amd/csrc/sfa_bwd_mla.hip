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
//    operand read serves both), P = 2^(S scale log2e - lse2) and
//    dS = P (dP - delta), then dQ^T += K^T dS^T (K^T by transposing LDS
//    reads; the S^T accumulator layout already is dS^T's B layout) into 144
//    AGPRs.  P and scale * dS leave as bf16 in the wave's register layout:
//    one 16-byte store per lane and matrix.
//  * dK/dV pass (mla_bwd_dkv_kernel): a workgroup owns one query with all its
//    heads, so the contraction over heads is complete inside it.  Q and dO sit
//    in registers as the B operands of dKV^T = (scale dS)^T Q + P^T dO
//    (16x16x32, keys as rows, dims as columns, heads as the contraction;
//    wave w owns dims 144 w .. 144 w + 143), staged once per query through LDS
//    and read transposed.  Per 32-key tile the P / dS tile of the dQ pass is
//    DMA'd into LDS and read back transposed as A operands; the 32 x 576 fp32
//    result is added to the key rows with fp32 atomics (the reference's
//    scheme, SFA.py:853: at this density, ~2000 queries per key, an inverted
//    index would re-read each query's 278 KB of Q and dO per key block).
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
  IdxStage<kMIdxCap, kMThreads> istage;
  istage.load(irow, nslots, tid);
  {
    MRG rg0;
    int raw[MRG::RPW];
#pragma unroll
    for (int r = 0; r < MRG::RPW; ++r) raw[r] = irow[min(wave * MRG::RPW + r, nslots - 1)];
#pragma unroll
    for (int r = 0; r < MRG::RPW; ++r)
      rg0.set_row(r, (wave * MRG::RPW + r < nslots) ? staged_id<false>(p, b, raw[r], bound) : -1, true, ksrc);
#pragma unroll
    for (int k = 0; k < MRG::NI; ++k) rg0.issue(k, ksrc, s_k0, wave, lane);
  }

  // this lane's head and its softmax statistics
  const int hl = hg * kMHG + wave * 16 + lt;  // head within the group
  const bool hvalid = hl < p.G;
  const int h = g * p.G + (hvalid ? hl : 0);
  const int64_t row = ((int64_t)b * p.Sq + t) * p.Hq + h;
  const float lse = p.lse[b * p.l_sb + t * p.l_ss + (int64_t)h * p.l_sh];
  const bool live = hvalid && lse != kNegInf;  // rows with no valid slot contribute nothing
  const float lse2 = live ? lse * kLog2e : 0.f;
  const float delta = live ? p.delta[row] : 0.f;

  // B operands over the head dims: lane holds head h, dims 32 s + 8 hq .. +7
  // (AGPRs: the VGPR file holds the dQ^T accumulators)
  bf16x8 qb[kMQS], dob[kMVS];
  {
    const bf16* qrow = reinterpret_cast<const bf16*>(p.q) + b * p.q_sb + t * p.q_ss + (int64_t)h * p.q_sh + 8 * hq;
    const bf16* dorow =
        reinterpret_cast<const bf16*>(p.dout) + b * p.do_sb + t * p.do_ss + (int64_t)h * p.do_sh + 8 * hq;
#pragma unroll
    for (int s = 0; s < kMQS; ++s) {
      bf16x8 x = *reinterpret_cast<const bf16x8*>(qrow + 32 * s);
      qb[s] = Mfma16A::to_agpr(hvalid ? x : bf16x8{});  // B operands read from AGPRs
    }
#pragma unroll
    for (int s = 0; s < kMVS; ++s) {
      bf16x8 x = *reinterpret_cast<const bf16x8*>(dorow + 32 * s);
      dob[s] = Mfma16A::to_agpr(hvalid ? x : bf16x8{});  // B operands read from AGPRs
    }
  }
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
      *reinterpret_cast<bf16x8*>(blk + 8 * ppos) = pb;
      *reinterpret_cast<bf16x8*>(blk + (int64_t)nhg * 4 * pd_block_elems() + 8 * ppos) = dse;
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
// dK/dV pass
// ---------------------------------------------------------------------------
constexpr int kQP = 73;   // LDS row pitch (16-byte slots) of the staged Q rows: conflict-free transposing reads
constexpr int kDP = 66;   // of the staged dO rows
constexpr int kMaxG = 128;
constexpr int kDN = 9;    // 16-dim column tiles per wave (dims 144 w .. 144 w + 143)
constexpr int kHS = 4;    // 32-head contraction steps over 128 heads

__global__ __launch_bounds__(kMThreads, 1) void mla_bwd_dkv_kernel(Params p, int64_t item0, const bf16* pd) {
  constexpr int kStage = kMaxG * kQP;  // 16-byte slots: Q rows, then dO rows, then the P / dS tiles
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

  // ---- Q and dO of the query's heads, as B operands over heads ----------
  // (lane: dim 144 w + 16 n + lt, heads 32 ks + 8 hq .. +7; read from the
  // staged [head][dim] rows with two transposing reads of 4 heads each)
  const bf16* q0 = reinterpret_cast<const bf16*>(p.q) + b * p.q_sb + t * p.q_ss + (int64_t)(g * p.G) * p.q_sh;
  const bf16* d0 = reinterpret_cast<const bf16*>(p.dout) + b * p.do_sb + t * p.do_ss + (int64_t)(g * p.G) * p.do_sh;
  bf16x8 qB[kDN][kHS];
  bf16x8 dB[kDN][kHS];
  const int dim0 = 144 * wave;
  const int ndv = wave < 3 ? kDN : 5;  // column tiles with dims < 512
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
  __syncthreads();  // the stage area now holds P / dS tiles

  // ---- P / dS tiles: DMA of the dQ pass's blocks into LDS -----------------
  // one tile = 2 matrices x nhg head groups x 4 waves blocks of 1 KiB
  const int tile_slots = 2 * nhg * 4 * 64;  // 16-byte slots per tile
  u32x4* buf0 = s_stage;
  u32x4* buf1 = s_stage + 2 * 2 * 4 * 64;
  const char* pd_item = reinterpret_cast<const char*>(pd + (int64_t)li * ntiles * 2 * nhg * 4 * pd_block_elems());
  const __amdgpu_buffer_rsrc_t rpd = make_rsrc(pd_item, (uint32_t)((int64_t)ntiles * tile_slots * 16));
  auto load_tile = [&](int tile, u32x4* dst) {
    for (int i = wave * 64; i < tile_slots; i += kMThreads)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rpd, (lds_void*)(dst + i), 16,
                                               (uint32_t)(tile * tile_slots + i + lane) * 16u, 0, 0, 0);
  };

  float* const dkv = p.dk_acc + ((int64_t)b * p.Skv * p.Hkv + g) * 576;
  const int64_t acc_row = (int64_t)p.Hkv * 576;

  // A operands (keys 16 mt + lt, heads 32 ks + 8 hq .. +7) of matrix mat:
  // heads 32 ks + 8 hq + 4 half + rr live in head group (32 ks + 8 hq) / 64,
  // wave ((32 ks + 8 hq) % 64) / 16, head 8 (hq & 1) + 4 half + rr of it
  auto read_a = [&](const u32x4* tb, int mat, int mt, int ks) -> bf16x8 {
    const int rr = lt >> 2, cc = lt & 3;
    const int hh = 32 * ks + 8 * hq;
    const int blk = (mat * nhg + hh / 64) * 4 + (hh % 64) / 16;
    bf16x4 part[2];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int src_lane = 16 * cc + 8 * (hq & 1) + 4 * half + rr;
      const uint32_t o = (uint32_t)(blk * 64 + pd_pos(src_lane)) * 16u + (uint32_t)mt * 8u;
      part[half] = lds_read_tr16(tb, o);
    }
    return bf16x8{part[0][0], part[0][1], part[0][2], part[0][3], part[1][0], part[1][1], part[1][2], part[1][3]};
  };

  if (ntiles > 0) load_tile(0, buf0);
  __syncthreads();
  for (int j = 0; j < ntiles; ++j) {
    const u32x4* tb = (j & 1) ? buf1 : buf0;
    if (j + 1 < ntiles) load_tile(j + 1, (j & 1) ? buf0 : buf1);
    // (the first contraction step starts each accumulator from 0 inside the
    // MFMA: no VALU write of an accumulator precedes its MFMA)
    Mfma16A::acc_t acc[2][kDN];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int ks = 0; ks < kHS; ++ks) {
        const bf16x8 as = read_a(tb, 1, mt, ks);
        const bf16x8 ap = read_a(tb, 0, mt, ks);
        bf16x8 prev = {};
#pragma unroll
        for (int n = 0; n < kDN; ++n) {
          if (ks == 0)
            Mfma16A::mma0(as, qB[n][ks], acc[mt][n], prev, qB[n > 0 ? n - 1 : 0][ks]);
          else
            Mfma16A::mma<false>(as, qB[n][ks], acc[mt][n], prev, qB[n > 0 ? n - 1 : 0][ks]);
          prev = as;
        }
#pragma unroll
        for (int n = 0; n < kDN; ++n)
          if (n < ndv) Mfma16A::mma_b_agpr(ap, dB[n][ks], acc[mt][n], as);
        Mfma16A::tail(as, ap);
      }
    }
    // the tile's rows: keys 16 mt + 4 hq + i of dims dim0 + 16 n + lt
    int ids[2][4];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) ids[mt][i] = s_idx[j * kMT + 16 * mt + 4 * hq + i];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int n = 0; n < kDN; ++n) Mfma16A::drain(acc[mt][n]);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (ids[mt][i] < 0) continue;
        float* dst = dkv + (int64_t)ids[mt][i] * acc_row + dim0 + lt;
#pragma unroll
        for (int n = 0; n < kDN; ++n) atomicAdd(dst + 16 * n, acc[mt][n][i]);
      }
    __syncthreads();  // the next tile's DMA has landed; this tile's buffer is free
  }
}

}  // namespace

bool bwd_mla_supported(const Params& p) {
  if (p.Dqk != 576 || p.Dv != 512 || p.G > kMaxG || p.G <= 64 || p.topk > kMIdxCap) return false;
  if (!(p.v == p.k && p.v_sb == p.k_sb && p.v_ss == p.k_ss && p.v_sh == p.k_sh)) return false;
  const int64_t kb = 2 * ((int64_t)(p.Skv - 1) * p.k_ss + p.Dqk);
  return kb < (int64_t)kOOB && fits_u24(2 * p.k_ss);
}

size_t bwd_mla_pd_bytes_per_item(const Params& p) {
  const int64_t ntiles = (p.topk + kMT - 1) / kMT;
  const int64_t nhg = (p.G + kMHG - 1) / kMHG;
  return (size_t)(ntiles * 2 * nhg * 4 * pd_block_elems() * 2);
}

// Items (b, t, kv-head) of the chunk [item0, item0 + n): dQ pass, then the
// dK/dV pass over the same items.  p.dk_acc holds [B, Skv, Hkv, 576] fp32.
hipError_t launch_bwd_mla_chunk(const Params& p, int64_t item0, int n, void* pd, hipStream_t s) {
  const int nhg = (p.G + kMHG - 1) / kMHG;
  hipLaunchKernelGGL(mla_bwd_dq_kernel, dim3((unsigned)(n * nhg)), dim3(kMThreads), 0, s, p, item0, n, (bf16*)pd);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(mla_bwd_dkv_kernel, dim3((unsigned)n), dim3(kMThreads), 0, s, p, item0, (const bf16*)pd);
  return hipGetLastError();
}

}  // namespace sfa

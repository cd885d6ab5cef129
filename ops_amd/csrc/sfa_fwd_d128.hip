// gfx950 forward for d_qk = d_v = 128 (the MQA prefill and GQA training
// shapes, and the reference's own single shared kv with G = 32, 64, 128 query
// heads), also instantiated for d = 64 (the reference's signature at that
// width, SFA.py:97, 554: any power-of-two head dim): register gather of whole
// rows.  The text below describes d = 128; at d = 64 a row is 8 lanes of 16
// bytes and a load instruction moves 8 rows.
//
// Reference: `_attn_fwd` / `_inner_fwd` (SFA.py:309-587); the math is the one
// of the MLA kernel in sfa_fwd_mfma.hip (masked base-2 online softmax with a
// lazy rescale, P V, sink, LSE, split-k partials).  The schedule follows from
// the shape: one wave holds up to 16 heads of a work item (G <= 16: all of
// them; larger G is split into head groups of 16, each its own workgroup,
// the groups of one item placed on one XCD so the re-gathered rows come from
// its L2), so a gathered K or V row is used by exactly one wave and its load
// pattern, not reuse, decides the gather rate.
//  * K and V rows of a 32-key tile are loaded one tile ahead into VGPRs as
//    whole 256-byte rows: each load instruction moves 4 rows (16 lanes per
//    row, 16 bytes each).  Loading them straight in the MFMA operand layout
//    (16 rows x 64 bytes per instruction) runs the texture path 3x slower per
//    byte on L2-resident rows, and that path bounds these kernels.
//  * At the start of a tile the K rows go to the wave's LDS tile (row pitch
//    17 slots: the row writes, the b128 operand reads of 16 rows and the
//    transposing reads are all bank-conflict free), are read back as the A
//    operands of S^T = K Q^T (16x16x32 MFMA), and the V rows then overwrite
//    the same tile (a wave's LDS operations complete in order), from where
//    the transposing reads (ds_read_b64_tr_b16) produce the V^T operands of
//    O^T = V^T P^T;
//  * one wave per workgroup, no barrier inside the tile loop, 12.5 KB of LDS
//    (an index window of 1024 slots: longer top-k sets are split) and at most
//    168 VGPRs, so three waves share each SIMD and hide each other's load
//    latency (6 % faster than two).
//  * paged KV (PAGED = true): indices are staged as pool rows (block table)
//    and the rows loaded from 64-bit addresses; padding rows read kZeroRow.

#include "sfa_common.h"
#include "sfa_lds.h"
#include "sfa_mfma.h"

namespace sfa {
namespace {

constexpr float kSlack = 8.0f;  // lazy-rescale slack (base-2 units), as in the MLA kernel
constexpr int kIdxCapD = 1024;  // slots staged in LDS per work item (longer top-k: split-k)
constexpr int kT = 16;          // heads per wave (MFMA N)
constexpr int kMaxGroupD = 256; // query heads per KV head (16 groups of 16)

// Geometry for head dim D = d_qk = d_v (128; 64 for the reference's
// signature at that width): contraction steps of S^T (32 dims), O^T dim
// tiles (16 dims), 16-byte chunks per row, the LDS row pitch (odd:
// conflict-free reads), and the whole-row load pattern: CH lanes per row,
// RPI rows per load instruction, NI instructions per 32-row tile.
template <int D>
struct Dh {
  static_assert(D == 64 || D == 128, "head dims of the register-gather kernels");
  static constexpr int kQSteps = D / 32;
  static constexpr int kOT = D / 16;
  static constexpr int kCH = D / 8;
  static constexpr int kPV = kCH + 1;
  static constexpr int kRPI = 64 / kCH;
  static constexpr int kNI = 32 / kRPI;
};

template <int D, bool PAGED>
__global__ __launch_bounds__(64, 3) void fwd_d128_kernel(Params p) {
  using M = Mfma<16>;
  typedef M::acc_t acc_t;
  typedef Dh<D> DH;
  constexpr int kQSteps = DH::kQSteps, kOT = DH::kOT, kPV = DH::kPV, kNI = DH::kNI;

  __shared__ __align__(16) int s_idx[kIdxCapD];
  __shared__ u32x4 s_v[32 * kPV];  // the K, then the V rows of the current tile

  const int lane = threadIdx.x;
  const int lt = lane & 15;  // head (MFMA column) / key row within a 16-row M-tile
  const int hq = lane >> 4;  // lane group: 8-element slice of the contraction
  const int lc = lane % DH::kCH, lr = lane / DH::kCH;  // row-load chunk and row group

  // ---- work item (same placement as the MLA kernel) ----------------------
  // A sub-item is (split, head group): the sub-items of one item go to the
  // same XCD, so its L2 serves them the item's rows.
  int wi = blockIdx.x;
  const int nhs = (p.G + kT - 1) / kT;  // head groups of 16
  const int nsub = p.num_splits * nhs;
  int sub;
  const int64_t nitems = (int64_t)p.B * p.Sq * p.Hkv;
  if (nsub > 1 && nitems % 8 == 0) {
    const int x = wi % 8, r = wi / 8;
    sub = r % nsub;
    wi = (r / nsub) * 8 + x;
  } else if (nsub == 1 && nitems % 256 == 0) {
    const int x = wi % 8, r = wi / 8;
    sub = 0;
    wi = ((r / 32) * 8 + x) * 32 + r % 32;
  } else {
    sub = wi % nsub;
    wi /= nsub;
  }
  const int split = sub / nhs;
  const int hg0 = (sub % nhs) * kT;  // first head (within the kv group) of this wave
  const int g = wi % p.Hkv;
  wi /= p.Hkv;
  const int t = wi % p.Sq;
  const int b = wi / p.Sq;
  const int slot0 = split * p.split_len;
  int nslots = p.topk - slot0;
  if (nslots > p.split_len) nslots = p.split_len;
  if (nslots < 0) nslots = 0;
  int ntiles = (nslots + 31) / 32;  // (trimmed to the last valid slot once the ids are staged)

  // ---- index row (invalid -> -1): its loads and Q's are in flight together --
  const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh + slot0;
  const int bound = bound_of(p, b);
  IdxStage<kIdxCapD, 64> istage;
  istage.load(irow, nslots, lane);

  // ---- Q^T B operands (16x16x32: lane holds head hg0 + lt, dims 32 s + 8 hq ..) ---
  const int hl = hg0 + lt;
  const bool hvalid = hl < p.G;
  bf16x8 qb[kQSteps];
  {
    const bf16* qrow = reinterpret_cast<const bf16*>(p.q) + b * p.q_sb + t * p.q_ss +
                       (int64_t)(g * p.G + (hvalid ? hl : 0)) * p.q_sh + 8 * hq;
#pragma unroll
    for (int s = 0; s < kQSteps; ++s) {
      bf16x8 x = *reinterpret_cast<const bf16x8*>(qrow + 32 * s);
      if (!hvalid) x = bf16x8{};
      qb[s] = x;
    }
  }

  // contiguous: buffer resources over this (batch, kv head)'s rows; paged:
  // the pools (the batch lives in the block table)
  const char* kbase = reinterpret_cast<const char*>(p.k) + 2 * ((PAGED ? 0 : b * p.k_sb) + g * p.k_sh);
  const uint32_t krow_bytes = (uint32_t)(2 * p.k_ss);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, PAGED ? 0u : (uint32_t)(2 * ((int64_t)(p.Skv - 1) * p.k_ss + D)));
  const char* vbase = reinterpret_cast<const char*>(p.v) + 2 * ((PAGED ? 0 : b * p.v_sb) + g * p.v_sh);
  const uint32_t vrow_bytes = (uint32_t)(2 * p.v_ss);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase, PAGED ? 0u : (uint32_t)(2 * ((int64_t)(p.Skv - 1) * p.v_ss + D)));

  const int used = wave_max_int(istage.template store<PAGED>(p, b, bound, nslots, ntiles * 32, s_idx, lane));
  __syncthreads();  // indices staged (one wave: orders the LDS writes and reads)
  // tiles past the last valid slot (trailing padding) contribute nothing
  ntiles = (used + 31) / 32;

  // Loads of tile j (keys 32 j .. 32 j + 31): instruction i of a lane loads
  // the 16 bytes at chunk lc of tile row i + NI lr, for K into kr[i] and for V
  // into vr[i] (RPI whole rows per instruction; a lane's NI rows are
  // consecutive, so their ids are NI / 4 16-byte LDS reads).  Invalid keys
  // read from an out-of-range offset (paged: the zero row) and get zeros.
  auto load_tile = [&](int j, bf16x8 (&kr)[kNI], bf16x8 (&vr)[kNI]) {
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    int ids[kNI];
#pragma unroll
    for (int q = 0; q < kNI / 4; ++q) {
      const i32x4 x = *reinterpret_cast<const i32x4*>(s_idx + 32 * j + kNI * lr + 4 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e) ids[4 * q + e] = x[e];
    }
    if constexpr (PAGED) {
#pragma unroll
      for (int i = 0; i < kNI; ++i) {
        const char* ka = ids[i] >= 0 ? kbase + pool_row_offset((uint32_t)ids[i], p.page_shift, (uint64_t)(2 * p.k_sb),
                                                                krow_bytes) + 16 * lc
                                     : reinterpret_cast<const char*>(kZeroRow) + 16 * lc;
        kr[i] = *reinterpret_cast<const bf16x8*>(ka);
      }
#pragma unroll
      for (int i = 0; i < kNI; ++i) {
        const char* va = ids[i] >= 0 ? vbase + pool_row_offset((uint32_t)ids[i], p.page_shift, (uint64_t)(2 * p.v_sb),
                                                                vrow_bytes) + 16 * lc
                                     : reinterpret_cast<const char*>(kZeroRow) + 16 * lc;
        vr[i] = *reinterpret_cast<const bf16x8*>(va);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kNI; ++i) {
        const uint32_t ko = ids[i] >= 0 ? __umul24((uint32_t)ids[i], krow_bytes) + 16u * (uint32_t)lc : kOOB;
        kr[i] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, ko, 0, 0));
      }
#pragma unroll
      for (int i = 0; i < kNI; ++i) {
        const uint32_t vo = ids[i] >= 0 ? __umul24((uint32_t)ids[i], vrow_bytes) + 16u * (uint32_t)lc : kOOB;
        vr[i] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rv, vo, 0, 0));
      }
    }
  };

  // ---- accumulators ----------------------------------------------------
  acc_t oacc[kOT];
#pragma unroll
  for (int i = 0; i < kOT; ++i) oacc[i] = acc_t{};
  float m_used = kNegInf;  // running max (base 2) the exponentials are taken against
  float l_part = 0.f;      // this lane's share of the row sum

  // V^T operand reads (the transposing-read layout of 16-row M-tiles): lane
  // group gi = lane % 16 reads 4-row runs at keys 4 hq .. and 16 + 4 hq ..
  // (the P^T B-operand order), 4-dim piece cc of dim tile ot.
  const int gi = lane & 15, rr = gi >> 2, cc = gi & 3;
  const uint32_t vb0 = (uint32_t)((4 * hq + rr) * kPV) * 16u + (uint32_t)(4 * cc) * 2u;
  const uint32_t vb1 = (uint32_t)((16 + 4 * hq + rr) * kPV) * 16u + (uint32_t)(4 * cc) * 2u;

  auto step = [&](int j, bf16x8 (&kr)[kNI], bf16x8 (&vr)[kNI]) {
    // K rows of this tile into the LDS tile (the previous tile's reads of it
    // are done: LDS operations of a wave complete in order), its S^T A
    // operands (row 16 mt + lt, chunk 4 s + hq) back, then the V rows over
    // them, then the loads of the next tile into the freed registers
#pragma unroll
    for (int i = 0; i < kNI; ++i) *reinterpret_cast<bf16x8*>(&s_v[(i + kNI * lr) * kPV + lc]) = kr[i];
    bf16x8 kc[2 * kQSteps];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int s = 0; s < kQSteps; ++s)
        kc[kQSteps * mt + s] = *reinterpret_cast<const bf16x8*>(&s_v[(16 * mt + lt) * kPV + 4 * s + hq]);
#pragma unroll
    for (int i = 0; i < kNI; ++i) *reinterpret_cast<bf16x8*>(&s_v[(i + kNI * lr) * kPV + lc]) = vr[i];
    const uint32_t vmask = (uint32_t)__ballot(s_idx[32 * j + (lane & 31)] >= 0);
    if (j + 1 < ntiles) load_tile(j + 1, kr, vr);

    // S^T = K Q^T: two 16-key M-tiles
    acc_t sacc[2] = {acc_t{}, acc_t{}};
#pragma unroll
    for (int s = 0; s < kQSteps; ++s)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) sacc[mt] = M::mma(kc[kQSteps * mt + s], qb[s], sacc[mt]);

    // softmax over this lane's 8 keys: key(mt, e) = 16 mt + 4 hq + e
    float sv[8];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = 16 * mt + 4 * hq + e;
        sv[4 * mt + e] = (vmask == 0xffffffffu || ((vmask >> key) & 1u)) ? sacc[mt][e] : kNegInf;
      }
    float ex[8];
    {
      const float moff = (m_used == kNegInf) ? 0.f : -m_used;
#pragma unroll
      for (int i = 0; i < 8; ++i) ex[i] = __builtin_amdgcn_exp2f(fmaf(sv[i], p.scale_log2, moff));
    }
    float tmax = sv[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) tmax = fmaxf(tmax, sv[i]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    tmax *= p.scale_log2;
    const float m_new = fmaxf(m_used, tmax);
    if (__any(m_new > m_used + kSlack)) {
      const float alpha = (m_new == kNegInf) ? 1.f : exp2f(m_used - m_new);
      l_part *= alpha;
#pragma unroll
      for (int i = 0; i < kOT; ++i) oacc[i] *= alpha;
      m_used = m_new;
      const float moff = (m_used == kNegInf) ? 0.f : -m_used;
#pragma unroll
      for (int i = 0; i < 8; ++i) ex[i] = __builtin_amdgcn_exp2f(fmaf(sv[i], p.scale_log2, moff));
    }
    bf16x8 pb;
#pragma unroll
    for (int i = 0; i < 8; ++i) pb[i] = (bf16)ex[i];
    l_part += ((ex[0] + ex[1]) + (ex[2] + ex[3])) + ((ex[4] + ex[5]) + (ex[6] + ex[7]));

    // O^T += V^T P^T (one 32-key contraction step per dim tile)
#pragma unroll
    for (int ot = 0; ot < kOT; ++ot) {
      const bf16x4 lo = lds_read_tr16(s_v, vb0 + (uint32_t)(ot * kT) * 2u);
      const bf16x4 hi = lds_read_tr16(s_v, vb1 + (uint32_t)(ot * kT) * 2u);
      const bf16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      oacc[ot] = M::mma(a, pb, oacc[ot]);
    }
  };

  {
    bf16x8 kr[kNI], vr[kNI];
    if (ntiles > 0) load_tile(0, kr, vr);
    for (int j = 0; j < ntiles; ++j) step(j, kr, vr);
  }

  // ---- finish: row sums over the lane groups sharing a head ---------------
  float l_sum = l_part;
  l_sum += __shfl_xor(l_sum, 16, 64);
  l_sum += __shfl_xor(l_sum, 32, 64);
  const float m_fin = m_used;

  if (!hvalid) return;
  const int h = g * p.G + hl;
  const int64_t row = ((int64_t)b * p.Sq + t) * p.Hq + h;
  // Split partials: normalised O of this split in bf16 plus its base-2 LSE
  // (no sink: the merge adds it once).  Final output: the sink joins the
  // denominator (SFA.py:469-478).
  const bool partial = p.num_splits > 1;
  const int64_t nrows = (int64_t)p.B * p.Sq * p.Hq;
  float scale_o;
  bf16* orow;
  if (partial) {
    scale_o = l_sum > 0.f ? 1.f / l_sum : 0.f;
    if (hq == 0) p.part_lse[split * nrows + row] = l_sum > 0.f ? m_fin + log2f(l_sum) : kNegInf;
    orow = p.part_o + (split * nrows + row) * D;
  } else {
    const float sink2 = p.sink ? p.sink[h] * kLog2e : kNegInf;
    const float mm = fmaxf(m_fin, sink2);
    const float fo = (m_fin == kNegInf) ? 0.f : exp2f(m_fin - mm);
    float lt_ = l_sum * fo;
    if (p.sink && mm != kNegInf) lt_ += exp2f(sink2 - mm);
    scale_o = lt_ > 0.f ? fo / lt_ : 0.f;
    if (hq == 0) p.lse[b * p.l_sb + t * p.l_ss + (int64_t)h * p.l_sh] = lt_ > 0.f ? (mm + log2f(lt_)) * kLn2 : kNegInf;
    orow = reinterpret_cast<bf16*>(p.out) + b * p.o_sb + t * p.o_ss + (int64_t)h * p.o_sh;
  }
  // C layout: lane holds head lt, dims 16 ot + 4 hq + e
#pragma unroll
  for (int ot = 0; ot < kOT; ++ot) {
    const bf16x4 v4 = {(bf16)(oacc[ot][0] * scale_o), (bf16)(oacc[ot][1] * scale_o), (bf16)(oacc[ot][2] * scale_o),
                       (bf16)(oacc[ot][3] * scale_o)};
    *reinterpret_cast<bf16x4*>(orow + 16 * ot + 4 * hq) = v4;
  }
}

// ---- head groups sharing each gathered tile: fwd_d128g_kernel -------------
// 16 < G <= 128 query heads on one kv head, contiguous rows (the reference's
// own shape class: one shared kv row for 32..128 query heads, SFA.py:35-48,
// 88, 104).  A workgroup of NW waves owns a work item, wave w its heads
// 16 w .. 16 w + 15 (NW = G / 16 rounded up to a power of two).  The waves
// gather each 32-key tile together, wave w its rows w R .. w R + R - 1
// (R = 32 / NW), as whole rows one tile ahead into VGPRs (the row-load
// pattern of fwd_d128_kernel), and write them into a double-buffered LDS tile
// from which all NW waves read their operands: a gathered row serves G heads
// instead of 16.  With VK (the v rows are the k rows, as with the reference's
// single kv) one gather serves both products.  One LDS-only barrier per tile;
// the math per wave is fwd_d128_kernel's.
constexpr int kIdxCapG = 2048;  // slots staged per work item (longer top-k: split-k)
constexpr int kMaxGroupG = 128;

template <int D, int NW, bool VK>
__global__ __launch_bounds__(64 * NW, 4) void fwd_d128g_kernel(Params p) {
  using M = Mfma<16>;
  typedef M::acc_t acc_t;
  typedef Dh<D> DH;
  constexpr int kQSteps = DH::kQSteps, kOT = DH::kOT, kPV = DH::kPV;
  constexpr int R = 32 / NW;         // tile rows each wave gathers
  constexpr int RI = R / DH::kRPI;   // its load instructions per matrix (RPI whole rows each)
  constexpr int THR = 64 * NW;
  constexpr int TS = 32 * kPV;  // 16-byte slots of one tile (pitch kPV)
  static_assert(R % DH::kRPI == 0 && NW * R == 32, "whole-row load instructions");

  __shared__ __align__(16) int s_idx[kIdxCapG];
  __shared__ u32x4 s_k[2][TS];
  __shared__ u32x4 s_v[2][VK ? 1 : TS];
  __shared__ int s_used[NW];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lt = lane & 15;  // head (MFMA column) / key row within a 16-row M-tile
  const int hq = lane >> 4;  // lane group
  const int lc = lane % DH::kCH, lr = lane / DH::kCH;  // row-load chunk and row group

  // ---- work item (placement of fwd_d128_kernel) ---------------------------
  int wi = blockIdx.x;
  int split;
  const int64_t nitems = (int64_t)p.B * p.Sq * p.Hkv;
  if (p.num_splits > 1 && nitems % 8 == 0) {
    const int x = wi % 8, r = wi / 8;
    split = r % p.num_splits;
    wi = (r / p.num_splits) * 8 + x;
  } else if (p.num_splits == 1 && nitems % 256 == 0) {
    const int x = wi % 8, r = wi / 8;
    split = 0;
    wi = ((r / 32) * 8 + x) * 32 + r % 32;
  } else {
    split = wi % p.num_splits;
    wi /= p.num_splits;
  }
  const int g = wi % p.Hkv;
  wi /= p.Hkv;
  const int t = wi % p.Sq;
  const int b = wi / p.Sq;
  const int slot0 = split * p.split_len;
  int nslots = p.topk - slot0;
  if (nslots > p.split_len) nslots = p.split_len;
  if (nslots < 0) nslots = 0;
  int ntiles = (nslots + 31) / 32;

  const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh + slot0;
  const int bound = bound_of(p, b);
  IdxStage<kIdxCapG, THR> istage;
  istage.load(irow, nslots, tid);

  // Q^T B operands of this wave's heads (16x16x32: lane holds head hl, dims 32 s + 8 hq ..)
  const int hl = 16 * wave + lt;
  const bool hvalid = hl < p.G;
  bf16x8 qb[kQSteps];
  {
    const bf16* qrow = reinterpret_cast<const bf16*>(p.q) + b * p.q_sb + t * p.q_ss +
                       (int64_t)(g * p.G + (hvalid ? hl : 0)) * p.q_sh + 8 * hq;
#pragma unroll
    for (int s = 0; s < kQSteps; ++s) {
      bf16x8 x = *reinterpret_cast<const bf16x8*>(qrow + 32 * s);
      if (!hvalid) x = bf16x8{};
      qb[s] = x;
    }
  }
  const char* kbase = reinterpret_cast<const char*>(p.k) + 2 * (b * p.k_sb + g * p.k_sh);
  const uint32_t krow_bytes = (uint32_t)(2 * p.k_ss);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, (uint32_t)(2 * ((int64_t)(p.Skv - 1) * p.k_ss + D)));
  const char* vbase = reinterpret_cast<const char*>(p.v) + 2 * (b * p.v_sb + g * p.v_sh);
  const uint32_t vrow_bytes = (uint32_t)(2 * p.v_ss);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase, (uint32_t)(2 * ((int64_t)(p.Skv - 1) * p.v_ss + D)));

  {
    const int used = wave_max_int(istage.template store<false>(p, b, bound, nslots, ntiles * 32, s_idx, tid));
    if (lane == 0) s_used[wave] = used;
  }
  __syncthreads();  // indices staged
  {
    int u = s_used[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) u = max(u, s_used[w]);
    ntiles = (u + 31) / 32;  // tiles past the last valid slot contribute nothing
  }

  // Rows of tile j this lane loads: instruction i, chunk lc of tile row
  // wave R + RI lr + i (a lane's RI rows are consecutive).  Invalid keys read
  // from an out-of-range offset and get zeros.
  const int row0 = wave * R + RI * lr;
  auto load_rows = [&](int j, bf16x8 (&kr)[RI], bf16x8 (&vr)[RI]) {
#pragma unroll
    for (int i = 0; i < RI; ++i) {
      const int id = s_idx[32 * j + row0 + i];
      const uint32_t ko = id >= 0 ? __umul24((uint32_t)id, krow_bytes) + 16u * (uint32_t)lc : kOOB;
      kr[i] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, ko, 0, 0));
      if constexpr (!VK) {
        const uint32_t vo = id >= 0 ? __umul24((uint32_t)id, vrow_bytes) + 16u * (uint32_t)lc : kOOB;
        vr[i] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rv, vo, 0, 0));
      }
    }
  };
  auto write_rows = [&](int buf, const bf16x8 (&kr)[RI], const bf16x8 (&vr)[RI]) {
#pragma unroll
    for (int i = 0; i < RI; ++i) {
      *reinterpret_cast<bf16x8*>(&s_k[buf][(row0 + i) * kPV + lc]) = kr[i];
      if constexpr (!VK) *reinterpret_cast<bf16x8*>(&s_v[buf][(row0 + i) * kPV + lc]) = vr[i];
    }
  };
  // (an LDS-only barrier: the next tile's row loads stay in flight across it)
  auto lds_barrier = []() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  acc_t oacc[kOT];
#pragma unroll
  for (int i = 0; i < kOT; ++i) oacc[i] = acc_t{};
  float m_used = kNegInf;  // running max (base 2) the exponentials are taken against
  float l_part = 0.f;      // this lane's share of the row sum
  const int gi = lane & 15, rr = gi >> 2, cc = gi & 3;
  const uint32_t vb0 = (uint32_t)((4 * hq + rr) * kPV) * 16u + (uint32_t)(4 * cc) * 2u;
  const uint32_t vb1 = (uint32_t)((16 + 4 * hq + rr) * kPV) * 16u + (uint32_t)(4 * cc) * 2u;

  bf16x8 kr[RI], vr[RI];
  if (ntiles > 0) {
    load_rows(0, kr, vr);
    write_rows(0, kr, vr);
  }
  if (ntiles > 1) load_rows(1, kr, vr);
  lds_barrier();
  for (int j = 0; j < ntiles; ++j) {
    const int cur = j & 1;
    const u32x4* kt = s_k[cur];
    const u32x4* vt = VK ? s_k[cur] : s_v[cur];
    const uint32_t vmask = (uint32_t)__ballot(s_idx[32 * j + (lane & 31)] >= 0);
    // S^T = K Q^T: two 16-key M-tiles, A operands row 16 mt + lt, chunk 4 s + hq
    bf16x8 kc[2 * kQSteps];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int s = 0; s < kQSteps; ++s)
        kc[kQSteps * mt + s] = *reinterpret_cast<const bf16x8*>(&kt[(16 * mt + lt) * kPV + 4 * s + hq]);
    acc_t sacc[2] = {acc_t{}, acc_t{}};
#pragma unroll
    for (int s = 0; s < kQSteps; ++s)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) sacc[mt] = M::mma(kc[kQSteps * mt + s], qb[s], sacc[mt]);

    // softmax over this lane's 8 keys: key(mt, e) = 16 mt + 4 hq + e
    float sv[8];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = 16 * mt + 4 * hq + e;
        sv[4 * mt + e] = (vmask == 0xffffffffu || ((vmask >> key) & 1u)) ? sacc[mt][e] : kNegInf;
      }
    float ex[8];
    {
      const float moff = (m_used == kNegInf) ? 0.f : -m_used;
#pragma unroll
      for (int i = 0; i < 8; ++i) ex[i] = __builtin_amdgcn_exp2f(fmaf(sv[i], p.scale_log2, moff));
    }
    float tmax = sv[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) tmax = fmaxf(tmax, sv[i]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    tmax *= p.scale_log2;
    const float m_new = fmaxf(m_used, tmax);
    if (__any(m_new > m_used + kSlack)) {
      const float alpha = (m_new == kNegInf) ? 1.f : exp2f(m_used - m_new);
      l_part *= alpha;
#pragma unroll
      for (int i = 0; i < kOT; ++i) oacc[i] *= alpha;
      m_used = m_new;
      const float moff = (m_used == kNegInf) ? 0.f : -m_used;
#pragma unroll
      for (int i = 0; i < 8; ++i) ex[i] = __builtin_amdgcn_exp2f(fmaf(sv[i], p.scale_log2, moff));
    }
    bf16x8 pb;
#pragma unroll
    for (int i = 0; i < 8; ++i) pb[i] = (bf16)ex[i];
    l_part += ((ex[0] + ex[1]) + (ex[2] + ex[3])) + ((ex[4] + ex[5]) + (ex[6] + ex[7]));

    // O^T += V^T P^T (one 32-key contraction step per dim tile)
#pragma unroll
    for (int ot = 0; ot < kOT; ++ot) {
      const bf16x4 lo = lds_read_tr16(vt, vb0 + (uint32_t)(ot * kT) * 2u);
      const bf16x4 hi = lds_read_tr16(vt, vb1 + (uint32_t)(ot * kT) * 2u);
      const bf16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      oacc[ot] = M::mma(a, pb, oacc[ot]);
    }
    // tile j + 1's rows into the other buffer (every wave finished reading
    // it, tile j - 1, before the last barrier), then tile j + 2's loads
    if (j + 1 < ntiles) {
      write_rows(cur ^ 1, kr, vr);
      if (j + 2 < ntiles) load_rows(j + 2, kr, vr);
    }
    lds_barrier();
  }

  // ---- finish (as fwd_d128_kernel) ----------------------------------------
  float l_sum = l_part;
  l_sum += __shfl_xor(l_sum, 16, 64);
  l_sum += __shfl_xor(l_sum, 32, 64);
  const float m_fin = m_used;
  if (!hvalid) return;
  const int h = g * p.G + hl;
  const int64_t row = ((int64_t)b * p.Sq + t) * p.Hq + h;
  const bool partial = p.num_splits > 1;
  const int64_t nrows = (int64_t)p.B * p.Sq * p.Hq;
  float scale_o;
  bf16* orow;
  if (partial) {
    scale_o = l_sum > 0.f ? 1.f / l_sum : 0.f;
    if (hq == 0) p.part_lse[split * nrows + row] = l_sum > 0.f ? m_fin + log2f(l_sum) : kNegInf;
    orow = p.part_o + (split * nrows + row) * D;
  } else {
    const float sink2 = p.sink ? p.sink[h] * kLog2e : kNegInf;
    const float mm = fmaxf(m_fin, sink2);
    const float fo = (m_fin == kNegInf) ? 0.f : exp2f(m_fin - mm);
    float lt_ = l_sum * fo;
    if (p.sink && mm != kNegInf) lt_ += exp2f(sink2 - mm);
    scale_o = lt_ > 0.f ? fo / lt_ : 0.f;
    if (hq == 0) p.lse[b * p.l_sb + t * p.l_ss + (int64_t)h * p.l_sh] = lt_ > 0.f ? (mm + log2f(lt_)) * kLn2 : kNegInf;
    orow = reinterpret_cast<bf16*>(p.out) + b * p.o_sb + t * p.o_ss + (int64_t)h * p.o_sh;
  }
#pragma unroll
  for (int ot = 0; ot < kOT; ++ot) {
    const bf16x4 v4 = {(bf16)(oacc[ot][0] * scale_o), (bf16)(oacc[ot][1] * scale_o), (bf16)(oacc[ot][2] * scale_o),
                       (bf16)(oacc[ot][3] * scale_o)};
    *reinterpret_cast<bf16x4*>(orow + 16 * ot + 4 * hq) = v4;
  }
}

// waves per workgroup of fwd_d128g_kernel for G: G / 16 rounded up to a power of two
int d128g_waves(int G) { return G <= 32 ? 2 : G <= 64 ? 4 : 8; }

}  // namespace

bool fwd_d128_supported(const Params& p) {
  if (!(p.Dqk == p.Dv && (p.Dqk == 128 || p.Dqk == 64))) return false;
  const int64_t kb = 2 * ((int64_t)(p.Skv - 1) * p.k_ss + p.Dqk);
  const int64_t vb = 2 * ((int64_t)(p.Skv - 1) * p.v_ss + p.Dv);
  // contiguous rows use 32-bit buffer offsets, paged pools 64-bit addresses
  const bool addressable = p.block_table != nullptr || (kb < (int64_t)kOOB && vb < (int64_t)kOOB &&
                                                        fits_u24(2 * p.k_ss) && fits_u24(2 * p.v_ss));
  return p.G <= kMaxGroupD && p.G > 0 && addressable;
}

int fwd_d128_head_groups(const Params& p) { return fwd_d128g_supported(p) ? 1 : (p.G + kT - 1) / kT; }

// The shared-tile kernel: contiguous rows, 16 < G <= 128 (d = 64: G <= 64,
// whose waves each gather whole load instructions of 8 rows).
bool fwd_d128g_supported(const Params& p) {
  return fwd_d128_supported(p) && p.block_table == nullptr && p.G > kT && p.G <= kMaxGroupG &&
         d128g_waves(p.G) * (p.Dqk == 64 ? Dh<64>::kRPI : Dh<128>::kRPI) <= 32;
}

int fwd_d128_idx_cap(const Params& p) { return fwd_d128g_supported(p) ? kIdxCapG : kIdxCapD; }

namespace {

template <int D>
hipError_t launch_fwd_dh(const Params& p, hipStream_t s) {
  if (fwd_d128g_supported(p)) {
    const int64_t n = (int64_t)p.B * p.Sq * p.Hkv * p.num_splits;
    const bool vk = p.v == p.k && p.v_sb == p.k_sb && p.v_ss == p.k_ss && p.v_sh == p.k_sh;
    const int nw = d128g_waves(p.G);
#define SFA_D128G(NW)                                                                                   \
  if (nw == NW) {                                                                                       \
    if (vk)                                                                                             \
      hipLaunchKernelGGL((fwd_d128g_kernel<D, NW, true>), dim3((unsigned)n), dim3(64 * NW), 0, s, p);   \
    else                                                                                                \
      hipLaunchKernelGGL((fwd_d128g_kernel<D, NW, false>), dim3((unsigned)n), dim3(64 * NW), 0, s, p);  \
    return hipGetLastError();                                                                           \
  }
    SFA_D128G(2)
    SFA_D128G(4)
    if constexpr (32 / 8 % Dh<D>::kRPI == 0) {
      SFA_D128G(8)
    }
#undef SFA_D128G
    return hipErrorInvalidValue;
  }
  const int64_t n = (int64_t)p.B * p.Sq * p.Hkv * p.num_splits * fwd_d128_head_groups(p);
  if (p.block_table)
    hipLaunchKernelGGL((fwd_d128_kernel<D, true>), dim3((unsigned)n), dim3(64), 0, s, p);
  else
    hipLaunchKernelGGL((fwd_d128_kernel<D, false>), dim3((unsigned)n), dim3(64), 0, s, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fwd_d128(const Params& p, hipStream_t s) {
  if (p.Dqk == 64) return launch_fwd_dh<64>(p, s);
  return launch_fwd_dh<128>(p, s);
}

}  // namespace sfa

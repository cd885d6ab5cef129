// gfx950 dQ (and dsink) kernel of the deterministic backward for d_qk = d_v =
// 128: register-direct gather, 16 query heads per wave (G > 16 is split into
// head groups of 16, each its own workgroup).
//
// Reference: `_attn_bwd_dq_dsink` / `_inner_dq` (SFA.py:856-1002, 613-716).
// With the deterministic dK/dV scheme (sfa_bwd_csr.hip) the query-major pass
// only produces dQ; the dK/dV rows of index slots that repeat an earlier
// slot's key (flagged in p.dup; absent from ordinary index sets) are added
// by bwd_dup_kernel with fp32 atomics, as in the atomic scheme, outside this
// kernel so their registers do not cost it its second wave per SIMD.  As in the d = 128 forward (sfa_fwd_d128.hip), one wave holds all
// G heads of a work item, so a gathered row is used by exactly one wave and
// the load pattern decides the gather rate:
//  * K and V rows of a 32-key tile are loaded one tile ahead into VGPRs as
//    whole 256-byte rows (4 rows per load instruction; the MFMA operand
//    layout, 16 rows x 64 bytes per instruction, runs the texture path 3x
//    slower per byte on L2-resident rows);
//  * at the start of a tile they go to the wave's two LDS tiles (row pitch
//    17 slots: row writes, b128 operand reads and transposing reads are all
//    bank-conflict free), from which the A operands of S^T = K Q^T and
//    dP^T = V dO^T (16x16x32 MFMA) are read back, and later the transposing
//    reads of the K^T operands of dQ^T += K^T dS^T (the S^T accumulator
//    layout is already dS^T's B-operand layout);
//  * one wave per workgroup and no barrier inside the tile loop.
// Per pair: P = 2^(S·scale·log2e − lse2) (masked), dS = P (dP − δ).

#include "sfa_common.h"
#include "sfa_lds.h"

namespace sfa {
namespace {

constexpr int kIdxCapQ = 2048;  // top-k slots a work item may have
constexpr int kIdxWin = 512;    // slots staged in LDS at a time (a window of the index row)
constexpr int kQS = 4;          // 128 / 32 contraction steps over the head dim
constexpr int kDT = 8;          // 128 / 16 dim tiles
constexpr int kPK = 17;         // K staging row pitch in 16-byte slots (odd: conflict-free reads)
constexpr int kMaxGroupQ = 256; // query heads per KV head (16 groups of 16)
__device__ __forceinline__ f32x4 mma16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(64, 2) void bwd_dq_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) int s_idx[kIdxWin];
  __shared__ u32x4 s_k[32 * kPK];
  __shared__ u32x4 s_v[32 * kPK];

  const int lane = threadIdx.x;
  const int lt = lane & 15;  // head column / key row within a 16-row M-tile
  const int hq = lane >> 4;  // lane group

  // work item and head group; the head groups of an item go to one XCD (its
  // L2 then serves the re-gathered rows)
  int wi = blockIdx.x;
  const int nhs = (p.G + 15) >> 4;
  int hs;
  const int64_t nitems = (int64_t)p.B * p.Sq * p.Hkv;
  if (nhs > 1 && nitems % 8 == 0) {
    const int x = wi % 8, r = wi / 8;
    hs = r % nhs;
    wi = (r / nhs) * 8 + x;
  } else {
    hs = wi % nhs;
    wi /= nhs;
  }
  const int g = wi % p.Hkv;
  wi /= p.Hkv;
  const int t = wi % p.Sq;
  const int b = wi / p.Sq;
  const int nslots = p.topk;
  const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh;
  const int bound = bound_of(p, b);

  const int hl = 16 * hs + lt;  // head within the kv group
  const bool hvalid = hl < p.G;
  const int h = g * p.G + (hvalid ? hl : 0);
  const int64_t row = ((int64_t)b * p.Sq + t) * p.Hq + h;
  const float lse = p.lse[b * p.l_sb + t * p.l_ss + (int64_t)h * p.l_sh];
  // rows with no valid slot (lse = -inf) and padding heads contribute nothing
  const bool live = hvalid && lse != kNegInf;
  const float lse2 = live ? lse * kLog2e : __builtin_huge_valf();
  const float delta = live ? p.delta[row] : 0.f;

  const bf16* qrow = reinterpret_cast<const bf16*>(p.q) + b * p.q_sb + t * p.q_ss + (int64_t)h * p.q_sh;
  const bf16* dorow = reinterpret_cast<const bf16*>(p.dout) + b * p.do_sb + t * p.do_ss + (int64_t)h * p.do_sh;
  // B operands over dims (16x16x32): lane holds head lt, dims 32s + 8hq .. +7
  bf16x8 qb[kQS], dob[kQS];
#pragma unroll
  for (int s = 0; s < kQS; ++s) {
    bf16x8 x = *reinterpret_cast<const bf16x8*>(qrow + 32 * s + 8 * hq);
    bf16x8 y = *reinterpret_cast<const bf16x8*>(dorow + 32 * s + 8 * hq);
    if (!hvalid) {
      x = bf16x8{};
      y = bf16x8{};
    }
    qb[s] = x;
    dob[s] = y;
  }

  const char* kbase = reinterpret_cast<const char*>(p.k) + 2 * (b * p.k_sb + g * p.k_sh);
  const char* vbase = reinterpret_cast<const char*>(p.v) + 2 * (b * p.v_sb + g * p.v_sh);
  const uint32_t krow_bytes = (uint32_t)(2 * p.k_ss), vrow_bytes = (uint32_t)(2 * p.v_ss);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, (uint32_t)(2 * ((int64_t)(p.Skv - 1) * p.k_ss + 128)));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase, (uint32_t)(2 * ((int64_t)(p.Skv - 1) * p.v_ss + 128)));


  // Loads of tile j (K or V rows): instruction i of a lane loads the 16 bytes
  // at chunk lt of tile row i + 8 hq (4 whole rows per instruction; a lane's 8
  // rows are consecutive, so their ids are two 16-byte LDS reads).  Invalid
  // keys read zeros.
  auto load_rows = [&](int j, bf16x8 (&kr)[8], bf16x8 (&vr)[8]) {
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    const i32x4 id0 = *reinterpret_cast<const i32x4*>(s_idx + 32 * j + 8 * hq);
    const i32x4 id1 = *reinterpret_cast<const i32x4*>(s_idx + 32 * j + 8 * hq + 4);
    const int ids[8] = {id0[0], id0[1], id0[2], id0[3], id1[0], id1[1], id1[2], id1[3]};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t o = ids[i] >= 0 ? __umul24((uint32_t)ids[i], krow_bytes) + 16u * (uint32_t)lt : kOOB;
      kr[i] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, o, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t o = ids[i] >= 0 ? __umul24((uint32_t)ids[i], vrow_bytes) + 16u * (uint32_t)lt : kOOB;
      vr[i] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rv, o, 0, 0));
    }
  };

  f32x4 dqacc[kDT];
#pragma unroll
  for (int i = 0; i < kDT; ++i) dqacc[i] = f32x4{};

  // K^T operand reads of dQ^T: 4-row runs at keys 4 hq .. and 16 + 4 hq ..
  // (the dS^T B-operand order), 4-dim piece cc of dim tile ot
  const int rr = lt >> 2, cc = lt & 3;
  const uint32_t r0 = (uint32_t)((4 * hq + rr) * kPK) * 16u + (uint32_t)(4 * cc) * 2u;
  const uint32_t r1 = r0 + (uint32_t)(16 * kPK) * 16u;

  // tile j of the staged window of wt tiles
  auto step = [&](int j, int wt, bf16x8 (&kr)[8], bf16x8 (&vr)[8]) {
    const int* ib = s_idx + 32 * j;
    const uint32_t vmask = (uint32_t)__ballot(ib[lane & 31] >= 0);
    const bool more = j + 1 < wt;
    if (vmask == 0u) {  // wave-uniform: no valid key in this tile
      if (more) load_rows(j + 1, kr, vr);
      return;
    }
    // K and V rows of this tile into the LDS tiles (the previous tile's reads
    // of them are done: LDS operations of a wave complete in order), the
    // S^T / dP^T A operands (row 16 mt + lt, chunk 4 s + hq) back, then the
    // loads of the next tile into the freed registers
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      *reinterpret_cast<bf16x8*>(&s_k[(i + 8 * hq) * kPK + lt]) = kr[i];
      *reinterpret_cast<bf16x8*>(&s_v[(i + 8 * hq) * kPK + lt]) = vr[i];
    }
    if (more) load_rows(j + 1, kr, vr);

    // S^T and dP^T: two 16-key M tiles; the A operands (row 16 mt + lt,
    // chunk 4 s + hq) are read one contraction step ahead of their MFMAs
    // (the pins keep the compiler from hoisting all 16 reads, whose registers
    // would not fit next to a second wave on the SIMD)
    f32x4 sacc[2] = {f32x4{}, f32x4{}}, dpacc[2] = {f32x4{}, f32x4{}};
    auto read_ops = [&](int s, bf16x8 (&kc)[2], bf16x8 (&vc)[2]) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        kc[mt] = *reinterpret_cast<const bf16x8*>(&s_k[(16 * mt + lt) * kPK + 4 * s + hq]);
        vc[mt] = *reinterpret_cast<const bf16x8*>(&s_v[(16 * mt + lt) * kPK + 4 * s + hq]);
      }
    };
    bf16x8 kc[2][2], vc[2][2];
    read_ops(0, kc[0], vc[0]);
#pragma unroll
    for (int s = 0; s < kQS; ++s) {
      if (s + 1 < kQS) read_ops(s + 1, kc[(s + 1) & 1], vc[(s + 1) & 1]);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        sacc[mt] = mma16x32(kc[s & 1][mt], qb[s], sacc[mt]);
        dpacc[mt] = mma16x32(vc[s & 1][mt], dob[s], dpacc[mt]);
      }
      asm volatile("" ::: "memory");
    }
    // dS (fp32), packed to bf16 in the B layout of dQ^T = K^T dS^T
    bf16x8 dsb;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = mt * 16 + 4 * hq + e;
        const bool valid = (vmask >> key) & 1u;
        const float pr = valid ? exp2f(sacc[mt][e] * p.scale_log2 - lse2) : 0.f;
        dsb[4 * mt + e] = (bf16)(pr * (dpacc[mt][e] - delta));
      }
    // dQ^T += K^T dS^T: A = K^T from the staged tile (transposing reads)
#pragma unroll
    for (int ot = 0; ot < kDT; ++ot) {
      const bf16x4 lo = lds_read_tr16(s_k, r0 + (uint32_t)(ot * 16) * 2u);
      const bf16x4 hi = lds_read_tr16(s_k, r1 + (uint32_t)(ot * 16) * 2u);
      const bf16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      dqacc[ot] = mma16x32(a, dsb, dqacc[ot]);
    }
  };

  // The index row in windows of kIdxWin slots (invalid -> -1), so the LDS
  // (window + two row tiles, 19.4 KB) leaves room for two waves per SIMD.
  for (int base = 0; base < nslots; base += kIdxWin) {
    const int wn = min(kIdxWin, nslots - base);
    const int wt = (wn + 31) / 32;
    __syncthreads();  // (one wave: the previous window's reads come first)
    for (int i = lane; i < wt * 32; i += 64) {
      const int id = (i < wn) ? irow[base + i] : -1;
      s_idx[i] = (id >= 0 && id < bound) ? id : -1;
    }
    __syncthreads();
    bf16x8 kr[8], vr[8];
    load_rows(0, kr, vr);
    for (int j = 0; j < wt; ++j) step(j, wt, kr, vr);
  }

  if (!hvalid) return;
  bf16* dqrow = reinterpret_cast<bf16*>(p.dq) + b * p.dq_sb + t * p.dq_ss + (int64_t)h * p.dq_sh;
  // C layout: lane holds head lt, dims 16 ot + 4 hq + e
#pragma unroll
  for (int ot = 0; ot < kDT; ++ot) {
    const bf16x4 v4 = {(bf16)(dqacc[ot][0] * p.scale), (bf16)(dqacc[ot][1] * p.scale), (bf16)(dqacc[ot][2] * p.scale),
                       (bf16)(dqacc[ot][3] * p.scale)};
    *reinterpret_cast<bf16x4*>(dqrow + 16 * ot + 4 * hq) = v4;
  }
}

// dQ with 16 < G <= 128 on contiguous rows: the head groups of a work item
// are the NW waves of one workgroup (wave w: heads 16 w .. 16 w + 15, NW = G /
// 16 rounded up to a power of two), which gather each 32-key tile together
// (wave w its rows w R .. w R + R - 1, R = 32 / NW, whole rows one tile ahead
// in VGPRs) into double-buffered LDS tiles that all waves read their
// operands from, one LDS-only barrier per tile: a gathered row serves all G
// heads; with VK (v rows are the k rows: the reference's single kv) one
// gather serves K and V.  The per-wave math is bwd_dq_kernel's.
constexpr int kIdxCapQG = 2048;
constexpr int kMaxGroupQG = 128;

template <int NW, bool VK>
__global__ __launch_bounds__(64 * NW, 2) void bwd_dq_g_kernel(Params p) {
  constexpr int R = 32 / NW, RI = R / 4, THR = 64 * NW, TS = 32 * kPK;
  static_assert(R % 4 == 0 && NW * R == 32, "whole 4-row load instructions");
  __shared__ __attribute__((aligned(16))) int s_idx[kIdxCapQG];
  __shared__ u32x4 s_k[2][TS];
  __shared__ u32x4 s_v[2][VK ? 1 : TS];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lt = lane & 15, hq = lane >> 4;

  int wi = blockIdx.x;
  const int g = wi % p.Hkv;
  wi /= p.Hkv;
  const int t = wi % p.Sq;
  const int b = wi / p.Sq;
  const int nslots = p.topk;
  const int ntiles = (nslots + 31) / 32;
  const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh;
  const int bound = bound_of(p, b);
  for (int i = tid; i < ntiles * 32; i += THR) {
    const int id = (i < nslots) ? irow[i] : -1;
    s_idx[i] = (id >= 0 && id < bound) ? id : -1;
  }

  const int hl = 16 * wave + lt;  // head within the kv group
  const bool hvalid = hl < p.G;
  const int h = g * p.G + (hvalid ? hl : 0);
  const int64_t row = ((int64_t)b * p.Sq + t) * p.Hq + h;
  const float lse = p.lse[b * p.l_sb + t * p.l_ss + (int64_t)h * p.l_sh];
  const bool live = hvalid && lse != kNegInf;
  const float lse2 = live ? lse * kLog2e : __builtin_huge_valf();
  const float delta = live ? p.delta[row] : 0.f;
  const bf16* qrow = reinterpret_cast<const bf16*>(p.q) + b * p.q_sb + t * p.q_ss + (int64_t)h * p.q_sh;
  const bf16* dorow = reinterpret_cast<const bf16*>(p.dout) + b * p.do_sb + t * p.do_ss + (int64_t)h * p.do_sh;
  bf16x8 qb[kQS], dob[kQS];
#pragma unroll
  for (int s = 0; s < kQS; ++s) {
    bf16x8 x = *reinterpret_cast<const bf16x8*>(qrow + 32 * s + 8 * hq);
    bf16x8 y = *reinterpret_cast<const bf16x8*>(dorow + 32 * s + 8 * hq);
    if (!hvalid) {
      x = bf16x8{};
      y = bf16x8{};
    }
    qb[s] = x;
    dob[s] = y;
  }
  const char* kbase = reinterpret_cast<const char*>(p.k) + 2 * (b * p.k_sb + g * p.k_sh);
  const char* vbase = reinterpret_cast<const char*>(p.v) + 2 * (b * p.v_sb + g * p.v_sh);
  const uint32_t krow_bytes = (uint32_t)(2 * p.k_ss), vrow_bytes = (uint32_t)(2 * p.v_ss);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, (uint32_t)(2 * ((int64_t)(p.Skv - 1) * p.k_ss + 128)));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase, (uint32_t)(2 * ((int64_t)(p.Skv - 1) * p.v_ss + 128)));

  // rows of tile j this lane loads: instruction i, chunk lt of tile row
  // wave R + RI hq + i; invalid keys read zeros
  const int row0 = wave * R + RI * hq;
  auto load_rows = [&](int j, bf16x8 (&kr)[RI], bf16x8 (&vr)[RI]) {
#pragma unroll
    for (int i = 0; i < RI; ++i) {
      const int id = s_idx[32 * j + row0 + i];
      const uint32_t ko = id >= 0 ? __umul24((uint32_t)id, krow_bytes) + 16u * (uint32_t)lt : kOOB;
      kr[i] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, ko, 0, 0));
      if constexpr (!VK) {
        const uint32_t vo = id >= 0 ? __umul24((uint32_t)id, vrow_bytes) + 16u * (uint32_t)lt : kOOB;
        vr[i] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rv, vo, 0, 0));
      }
    }
  };
  auto write_rows = [&](int buf, const bf16x8 (&kr)[RI], const bf16x8 (&vr)[RI]) {
#pragma unroll
    for (int i = 0; i < RI; ++i) {
      *reinterpret_cast<bf16x8*>(&s_k[buf][(row0 + i) * kPK + lt]) = kr[i];
      if constexpr (!VK) *reinterpret_cast<bf16x8*>(&s_v[buf][(row0 + i) * kPK + lt]) = vr[i];
    }
  };
  auto lds_barrier = []() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  f32x4 dqacc[kDT];
#pragma unroll
  for (int i = 0; i < kDT; ++i) dqacc[i] = f32x4{};
  const int rr = lt >> 2, cc = lt & 3;
  const uint32_t r0 = (uint32_t)((4 * hq + rr) * kPK) * 16u + (uint32_t)(4 * cc) * 2u;
  const uint32_t r1 = r0 + (uint32_t)(16 * kPK) * 16u;

  __syncthreads();  // ids staged
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
    const int* ib = s_idx + 32 * j;
    const uint32_t vmask = (uint32_t)__ballot(ib[lane & 31] >= 0);
    if (vmask != 0u) {  // (uniform over the workgroup: every wave sees the same ids)
      // S^T and dP^T: two 16-key M tiles; A operands (row 16 mt + lt,
      // chunk 4 s + hq) read one contraction step ahead of their MFMAs
      f32x4 sacc[2] = {f32x4{}, f32x4{}}, dpacc[2] = {f32x4{}, f32x4{}};
      auto read_ops = [&](int s, bf16x8 (&kc)[2], bf16x8 (&vc)[2]) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          kc[mt] = *reinterpret_cast<const bf16x8*>(&kt[(16 * mt + lt) * kPK + 4 * s + hq]);
          vc[mt] = *reinterpret_cast<const bf16x8*>(&vt[(16 * mt + lt) * kPK + 4 * s + hq]);
        }
      };
      bf16x8 kc[2][2], vc[2][2];
      read_ops(0, kc[0], vc[0]);
#pragma unroll
      for (int s = 0; s < kQS; ++s) {
        if (s + 1 < kQS) read_ops(s + 1, kc[(s + 1) & 1], vc[(s + 1) & 1]);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          sacc[mt] = mma16x32(kc[s & 1][mt], qb[s], sacc[mt]);
          dpacc[mt] = mma16x32(vc[s & 1][mt], dob[s], dpacc[mt]);
        }
        asm volatile("" ::: "memory");
      }
      bf16x8 dsb;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = mt * 16 + 4 * hq + e;
          const bool valid = (vmask >> key) & 1u;
          const float pr = valid ? exp2f(sacc[mt][e] * p.scale_log2 - lse2) : 0.f;
          dsb[4 * mt + e] = (bf16)(pr * (dpacc[mt][e] - delta));
        }
      // dQ^T += K^T dS^T: A = K^T from the staged tile (transposing reads)
#pragma unroll
      for (int ot = 0; ot < kDT; ++ot) {
        const bf16x4 lo = lds_read_tr16(kt, r0 + (uint32_t)(ot * 16) * 2u);
        const bf16x4 hi = lds_read_tr16(kt, r1 + (uint32_t)(ot * 16) * 2u);
        const bf16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        dqacc[ot] = mma16x32(a, dsb, dqacc[ot]);
      }
    }
    // tile j + 1's rows into the other buffer (read by nobody since the last
    // barrier), then tile j + 2's loads
    if (j + 1 < ntiles) {
      write_rows(cur ^ 1, kr, vr);
      if (j + 2 < ntiles) load_rows(j + 2, kr, vr);
    }
    lds_barrier();
  }

  if (!hvalid) return;
  bf16* dqrow = reinterpret_cast<bf16*>(p.dq) + b * p.dq_sb + t * p.dq_ss + (int64_t)h * p.dq_sh;
#pragma unroll
  for (int ot = 0; ot < kDT; ++ot) {
    const bf16x4 v4 = {(bf16)(dqacc[ot][0] * p.scale), (bf16)(dqacc[ot][1] * p.scale), (bf16)(dqacc[ot][2] * p.scale),
                       (bf16)(dqacc[ot][3] * p.scale)};
    *reinterpret_cast<bf16x4*>(dqrow + 16 * ot + 4 * hq) = v4;
  }
}

bool dq_g_supported(const Params& p) { return p.G > 16 && p.G <= kMaxGroupQG && p.topk <= kIdxCapQG; }

// dK/dV of index slots that repeat an earlier slot's key in their row (p.dup,
// written by the index inversion; the key-major pass counts each key once
// per row).  Such slots are absent from ordinary index sets, so this is
// plain VALU code: one wave per work item scans its flags and, per flagged
// slot and head, forms S and dP as dot products over the 128 dims (2 per
// lane), P and dS, and adds P dO and scale dS Q to the key's rows with fp32
// atomics (SFA.py:719-853 for the math).
__global__ __launch_bounds__(256) void bwd_dup_kernel(Params p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t item = (int64_t)blockIdx.x * 4 + wave;
  if (item >= (int64_t)p.B * p.Sq * p.Hkv) return;  // the whole wave
  const int g = (int)(item % p.Hkv);
  const int t = (int)((item / p.Hkv) % p.Sq);
  const int b = (int)(item / ((int64_t)p.Hkv * p.Sq));
  const uint8_t* drow = p.dup + item * p.topk;
  const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh;
  const int bound = bound_of(p, b);
  float* const dkb = p.dk_acc + ((int64_t)b * p.Skv * p.Hkv + g) * 128 + 2 * lane;
  float* const dvb = p.dv_acc + ((int64_t)b * p.Skv * p.Hkv + g) * 128 + 2 * lane;
  const int64_t acc_row = (int64_t)p.Hkv * 128;
  auto wave_sum = [](float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
  };
  // skip 1024-slot blocks without a flag with one 16-byte read per lane (the
  // flag rows are 16-byte aligned when topk is a multiple of 16)
  const bool vec = p.topk % 16 == 0;
  for (int i0 = 0; i0 < p.topk; i0 += 64) {
    if (vec && i0 % 1024 == 0) {
      const int v0 = i0 + 16 * lane;
      const u32x4 f = v0 < p.topk ? *reinterpret_cast<const u32x4*>(drow + v0) : u32x4{0u, 0u, 0u, 0u};
      if (__ballot((f.x | f.y | f.z | f.w) != 0u) == 0) {
        i0 += 1024 - 64;  // (the loop adds the other 64)
        continue;
      }
    }
    const int i = i0 + lane;
    int id = -1;
    if (i < p.topk && drow[i] != 0) id = irow[i];
    const bool flagged = id >= 0 && id < bound;
    uint64_t m = __ballot(flagged);
    while (m != 0) {
      const int sl = __builtin_ctzll(m);
      m &= m - 1;
      const int key = __shfl(id, sl, 64);
      const bf16* krow = reinterpret_cast<const bf16*>(p.k) + b * p.k_sb + (int64_t)key * p.k_ss + g * p.k_sh;
      const bf16* vrow = reinterpret_cast<const bf16*>(p.v) + b * p.v_sb + (int64_t)key * p.v_ss + g * p.v_sh;
      const float k0 = (float)krow[2 * lane], k1 = (float)krow[2 * lane + 1];
      const float v0 = (float)vrow[2 * lane], v1 = (float)vrow[2 * lane + 1];
      float dv0 = 0.f, dv1 = 0.f, dk0 = 0.f, dk1 = 0.f;
      for (int hh = 0; hh < p.G; ++hh) {
        const int h = g * p.G + hh;
        const float lse = p.lse[b * p.l_sb + t * p.l_ss + (int64_t)h * p.l_sh];
        if (lse == kNegInf) continue;  // a row with no valid slot
        const bf16* qrow = reinterpret_cast<const bf16*>(p.q) + b * p.q_sb + t * p.q_ss + (int64_t)h * p.q_sh;
        const bf16* dorow =
            reinterpret_cast<const bf16*>(p.dout) + b * p.do_sb + t * p.do_ss + (int64_t)h * p.do_sh;
        const float q0 = (float)qrow[2 * lane], q1 = (float)qrow[2 * lane + 1];
        const float d0 = (float)dorow[2 * lane], d1 = (float)dorow[2 * lane + 1];
        const float sc = wave_sum(q0 * k0 + q1 * k1);
        const float dp = wave_sum(d0 * v0 + d1 * v1);
        const float pr = exp2f(sc * p.scale_log2 - lse * kLog2e);
        const float ds = pr * (dp - p.delta[((int64_t)b * p.Sq + t) * p.Hq + h]);
        dv0 += pr * d0;
        dv1 += pr * d1;
        dk0 += ds * q0;
        dk1 += ds * q1;
      }
      atomicAdd(dvb + (int64_t)key * acc_row, dv0);
      atomicAdd(dvb + (int64_t)key * acc_row + 1, dv1);
      atomicAdd(dkb + (int64_t)key * acc_row, dk0 * p.scale);
      atomicAdd(dkb + (int64_t)key * acc_row + 1, dk1 * p.scale);
    }
  }
}

}  // namespace

bool bwd_dq_supported(const Params& p) {
  if (p.Dqk != 128 || p.Dv != 128) return false;
  if (p.G > kMaxGroupQ || p.G < 1 || p.topk > kIdxCapQ) return false;
  const int64_t kb = 2 * ((int64_t)(p.Skv - 1) * p.k_ss + 128);
  const int64_t vb = 2 * ((int64_t)(p.Skv - 1) * p.v_ss + 128);
  return kb < (int64_t)kOOB && vb < (int64_t)kOOB && fits_u24(2 * p.k_ss) && fits_u24(2 * p.v_ss);
}

hipError_t launch_bwd_dq(const Params& p, hipStream_t s) {
  if (dq_g_supported(p)) {
    const int64_t n = (int64_t)p.B * p.Sq * p.Hkv;
    const bool vk = p.v == p.k && p.v_sb == p.k_sb && p.v_ss == p.k_ss && p.v_sh == p.k_sh;
    const int nw = p.G <= 32 ? 2 : p.G <= 64 ? 4 : 8;
#define SFA_DQG(NW)                                                                                \
  if (nw == NW) {                                                                                  \
    if (vk)                                                                                        \
      hipLaunchKernelGGL((bwd_dq_g_kernel<NW, true>), dim3((unsigned)n), dim3(64 * NW), 0, s, p);  \
    else                                                                                           \
      hipLaunchKernelGGL((bwd_dq_g_kernel<NW, false>), dim3((unsigned)n), dim3(64 * NW), 0, s, p); \
    return hipGetLastError();                                                                      \
  }
    SFA_DQG(2)
    SFA_DQG(4)
    SFA_DQG(8)
#undef SFA_DQG
  }
  const int64_t n = (int64_t)p.B * p.Sq * p.Hkv * ((p.G + 15) / 16);
  hipLaunchKernelGGL(bwd_dq_kernel, dim3((unsigned)n), dim3(64), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_bwd_dup(const Params& p, hipStream_t s) {
  const int64_t n = (int64_t)p.B * p.Sq * p.Hkv;
  hipLaunchKernelGGL(bwd_dup_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace sfa

// gfx950 dQ (and dsink) kernel of the deterministic backward for d_qk = d_v =
// 128 and G <= 16 query heads per KV head: register-direct gather.
//
// Reference: `_attn_bwd_dq_dsink` / `_inner_dq` (SFA.py:856-1002, 613-716).
// With the deterministic dK/dV scheme (sfa_bwd_csr.hip) the query-major pass
// only produces dQ and dsink, plus the dK/dV rows of index slots that repeat
// an earlier slot's key (flagged in p.dup; fp32 atomics, as in the atomic
// scheme).  As in the d = 128 forward (sfa_fwd_d128.hip), one wave holds all
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

constexpr int kIdxCapQ = 2048;  // slots staged in LDS per work item
constexpr int kQS = 4;          // 128 / 32 contraction steps over the head dim
constexpr int kDT = 8;          // 128 / 16 dim tiles
constexpr int kPK = 17;         // K staging row pitch in 16-byte slots (odd: conflict-free reads)
constexpr int kPStride = 36;    // P / dS patch row stride (keys) in bf16

typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;

__device__ __forceinline__ f32x4 mma16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma16x16(bf16x4_t a, bf16x4_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(64, 1) void bwd_dq_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) int s_idx[kIdxCapQ];
  __shared__ __attribute__((aligned(16))) uint8_t s_dup[kIdxCapQ];  // slot takes the dK/dV scatter
  __shared__ u32x4 s_k[32 * kPK];
  __shared__ u32x4 s_v[32 * kPK];
  __shared__ __attribute__((aligned(16))) bf16 s_patch[2][16 * kPStride];

  const int lane = threadIdx.x;
  const int lt = lane & 15;  // head column / key row within a 16-row M-tile
  const int hq = lane >> 4;  // lane group

  int wi = blockIdx.x;
  const int g = wi % p.Hkv;
  wi /= p.Hkv;
  const int t = wi % p.Sq;
  const int b = wi / p.Sq;
  const int nslots = p.topk;
  const int ntiles = (nslots + 31) / 32;

  {
    const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh;
    const uint8_t* drow = p.dup + (((int64_t)b * p.Sq + t) * p.Hkv + g) * p.topk;
    const int bound = bound_of(p, b);
    for (int i = lane; i < ntiles * 32; i += 64) {
      const int id = (i < nslots) ? irow[i] : -1;
      const bool valid = id >= 0 && id < bound;
      s_idx[i] = valid ? id : -1;
      s_dup[i] = valid && drow[i] != 0;
    }
  }

  const bool hvalid = lt < p.G;
  const int h = g * p.G + (hvalid ? lt : 0);
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

  __syncthreads();  // indices staged (one wave: orders the LDS writes and reads)

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

  float* dkb = p.dk_acc + ((int64_t)b * p.Skv * p.Hkv + g) * 128;
  float* dvb = p.dv_acc + ((int64_t)b * p.Skv * p.Hkv + g) * 128;
  const int64_t acc_row = (int64_t)p.Hkv * 128;

  f32x4 dqacc[kDT];
#pragma unroll
  for (int i = 0; i < kDT; ++i) dqacc[i] = f32x4{};

  // K^T operand reads of dQ^T: 4-row runs at keys 4 hq .. and 16 + 4 hq ..
  // (the dS^T B-operand order), 4-dim piece cc of dim tile ot
  const int rr = lt >> 2, cc = lt & 3;
  const uint32_t r0 = (uint32_t)((4 * hq + rr) * kPK) * 16u + (uint32_t)(4 * cc) * 2u;
  const uint32_t r1 = r0 + (uint32_t)(16 * kPK) * 16u;

  auto step = [&](int j, bf16x8 (&kr)[8], bf16x8 (&vr)[8]) {
    const int* ib = s_idx + 32 * j;
    const uint32_t vmask = (uint32_t)__ballot(ib[lane & 31] >= 0);
    const bool more = j + 1 < ntiles;
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
    bf16x8 kc[8], vc[8];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        kc[4 * mt + s] = *reinterpret_cast<const bf16x8*>(&s_k[(16 * mt + lt) * kPK + 4 * s + hq]);
        vc[4 * mt + s] = *reinterpret_cast<const bf16x8*>(&s_v[(16 * mt + lt) * kPK + 4 * s + hq]);
      }
    if (more) load_rows(j + 1, kr, vr);

    // S^T and dP^T: two 16-key M tiles
    f32x4 sacc[2] = {f32x4{}, f32x4{}}, dpacc[2] = {f32x4{}, f32x4{}};
#pragma unroll
    for (int s = 0; s < kQS; ++s)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        sacc[mt] = mma16x32(kc[4 * mt + s], qb[s], sacc[mt]);
        dpacc[mt] = mma16x32(vc[4 * mt + s], dob[s], dpacc[mt]);
      }
    // P and dS (fp32), packed to bf16 in the B layout of dQ^T = K^T dS^T
    bf16x8 dsb;
    bf16x4_t pv[2], dv[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = mt * 16 + 4 * hq + e;
        const bool valid = (vmask >> key) & 1u;
        const float pr = valid ? exp2f(sacc[mt][e] * p.scale_log2 - lse2) : 0.f;
        const float ds = pr * (dpacc[mt][e] - delta);
        pv[mt][e] = (bf16)pr;
        dv[mt][e] = (bf16)ds;
        dsb[4 * mt + e] = dv[mt][e];
      }
    // dQ^T += K^T dS^T: A = K^T from the staged tile (transposing reads)
#pragma unroll
    for (int ot = 0; ot < kDT; ++ot) {
      const bf16x4 lo = lds_read_tr16(s_k, r0 + (uint32_t)(ot * 16) * 2u);
      const bf16x4 hi = lds_read_tr16(s_k, r1 + (uint32_t)(ot * 16) * 2u);
      const bf16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      dqacc[ot] = mma16x32(a, dsb, dqacc[ot]);
    }
    // Repeated keys: dV = P^T dO and dK = scale dS^T Q over the G heads for
    // the flagged slots, rows scattered atomically.  P^T / dS^T go through a
    // [head][key] patch and come back (transposing reads) as the A operands
    // of the head contractions (16x16x16); the head-side B operands are read
    // from global memory here (rare path).
    const uint8_t* fb = s_dup + 32 * j;
    if (__ballot(fb[lane & 31] != 0) == 0u) return;  // wave-uniform: nothing to scatter
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      *reinterpret_cast<bf16x4_t*>(&s_patch[0][lt * kPStride + mt * 16 + 4 * hq]) = pv[mt];
      *reinterpret_cast<bf16x4_t*>(&s_patch[1][lt * kPStride + mt * 16 + 4 * hq]) = dv[mt];
    }
    const bf16* q0 = reinterpret_cast<const bf16*>(p.q) + b * p.q_sb + t * p.q_ss + (int64_t)(g * p.G) * p.q_sh;
    const bf16* d0 = reinterpret_cast<const bf16*>(p.dout) + b * p.do_sb + t * p.do_ss + (int64_t)(g * p.G) * p.do_sh;
#pragma unroll 1
    for (int mk = 0; mk < 2; ++mk) {
      const uint32_t poff = (uint32_t)(((4 * hq + rr) * kPStride + mk * 16 + 4 * cc) * 2);
      const bf16x4 ap = lds_read_tr16(s_patch[0], poff);
      const bf16x4 as = lds_read_tr16(s_patch[1], poff);
      const int4 ids = *reinterpret_cast<const int4*>(ib + mk * 16 + 4 * hq);
      const uchar4 fl = *reinterpret_cast<const uchar4*>(fb + mk * 16 + 4 * hq);
      const int idv[4] = {fl.x ? ids.x : -1, fl.y ? ids.y : -1, fl.z ? ids.z : -1, fl.w ? ids.w : -1};
#pragma unroll 1
      for (int nd = 0; nd < kDT; ++nd) {
        // B operands over heads: lane holds heads 4hq .. 4hq+3 of dim 16nd + lt
        bf16x4_t qh, doh;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int hh = 4 * hq + e;
          const bool ok = hh < p.G;
          qh[e] = ok ? q0[(int64_t)hh * p.q_sh + 16 * nd + lt] : (bf16)0.f;
          doh[e] = ok ? d0[(int64_t)hh * p.do_sh + 16 * nd + lt] : (bf16)0.f;
        }
        const f32x4 dvr = mma16x16(ap, doh, f32x4{});
        const f32x4 dkr = mma16x16(as, qh, f32x4{});
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (idv[e] >= 0) {
            atomicAdd(dvb + (int64_t)idv[e] * acc_row + 16 * nd + lt, dvr[e]);
            atomicAdd(dkb + (int64_t)idv[e] * acc_row + 16 * nd + lt, dkr[e] * p.scale);
          }
        }
      }
    }
  };

  {
    bf16x8 kr[8], vr[8];
    if (ntiles > 0) load_rows(0, kr, vr);
    for (int j = 0; j < ntiles; ++j) step(j, kr, vr);
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

}  // namespace

bool bwd_dq_supported(const Params& p) {
  if (p.Dqk != 128 || p.Dv != 128) return false;
  if (p.G > 16 || p.G < 1 || p.topk > kIdxCapQ) return false;
  const int64_t kb = 2 * ((int64_t)(p.Skv - 1) * p.k_ss + 128);
  const int64_t vb = 2 * ((int64_t)(p.Skv - 1) * p.v_ss + 128);
  return kb < (int64_t)kOOB && vb < (int64_t)kOOB && fits_u24(2 * p.k_ss) && fits_u24(2 * p.v_ss);
}

hipError_t launch_bwd_dq(const Params& p, hipStream_t s) {
  const int64_t n = (int64_t)p.B * p.Sq * p.Hkv;
  hipLaunchKernelGGL(bwd_dq_kernel, dim3((unsigned)n), dim3(64), 0, s, p);
  return hipGetLastError();
}

}  // namespace sfa

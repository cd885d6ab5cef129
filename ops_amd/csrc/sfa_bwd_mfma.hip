// gfx950 MFMA backward of top-k sparse flash attention (bf16 in, fp32
// accumulate), for head dims D = d_qk = d_v that are multiples of 32
// (instantiated for 128 and 64); up to 16 query heads per workgroup (G > 16
// is split into head groups of 16).
//
// Reference: `_attn_bwd_dq_dsink` / `_inner_dq` (SFA.py:856-1002, 613-716) and
// `_attn_bwd_dk_dv` / `_inner_dkv` (SFA.py:1005-1145, 719-853).  The reference
// recomputes S and dP twice (once per kernel) and stages every intermediate in
// global memory; here one kernel computes each (query, key) pair once:
//
//  * One workgroup owns one (batch, query, kv-head) work item and all its G
//    query heads; its 4 waves split every 128-key tile into 4 x 32 keys.
//  * Per 32-key wave tile (16x16x32 MFMA, keys as rows, heads as columns):
//      S^T  = K Q^T,  dP^T = V dO^T
//      P    = 2^(S·scale·log2e − lse2)  (masked),  dS = P (dP − δ)
//      dQ^T += K^T dS^T      (K^T read with ds_read_b64_tr_b16; the S^T
//                             accumulator layout is already dS^T's B layout)
//      P^T and dS^T go through a 1 KiB per-wave LDS patch ([head][key]) and
//      come back, via transposing reads, as the A operands of the
//      head-contractions (16x16x16 MFMA):
//      dV  = P^T  dO          dK = scale · dS^T Q
//    and dV/dK rows are scattered with fp32 atomics into per-key
//    accumulators (the reference's scheme, SFA.py:849-853): its cost does
//    not grow with the density of the index set and it needs no inverted
//    index of the top-k rows.  This kernel serves the atomic dK/dV mode; the
//    deterministic mode runs sfa_bwd_dq.hip (dQ) and sfa_bwd_csr.hip (dK/dV).
//  * dQ partials of the 4 waves are summed through LDS at the end and
//    written once (no atomics on dQ).
//  * δ = Σ O·dO (minus any gradient on lse) comes from a preceding kernel.

#include "sfa_common.h"
#include "sfa_lds.h"

namespace sfa {
namespace {

constexpr int kBwdIdxCap = 2048;  // slots staged in LDS per work item
constexpr int kMaxGroupB = 256;   // query heads per KV head (16 groups of 16)

typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;

template <int D_>
struct BwdCfg {
  static constexpr int D = D_;
  static constexpr int kWaves = 4;
  static constexpr int kThreads = 256;
  static constexpr int NKT = 128;          // keys per workgroup tile (32 per wave)
  static constexpr int CH = D / 8;         // 16-byte chunks per row
  static constexpr int PITCH = CH + 1;     // LDS row pitch in 16-byte slots
  static constexpr int TBUF = NKT * PITCH;
  static constexpr int QS = D / 32;        // 16x16x32 steps over the head dim
  static constexpr int DT = D / 16;        // 16-wide dim tiles
  static constexpr int PSTRIDE = 36;       // patch row stride (keys) in bf16
  static_assert(D % 32 == 0, "head dim must be a multiple of 32");
};

__device__ __forceinline__ f32x4 mma16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma16x16(bf16x4_t a, bf16x4_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

template <class C>
__global__ __launch_bounds__(C::kThreads, 1) void bwd_mfma_kernel(Params p) {
  constexpr int D = C::D;
  __shared__ __attribute__((aligned(16))) int s_idx[kBwdIdxCap];
  __shared__ u32x4 s_k0[C::TBUF];
  __shared__ u32x4 s_k1[C::TBUF];
  __shared__ u32x4 s_v0[C::TBUF];
  __shared__ u32x4 s_v1[C::TBUF];
  __shared__ __attribute__((aligned(16))) bf16 s_patch[C::kWaves][2][16 * C::PSTRIDE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ks = wave;          // key sub-range of this wave within a tile
  const int lt = lane & 15;     // head column / MFMA row within 16
  const int hq = lane >> 4;     // lane group

  // work item and head group (the head groups of an item on one XCD)
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
  const int ntiles = (nslots + C::NKT - 1) / C::NKT;
  const int hg0 = 16 * hs;  // first head (within the kv group) of this workgroup

  {
    const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh;
    const int bound = bound_of(p, b);
    for (int i = tid; i < ntiles * C::NKT; i += C::kThreads) {
      const int id = (i < nslots) ? irow[i] : -1;
      s_idx[i] = (id >= 0 && id < bound) ? id : -1;
    }
  }

  // per-lane head: hl = hg0 + lt
  const int hl = hg0 + lt;
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
  // B operands over dims (16x16x32): lane holds head hl, dims 32s + 8hq .. +7
  bf16x8 qb[C::QS], dob[C::QS];
#pragma unroll
  for (int s = 0; s < C::QS; ++s) {
    bf16x8 x = *reinterpret_cast<const bf16x8*>(qrow + 32 * s + 8 * hq);
    bf16x8 y = *reinterpret_cast<const bf16x8*>(dorow + 32 * s + 8 * hq);
    if (!hvalid) {
      x = bf16x8{};
      y = bf16x8{};
    }
    qb[s] = x;
    dob[s] = y;
  }
  // B operands over heads (16x16x16): lane holds heads hg0 + 4hq .. +3 of dim 16nd + lt
  bf16x4_t qh[C::DT], doh[C::DT];
  {
    const bf16* q0 = reinterpret_cast<const bf16*>(p.q) + b * p.q_sb + t * p.q_ss + (int64_t)(g * p.G) * p.q_sh;
    const bf16* d0 = reinterpret_cast<const bf16*>(p.dout) + b * p.do_sb + t * p.do_ss + (int64_t)(g * p.G) * p.do_sh;
#pragma unroll
    for (int nd = 0; nd < C::DT; ++nd) {
      bf16x4_t x, y;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int hh = hg0 + 4 * hq + j;
        const bool ok = hh < p.G;
        x[j] = ok ? q0[(int64_t)hh * p.q_sh + 16 * nd + lt] : (bf16)0.f;
        y[j] = ok ? d0[(int64_t)hh * p.do_sh + 16 * nd + lt] : (bf16)0.f;
      }
      qh[nd] = x;
      doh[nd] = y;
    }
  }

  const char* kbase = reinterpret_cast<const char*>(p.k) + 2 * (b * p.k_sb + g * p.k_sh);
  const char* vbase = reinterpret_cast<const char*>(p.v) + 2 * (b * p.v_sb + g * p.v_sh);
  const uint32_t krow_bytes = (uint32_t)(2 * p.k_ss), vrow_bytes = (uint32_t)(2 * p.v_ss);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, (uint32_t)(2 * ((int64_t)(p.Skv - 1) * p.k_ss + D)));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase, (uint32_t)(2 * ((int64_t)(p.Skv - 1) * p.v_ss + D)));
  auto gather = [&](int tile, u32x4* kdst, u32x4* vdst) {
    const int* ib = s_idx + tile * C::NKT;
    gather_tile<C::NKT, C::CH, C::kThreads>(ib, kdst, rk, krow_bytes, tid, wave);
    gather_tile<C::NKT, C::CH, C::kThreads>(ib, vdst, rv, vrow_bytes, tid, wave);
  };

  float* dkb = p.dk_acc + ((int64_t)b * p.Skv * p.Hkv + g) * D;
  float* dvb = p.dv_acc + ((int64_t)b * p.Skv * p.Hkv + g) * D;
  const int64_t acc_row = (int64_t)p.Hkv * D;

  f32x4 dqacc[C::DT];
#pragma unroll
  for (int i = 0; i < C::DT; ++i) dqacc[i] = f32x4{};

  bf16* patch_p = s_patch[wave][0];
  bf16* patch_s = s_patch[wave][1];

  auto compute = [&](int tile, const u32x4* kt, const u32x4* vt) {
    const int* ib = s_idx + tile * C::NKT + ks * 32;
    const uint32_t vmask = (uint32_t)__ballot(ib[lane & 31] >= 0);
    if (vmask == 0u) return;  // wave-uniform: no valid key in this sub-tile

    // S^T and dP^T: two 16-key M tiles
    f32x4 sacc[2] = {f32x4{}, f32x4{}}, dpacc[2] = {f32x4{}, f32x4{}};
#pragma unroll
    for (int s = 0; s < C::QS; ++s) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const uint32_t off = (uint32_t)((ks * 32 + mt * 16 + lt) * C::PITCH + 4 * s + hq) * 16u;
        sacc[mt] = mma16x32(lds_read_b128(kt, off), qb[s], sacc[mt]);
        dpacc[mt] = mma16x32(lds_read_b128(vt, off), dob[s], dpacc[mt]);
      }
    }
    // P and dS (fp32), packed to bf16 in the B layout of dQ^T = K^T dS^T and
    // written transposed ([head][key]) to this wave's patch
    bf16x8 dsb;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      bf16x4_t pv, dv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = mt * 16 + 4 * hq + e;
        const bool valid = (vmask >> key) & 1u;
        const float pr = valid ? exp2f(sacc[mt][e] * p.scale_log2 - lse2) : 0.f;
        const float ds = pr * (dpacc[mt][e] - delta);
        pv[e] = (bf16)pr;
        dv[e] = (bf16)ds;
        dsb[4 * mt + e] = dv[e];
      }
      *reinterpret_cast<bf16x4_t*>(patch_p + lt * C::PSTRIDE + mt * 16 + 4 * hq) = pv;
      *reinterpret_cast<bf16x4_t*>(patch_s + lt * C::PSTRIDE + mt * 16 + 4 * hq) = dv;
    }
    // dQ^T += K^T dS^T: A = K^T from the k tile (transposing reads)
    {
      const int rr = lt >> 2, cc = lt & 3;
      const uint32_t r0 = (uint32_t)((ks * 32 + 4 * hq + rr) * C::PITCH) * 16u + (uint32_t)(4 * cc) * 2u;
      const uint32_t r1 = r0 + (uint32_t)(16 * C::PITCH) * 16u;
#pragma unroll
      for (int ot = 0; ot < C::DT; ++ot) {
        const bf16x4 lo = lds_read_tr16(kt, r0 + (uint32_t)(ot * 16) * 2u);
        const bf16x4 hi = lds_read_tr16(kt, r1 + (uint32_t)(ot * 16) * 2u);
        const bf16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        dqacc[ot] = mma16x32(a, dsb, dqacc[ot]);
      }
    }
    // dV = P^T dO and dK = dS^T Q over the G heads; rows scattered atomically
    const int rr = lt >> 2, cc = lt & 3;
#pragma unroll
    for (int mk = 0; mk < 2; ++mk) {
      const uint32_t poff = (uint32_t)(((4 * hq + rr) * C::PSTRIDE + mk * 16 + 4 * cc) * 2);
      const bf16x4 ap = lds_read_tr16(patch_p, poff);
      const bf16x4 as = lds_read_tr16(patch_s, poff);
      const int4 ids = *reinterpret_cast<const int4*>(ib + mk * 16 + 4 * hq);
      const int idv[4] = {ids.x, ids.y, ids.z, ids.w};
#pragma unroll
      for (int nd = 0; nd < C::DT; ++nd) {
        const f32x4 dv = mma16x16(ap, doh[nd], f32x4{});
        const f32x4 dk = mma16x16(as, qh[nd], f32x4{});
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (idv[e] >= 0) {
            atomicAdd(dvb + (int64_t)idv[e] * acc_row + 16 * nd + lt, dv[e]);
            atomicAdd(dkb + (int64_t)idv[e] * acc_row + 16 * nd + lt, dk[e] * p.scale);
          }
        }
      }
    }
  };

  __syncthreads();  // indices staged
  if (ntiles > 0) gather(0, s_k0, s_v0);
  __syncthreads();
  for (int j = 0; j < ntiles; j += 2) {
    if (j + 1 < ntiles) gather(j + 1, s_k1, s_v1);
    compute(j, s_k0, s_v0);
    __syncthreads();
    if (j + 1 < ntiles) {
      if (j + 2 < ntiles) gather(j + 2, s_k0, s_v0);
      compute(j + 1, s_k1, s_v1);
      __syncthreads();
    }
  }

  // dQ: sum the 4 waves' partials through LDS (the last barrier ended every
  // use of the tiles), scale, write
  float* s_dq = reinterpret_cast<float*>(s_k0);  // [kWaves][DT][4][64]
  static_assert(C::kWaves * C::DT * 4 * 64 * 4 <= C::TBUF * 16, "dQ merge fits");
#pragma unroll
  for (int ot = 0; ot < C::DT; ++ot)
#pragma unroll
    for (int e = 0; e < 4; ++e) s_dq[((wave * C::DT + ot) * 4 + e) * 64 + lane] = dqacc[ot][e];
  __syncthreads();
  if (!hvalid) return;
  bf16* dqrow = reinterpret_cast<bf16*>(p.dq) + b * p.dq_sb + t * p.dq_ss + (int64_t)h * p.dq_sh;
  // wave w writes dim tiles w, w + 4, ...
  for (int ot = wave; ot < C::DT; ot += C::kWaves) {
    bf16x4 v4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < C::kWaves; ++w) acc += s_dq[((w * C::DT + ot) * 4 + e) * 64 + lane];
      v4[e] = (bf16)(acc * p.scale);
    }
    *reinterpret_cast<bf16x4*>(dqrow + 16 * ot + 4 * hq) = v4;
  }
}

using CfgBwdD128 = BwdCfg<128>;
using CfgBwdD64 = BwdCfg<64>;

}  // namespace

bool bwd_mfma_supported(const Params& p) {
  if (p.Dqk != p.Dv || (p.Dqk != 128 && p.Dqk != 64)) return false;
  if (p.G > kMaxGroupB || p.topk > kBwdIdxCap) return false;
  const int64_t kb = 2 * ((int64_t)(p.Skv - 1) * p.k_ss + p.Dqk);
  const int64_t vb = 2 * ((int64_t)(p.Skv - 1) * p.v_ss + p.Dv);
  return kb < (int64_t)kOOB && vb < (int64_t)kOOB && fits_u24(2 * p.k_ss) && fits_u24(2 * p.v_ss);
}

hipError_t launch_bwd_mfma(const Params& p, hipStream_t s) {
  const int64_t n = (int64_t)p.B * p.Sq * p.Hkv * ((p.G + 15) / 16);
  if (p.Dqk == 128 && p.Dv == 128) {
    hipLaunchKernelGGL(bwd_mfma_kernel<CfgBwdD128>, dim3((unsigned)n), dim3(CfgBwdD128::kThreads), 0, s, p);
    return hipGetLastError();
  }
  if (p.Dqk == 64 && p.Dv == 64) {
    hipLaunchKernelGGL(bwd_mfma_kernel<CfgBwdD64>, dim3((unsigned)n), dim3(CfgBwdD64::kThreads), 0, s, p);
    return hipGetLastError();
  }
  return hipErrorNotSupported;
}

}  // namespace sfa

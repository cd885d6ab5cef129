// gfx950 top-k index producer: the step that creates the index rows the
// sparse attention consumes (`topk_idxs`, "Sparse indices mapping queries to
// KV blocks", SFA.py:88-90).  The reference takes them as an input; the
// scores follow DeepSeek-V3.2's lightning indexer:
//
//   I[b,t,s] = sum_h w[b,t,h] * max(0, <q[b,t,h,:], k[b,s,:]>)
//
// over the keys s a query may see (s <= t + L_b - Sq, L_b = kv_lens[b] or
// Skv), then the top-k keys of every query row.  With fp8 (e4m3) q / k, a
// positive per-token scale multiplies each key's score (DeepSeek-V3.2 stores
// the indexer inputs that way, the q scales folded into w).
//
// Two kernels:
//  * indexer_logits_kernel<H, F8>: MFMA with heads as rows and keys as
//    columns (bf16: 32x32x16, fp8: 32x32x64 at twice the rate).  A wave keeps
//    4 M-tiles of q in VGPRs (128 / H queries x H heads, d = 128), the
//    workgroup's 4 waves share each 32-key tile of k, DMA'd into a
//    double-buffered LDS tile (row pitch: the row's 16-byte chunks + 1, so
//    the b128 operand reads are bank-conflict free); the head weights sit in
//    LDS, so two workgroups fit a CU and one's MFMAs cover the other's
//    epilogue and tile wait.  The epilogue applies the weights and the ReLU
//    to the fp32 accumulators and sums over the heads in registers (16 rows
//    per lane, then the lane pair l, l ^ 32), so one coalesced 128-byte store
//    per query writes 32 scores.
//  * topk_select_kernel: one 1024-thread workgroup per query row, the row's
//    scores spread over the threads in contiguous runs of 4, 8, 16, 32 or 64
//    (the smallest that holds the row; one instantiation each) in VGPRs as
//    order-preserving u32 keys.  The k-th largest key is found exactly by
//    bisection over its 32 bits: the top 16 block-wide (per step one compare
//    per score and one block sum; no histogram atomics), the low 16 by one
//    wave over the keys still in play, compacted into LDS.  Then the selected
//    keys are written in ascending key order: all keys above the threshold,
//    and the lowest-index keys equal to it until k are chosen (block scans).

#include "sfa_common.h"
#include "sfa_lds.h"
#include "sfa_mfma.h"

namespace sfa {

namespace {

constexpr int kD = 128;          // index head dim
constexpr int kKT = 32;          // keys per tile
constexpr int kLogitThreads = 256;
constexpr int kLogitSlots = 512;       // resident scores workgroups (two per CU)
constexpr int kLogitTargetWGs = 2048;  // workgroups a split scores launch aims for
constexpr int kLogitMinSpan = 32;      // fewest key tiles (1024 keys) per workgroup
constexpr int kOneQMaxSq = 2;          // queries per sequence up to which the one-query kernel runs
constexpr int kOneQTargetWGs = 16384;   // workgroups a one-query launch aims for
constexpr int kOneQMinSpan = 8;        // fewest key tiles per one-query workgroup (2 per wave)

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Operand geometry of the scores kernel per element type.  bf16: 32x32x16
// MFMA, 8 contraction steps of 16 dims, a key row is 16 chunks of 16 bytes;
// fp8 e4m3: 32x32x64 MFMA (twice the bf16 rate), 2 steps of 64 dims, a key
// row is 8 chunks.  The LDS tile pitch is the row's chunks + 1 (odd, so the
// operand reads of 16 consecutive rows hit distinct banks).
template <bool F8>
struct IdxOps {
  static constexpr int kChunks = F8 ? 8 : 16;       // 16-byte chunks per key row
  static constexpr int kPitch = kChunks + 1;
  static constexpr int kTileSlots = kKT * kPitch;
  static constexpr int kSteps = F8 ? 2 : 8;         // contraction steps over d = 128
  static constexpr int kElem = F8 ? 1 : 2;          // bytes per element
  typedef typename std::conditional<F8, i32x8, bf16x8>::type op_t;
};
constexpr int kSelThreads = 1024;
constexpr int kSelEpt = 64;      // most scores per thread in the selection kernel
constexpr int kSelCap = kSelThreads * kSelEpt;  // longest score row (the API admits Skv <= 65536)
constexpr int kCompact = 4096;   // keys still in play after the top 16 bits that one wave finishes
// segmented selection (launches of fewer than kSegMaxRows rows of at least
// kSegMinKeys keys): up to kSegMax segments per row, about kSegTargetWGs
// phase-1 workgroups
constexpr int kSegMaxRows = 256;
constexpr int kSegMinKeys = 16384;
constexpr int kSegMax = 8;
constexpr int kSegTargetWGs = 256;
static_assert(kSelCap == 65536, "selection capacity");

// Keys query t of sequence b may see: [0, end).
__device__ __forceinline__ int key_end(const IndexerParams& p, int b, int t) {
  int L = p.Skv;
  if (p.kv_lens) L = min(p.kv_lens[b], p.Skv);
  int e = t + 1 + L - p.Sq;
  e = min(e, L);
  return max(e, 0);
}

template <int H, bool F8>
__global__ __launch_bounds__(kLogitThreads, 2) void indexer_logits_kernel(IndexerParams p, int t_begin, int t_end,
                                                                           int nks, int span) {
  constexpr int QPW = 128 / H;        // queries per wave
  constexpr int HT = H / 32;          // M-tiles (32 heads) per query
  constexpr int QB = 4 * QPW;         // queries per workgroup
  static_assert(QPW * HT == 4, "four M-tiles per wave");
  using M = Mfma<32>;
  typedef typename M::acc_t acc_t;
  typedef IdxOps<F8> O;
  typedef typename O::op_t op_t;
  constexpr int kPitch = O::kPitch, kTileSlots = O::kTileSlots;

  // two distinct arrays (not one indexed by parity): the compiler then knows
  // the DMA into one does not feed the operand reads of the other
  __shared__ u32x4 s_k0[kTileSlots];
  __shared__ u32x4 s_k1[kTileSlots];
  // head weights of the workgroup's queries: wave w, M-tile mt, at
  // [(w * 4 + mt) * 32 + head within the tile]
  __shared__ float s_w[4 * 4 * 32];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nqb = (t_end - t_begin + QB - 1) / QB;
  // workgroup -> (sequence, query block, key split): heaviest (latest) query
  // blocks first, the key splits of a block side by side
  const int per_b = nqb * nks;
  const int b = blockIdx.x / per_b;
  const int r = (int)(blockIdx.x % per_b);
  const int qb = nqb - 1 - r / nks;
  const int ks = r % nks;
  const int tq0 = t_begin + qb * QB;  // first query of the workgroup

  // key tiles of the query block: up to the largest end among its queries;
  // this workgroup takes tiles [kt0, kt1) of them
  const int t_last = min(tq0 + QB, t_end) - 1;
  const int kend_wg = key_end(p, b, t_last);
  const int ntiles = (kend_wg + kKT - 1) / kKT;
  const int kt0 = ks * span;
  const int kt1 = min(kt0 + span, ntiles);
  if (kt0 >= kt1) return;  // the whole workgroup, before any barrier

  // ---- q operands (A: lane l holds head 32 hg + l % 32; bf16: dims
  // 16 s + 8 (l / 32) .. + 7, fp8: dims 64 s + 32 (l / 32) .. + 31) and weights
  const int hl = lane & 31, lg = lane >> 5;
  op_t qa[4][O::kSteps];
  float wv[4];  // weights of heads 32 hg + hl (both lane halves load them)
  int tq[QPW];
  bool qok[QPW];
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    tq[i] = tq0 + wave * QPW + i;
    qok[i] = tq[i] < t_end;
  }
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int i = mt / HT, hg = mt % HT;
    const int t = qok[i] ? tq[i] : t_begin;
    const char* qrow = reinterpret_cast<const char*>(p.q) +
                       O::kElem * (b * p.q_sb + t * p.q_ss + (int64_t)(hg * 32 + hl) * p.q_sh);
#pragma unroll
    for (int s = 0; s < O::kSteps; ++s) {
      if constexpr (F8) {
        const u32x4 lo = *reinterpret_cast<const u32x4*>(qrow + 64 * s + 32 * lg);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(qrow + 64 * s + 32 * lg + 16);
        qa[mt][s] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      } else {
        qa[mt][s] = *reinterpret_cast<const bf16x8*>(qrow + 32 * s + 16 * lg);
      }
    }
    const float* wrow = p.w + b * p.w_sb + t * p.w_ss + hg * 32;
    wv[mt] = wrow[hl];
  }
  // weight of accumulator element e of M-tile mt: head 8 (e / 4) + 4 lg + e % 4
  // of the tile, read as 4 consecutive floats per group of 4 elements
  auto wq = [&](int mt, int g4) -> f32x4 {
    return *reinterpret_cast<const f32x4*>(&s_w[(wave * 4 + mt) * 32 + 8 * g4 + 4 * lg]);
  };

  // ---- key tile DMA: slot u = kPitch r + c holds chunk c of key row r (the
  // last chunk of a row is the pad)
  const char* kbase = reinterpret_cast<const char*>(p.k) + O::kElem * (b * p.k_sb);
  const uint32_t krow = (uint32_t)(O::kElem * p.k_ss);
  const __amdgpu_buffer_rsrc_t rk =
      make_rsrc(kbase, (uint32_t)(O::kElem * ((int64_t)(p.Skv - 1) * p.k_ss + kD)));
  auto load_tile = [&](int kt, u32x4* dst) {
#pragma unroll
    for (int it = 0; it < (kTileSlots + kLogitThreads - 1) / kLogitThreads; ++it) {
      const int u = it * kLogitThreads + tid;
      if (u < kTileSlots) {
        const int r = u / kPitch, c = u - r * kPitch;
        const int key = kt * kKT + r;
        const uint32_t off =
            (c < O::kChunks && key < kend_wg) ? __umul24((uint32_t)key, krow) + 16u * (uint32_t)c : kOOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(dst + it * kLogitThreads + wave * 64), 16, off, 0, 0,
                                                 0);
      }
    }
  };

  // per-query row of the logits buffer and its end
  float* orow[QPW];
  int qend[QPW];
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    orow[i] = p.logits + b * p.g_sb + (int64_t)(qok[i] ? tq[i] - p.g_t0 : 0) * p.g_ss;
    qend[i] = qok[i] ? key_end(p, b, tq[i]) : 0;
  }

  // one 32-key tile: 32 MFMAs per wave, then the weighted ReLU sum over the
  // heads and the stores (the other workgroup on the CU runs its MFMAs
  // meanwhile; the next tile's DMA is in flight)
  auto compute = [&](int kt, const u32x4* kt_lds) {
    acc_t acc[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[mt] = acc_t{};
#pragma unroll
    for (int s = 0; s < O::kSteps; ++s) {
      if constexpr (F8) {
        // B operand: key l % 32, dims 64 s + 32 (l / 32) .. = chunks 4 s + 2 (l / 32) + {0, 1}
        const uint32_t a0 = (uint32_t)(hl * kPitch + 4 * s + 2 * lg) * 16u;
        const u32x4 lo = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(kt_lds) + a0);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(kt_lds) + a0 + 16u);
        const i32x8 kb = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
          acc[mt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qa[mt][s], kb, acc[mt], 0, 0, 0, 0, 0, 0);
      } else {
        // B operand: key l % 32, dims 16 s + 8 (l / 32) .. = chunk 2 s + l / 32
        const bf16x8 kb = lds_read_b128(kt_lds, (uint32_t)(hl * kPitch + 2 * s + lg) * 16u);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) acc[mt] = M::mma(qa[mt][s], kb, acc[mt]);
      }
    }
    float sc[QPW];
#pragma unroll
    for (int i = 0; i < QPW; ++i) {
      float x = 0.f;
#pragma unroll
      for (int hg = 0; hg < HT; ++hg) {
        const int mt = i * HT + hg;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const f32x4 w4 = wq(mt, g4);
#pragma unroll
          for (int e = 0; e < 4; ++e) x = fmaf(w4[e], fmaxf(acc[mt][4 * g4 + e], 0.f), x);
        }
      }
      sc[i] = xor32_sum(x);  // lanes l and l ^ 32 hold the two halves of the heads
    }
    // stores: lane half lg writes query i0 + lg (lanes 0-31 only when QPW == 1)
    const int key = kt * kKT + hl;
    if constexpr (F8) {
      // positive per-key scale: k_scale * sum_h w relu(dot) = sum_h w relu(dot * k_scale)
      if (p.k_scale) {
        const float ks = key < p.Skv ? p.k_scale[b * p.ks_sb + key] : 0.f;
#pragma unroll
        for (int i = 0; i < QPW; ++i) sc[i] *= ks;
      }
    }
#pragma unroll
    for (int i0 = 0; i0 < QPW; i0 += 2) {
      float v;
      bool ok;
      int e;
      float* dst;
      if constexpr (QPW == 1) {
        v = sc[0];
        ok = lg == 0 && qok[0];
        e = qend[0];
        dst = orow[0];
      } else {
        v = lg ? sc[i0 + 1] : sc[i0];
        ok = lg ? qok[i0 + 1] : qok[i0];
        e = lg ? qend[i0 + 1] : qend[i0];
        dst = lg ? orow[i0 + 1] : orow[i0];
      }
      if (ok && key < p.Skv) dst[key] = key < e ? v : kNegInf;
    }
  };

  load_tile(kt0, s_k0);
  // the weights go to LDS once tile kt0 is in flight (a load under the lane
  // test would be waited for where issued, before the tile's DMA)
  if (lg == 0) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) s_w[(wave * 4 + mt) * 32 + hl] = wv[mt];
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();                     // tile kt0 and the weights are in place
  for (int kt = kt0; kt < kt1; kt += 2) {
    if (kt + 1 < kt1) load_tile(kt + 1, s_k1);
    compute(kt, s_k0);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // tile kt + 1 has landed
    __syncthreads();                     // and every wave is done with tile kt
    if (kt + 1 < kt1) {
      if (kt + 2 < kt1) load_tile(kt + 2, s_k0);
      compute(kt + 1, s_k1);
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
    }
  }
}

// One query per workgroup (the decode shape: a sequence or two of queries
// per cache, where the 512 / H-query blocks above would compute for empty
// query slots).  The query's H heads are the MFMA rows (H / 32 M-tiles): the
// workgroup copies its q row and head weights into LDS once, and every wave
// streams its own 32-key tiles (tiles kt0 + wave, kt0 + wave + 4, ... of the
// workgroup's split) straight from global memory into B-operand registers,
// NB tiles in flight, taking the q operands from LDS per tile (which keeps
// the kernel at 126 VGPRs, four waves per SIMD, for H = 64).  Operand layout
// as in the block kernel: lane l holds key (B) or head (A) l % 32 and, for
// lane half h = l / 32, bf16 dims 16 s + 8 h .. + 7 at contraction step s
// (fp8: 64 s + 32 h .. + 31), so a load instruction reads 32 contiguous
// bytes of each of 32 key rows.  The epilogue is the block kernel's:
// weighted ReLU over the heads in registers, then the lane pair l, l ^ 32;
// lanes 0-31 store the tile's 32 scores.
template <int H, bool F8, int NB>
__global__ __launch_bounds__(kLogitThreads, 2) void indexer_logits_1q_kernel(IndexerParams p, int t_begin, int t_end,
                                                                              int nks, int span) {
  constexpr int HT = H / 32;  // M-tiles
  using M = Mfma<32>;
  typedef typename M::acc_t acc_t;
  typedef IdxOps<F8> O;
  typedef typename O::op_t op_t;
  __shared__ float s_w[H];
  __shared__ u32x4 s_q[H * O::kPitch];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // workgroup -> (sequence, query, key split)
  const int nq = t_end - t_begin;
  const int per_b = nq * nks;
  const int b = blockIdx.x / per_b;
  const int r = (int)(blockIdx.x % per_b);
  const int t = t_begin + r / nks;
  const int ks = r % nks;
  const int kend = key_end(p, b, t);
  const int ntiles = (kend + kKT - 1) / kKT;
  const int kt0 = ks * span;
  const int kt1 = min(kt0 + span, ntiles);
  if (kt0 >= kt1) return;  // the whole workgroup, before the barrier

  const int hl = lane & 31, lg = lane >> 5;
  // the query's heads into LDS once (row pitch: the row's chunks + 1, so the
  // operand reads of 16 consecutive heads hit distinct banks), the weights
  // beside them; each wave then takes its q operands from there
  const float* wrow = p.w + b * p.w_sb + t * p.w_ss;
  for (int h = tid; h < H; h += kLogitThreads) s_w[h] = wrow[h];
  const char* qbase = reinterpret_cast<const char*>(p.q) + O::kElem * (b * p.q_sb + t * p.q_ss);
  for (int c = tid; c < H * O::kChunks; c += kLogitThreads) {
    const int h = c / O::kChunks, ch = c - h * O::kChunks;
    s_q[h * O::kPitch + ch] = *reinterpret_cast<const u32x4*>(qbase + O::kElem * (int64_t)h * p.q_sh + 16 * ch);
  }
  __syncthreads();  // q and the weights are in place
  // A operand of head 32 mt + l % 32 at step s: bf16 chunk 2 s + lg (dims
  // 16 s + 8 lg ..), fp8 chunks 4 s + 2 lg, + 1 (dims 64 s + 32 lg ..)
  auto qop = [&](int mt, int s) -> op_t {
    const u32x4* qrow = s_q + (mt * 32 + hl) * O::kPitch;
    if constexpr (F8) {
      const u32x4 lo = qrow[4 * s + 2 * lg];
      const u32x4 hi = qrow[4 * s + 2 * lg + 1];
      return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    } else {
      return __builtin_bit_cast(bf16x8, qrow[2 * s + lg]);
    }
  };
  int kt = kt0 + wave;
  if (kt >= kt1) return;  // this wave has no tile (no barrier follows)

  const char* kbase = reinterpret_cast<const char*>(p.k) + O::kElem * (b * p.k_sb);
  const uint32_t krow = (uint32_t)(O::kElem * p.k_ss);
  const __amdgpu_buffer_rsrc_t rk =
      make_rsrc(kbase, (uint32_t)(O::kElem * ((int64_t)(p.Skv - 1) * p.k_ss + kD)));
  float* orow = p.logits + b * p.g_sb + (int64_t)(t - p.g_t0) * p.g_ss;

  // tile i of this wave: kt + 4 i, i < n; the loads are issued without a
  // branch (tiles past the wave's last read nothing: offset kOOB), so the
  // compiler's wait counts stay exact and NB - 1 tiles stay in flight
  const int n = (kt1 - kt + 3) / 4;
  auto load = [&](int i, op_t* kb) {
    const int key = (kt + 4 * i) * kKT + hl;
    const uint32_t base = (i < n && key < kend) ? __umul24((uint32_t)key, krow) + (uint32_t)((F8 ? 32 : 16) * lg) : kOOB;
#pragma unroll
    for (int s = 0; s < O::kSteps; ++s) {
      if constexpr (F8) {
        const i32x4 lo = __builtin_amdgcn_raw_buffer_load_b128(rk, base + 64u * s, 0, 0);
        const i32x4 hi = __builtin_amdgcn_raw_buffer_load_b128(rk, base + 64u * s + 16u, 0, 0);
        kb[s] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      } else {
        kb[s] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, base + 32u * s, 0, 0));
      }
    }
  };
  auto compute = [&](int i, const op_t* kb) {
    acc_t acc[HT];
#pragma unroll
    for (int mt = 0; mt < HT; ++mt) acc[mt] = acc_t{};
#pragma unroll
    for (int s = 0; s < O::kSteps; ++s) {
#pragma unroll
      for (int mt = 0; mt < HT; ++mt) {
        if constexpr (F8)
          acc[mt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qop(mt, s), kb[s], acc[mt], 0, 0, 0, 0, 0, 0);
        else
          acc[mt] = M::mma(qop(mt, s), kb[s], acc[mt]);
      }
    }
    // accumulator element e of M-tile mt: head 32 mt + 8 (e / 4) + 4 lg + e % 4
    float x = 0.f;
#pragma unroll
    for (int mt = 0; mt < HT; ++mt) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const f32x4 w4 = *reinterpret_cast<const f32x4*>(&s_w[mt * 32 + 8 * g4 + 4 * lg]);
#pragma unroll
        for (int e = 0; e < 4; ++e) x = fmaf(w4[e], fmaxf(acc[mt][4 * g4 + e], 0.f), x);
      }
    }
    x = xor32_sum(x);
    const int key = (kt + 4 * i) * kKT + hl;
    if constexpr (F8) {
      if (p.k_scale) x *= key < p.Skv ? p.k_scale[b * p.ks_sb + key] : 0.f;
    }
    if (lg == 0 && key < p.Skv) orow[key] = key < kend ? x : kNegInf;
  };

  // a ring of NB register tiles: tile i + NB - 1 is issued before tile i is used
  op_t kb[NB][O::kSteps];
#pragma unroll
  for (int j = 0; j < NB - 1; ++j) load(j, kb[j]);
  for (int i = 0; i < n; i += NB) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (i + j >= n) break;
      load(i + j + NB - 1, kb[(j + NB - 1) % NB]);
      // keep the next tile's loads ahead of this tile's MFMAs (the scheduler
      // would sink them below and reuse the registers of a pending load)
      __builtin_amdgcn_sched_barrier(0);
      compute(i + j, kb[j]);
    }
  }
}

// Order-preserving map of a float to u32 (larger float -> larger key).
__device__ __forceinline__ uint32_t order_key(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Block-wide sum of one wave-uniform count per wave (kSelThreads threads);
// `red` holds 2 x 16 ints, alternated by the caller's parity so one barrier
// per call suffices.
__device__ __forceinline__ int block_sum_waves(int wave_count, int* red, int parity) {
  const int wave = threadIdx.x >> 6;
  int* r = red + 16 * parity;
  if ((threadIdx.x & 63) == 0) r[wave] = wave_count;
  __syncthreads();
  int s = 0;
#pragma unroll
  for (int w = 0; w < kSelThreads / 64; ++w) s += r[w];
  return s;
}

// Exclusive block scan of one int per thread, and the total.
__device__ __forceinline__ int block_exscan(int x, int* red, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(inc, o, 64);
    if (lane >= o) inc += y;
  }
  __syncthreads();  // earlier readers of red are done
  if (lane == 63) red[wave] = inc;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kSelThreads / 64; ++w) {
    const int v = red[w];
    base += (w < wave) ? v : 0;
    tot += v;
  }
  *total = tot;
  return base + inc - x;
}

// Two exclusive scans at once: (hi, lo) packed as hi 2^16 + lo, valid when
// both block totals stay below 2^16 (rows of at most 32768 scores).
__device__ __forceinline__ void block_exscan2(int hi, int lo, int* red, int* hi_base, int* lo_base, int* hi_total,
                                              int* lo_total) {
  int tot;
  const int base = block_exscan((hi << 16) | lo, red, &tot);
  *hi_base = base >> 16;
  *lo_base = base & 0xFFFF;
  *hi_total = tot >> 16;
  *lo_total = tot & 0xFFFF;
}

// Selection over one row of n > K scores held as NG groups of 4 per thread
// (thread tid owns keys [4 NG tid, 4 NG tid + 4 NG)); NG is fixed per
// instantiation, so the bisection steps are straight-line code.
// Candidate list stride of the segmented selection: topk rounded up to 4
// entries (16 bytes), the tail -1.
__host__ __device__ __forceinline__ int topk_list_stride(int K) { return (K + 3) / 4 * 4; }

// Key sources of select_row: position i of the selection row -> order key
// (4 at a time, i a multiple of 4) and the index written for it.
// A contiguous score row; position i is key base + i.
struct RowSrc {
  static constexpr bool kIds = false;  // ids computed, not loaded
  const float* row;  // scores of positions 0, 1, ... (16-byte aligned)
  int base;
  __device__ __forceinline__ void keys4(int i, uint32_t* k) const {
    const f32x4 x = *reinterpret_cast<const f32x4*>(row + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) k[e] = order_key(x[e]);
  }
  __device__ __forceinline__ int32_t id(int i) const { return base + i; }
};
// A candidate list: position i is key cand[i] with order key ckey[i]
// (cand -1, ckey 0: no candidate, below every real key).  The ids are
// loaded with the keys and kept in registers.
struct CandSrc {
  static constexpr bool kIds = true;
  const int32_t* cand;  // 16-byte aligned
  const uint32_t* ckey;
  __device__ __forceinline__ void keys4(int i, uint32_t* k) const {
    const uint4 c = *reinterpret_cast<const uint4*>(ckey + i);
    k[0] = c.x; k[1] = c.y; k[2] = c.z; k[3] = c.w;
  }
  __device__ __forceinline__ void ids4(int i, int32_t* d) const {
    const int4 c = *reinterpret_cast<const int4*>(cand + i);
    d[0] = c.x; d[1] = c.y; d[2] = c.z; d[3] = c.w;
  }
};

// The K best positions of src (n > K) into out[0, K) in ascending position
// order, and with kout their order keys into kout[0, K).
template <int NG, int MAXR, bool KOUT, class Src>
__device__ __forceinline__ void select_row(const Src& src, int n, int K, int32_t* out, uint32_t* kout, int* red,
                                           uint32_t* s_c) {
  constexpr int EPT = 4 * NG;
  const int tid = threadIdx.x;
  const int i0 = tid * EPT;
  const int cnt = min(max(n - i0, 0), EPT);
  // order keys (0 = absent: every real key is >= order_key(-inf) > 0)
  uint32_t u[EPT];
  int32_t idv[Src::kIds ? EPT : 1];
#pragma unroll
  for (int v = 0; v < NG; ++v) {
    uint32_t k4[4] = {0u, 0u, 0u, 0u};
    if (4 * v < cnt) {
      src.keys4(i0 + 4 * v, k4);
      if constexpr (Src::kIds) src.ids4(i0 + 4 * v, idv + 4 * v);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) u[4 * v + e] = (4 * v + e < cnt) ? k4[e] : 0u;
  }
  // the K-th largest key, bit by bit from the top (a wave counts with
  // ballots: one compare and a scalar popcount per score register; with 64
  // scores per thread the 64 ballot masks would not fit the SGPRs and the
  // compiler spills them into VGPR lanes, so that instance counts per lane
  // and sums the wave once per step)
  uint32_t thr = 0;
  auto block_steps = [&](int hi, int lo) {
#pragma unroll 1
    for (int bit = hi; bit >= lo; --bit) {
      const uint32_t cand = thr | (1u << bit);
      int c = 0;
      if constexpr (EPT >= 64) {
#pragma unroll
        for (int e = 0; e < EPT; ++e) c += u[e] >= cand ? 1 : 0;
        c = __builtin_amdgcn_readfirstlane(wave_sum_int(c));
      } else {
#pragma unroll
        for (int e = 0; e < EPT; ++e) c += __popcll(__ballot(u[e] >= cand));
      }
      if (block_sum_waves(c, red, bit & 1) >= K) thr = cand;
    }
  };
  block_steps(31, 16);
  // Keys whose top 16 bits equal the threshold's are the only ones the low
  // bits still decide ("in play"; typically a few hundred): compact them into
  // LDS and let one wave finish without block barriers.  count(u >= cand)
  // for a candidate with the same top bits = (keys above that prefix) +
  // (in-play keys >= cand).
  {
    const uint32_t top = thr >> 16;
    int above = 0, inplay = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      above += (u[e] >> 16) > top ? 1 : 0;
      inplay += (u[e] >> 16) == top ? 1 : 0;
    }
    int above_total, inplay_total, w;
    if constexpr (NG <= 8) {
      int above_base;
      block_exscan2(above, inplay, red, &above_base, &w, &above_total, &inplay_total);
    } else {
      (void)block_exscan(above, red + 32, &above_total);
      w = block_exscan(inplay, red, &inplay_total);
    }
    if (inplay_total <= kCompact) {
#pragma unroll
      for (int e = 0; e < EPT; ++e)
        if ((u[e] >> 16) == top) s_c[w++] = u[e];
      __syncthreads();
      if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        // up to 64 R in-play keys in registers (absent: 0, below every
        // candidate), counted with ballots like the block steps
        auto finish_regs = [&](auto r_tag) {
          constexpr int R = decltype(r_tag)::value;
          uint32_t kv[R];
#pragma unroll
          for (int i = 0; i < R; ++i) {
            const int j = lane + 64 * i;
            kv[i] = j < inplay_total ? s_c[j] : 0u;
          }
#pragma unroll 1
          for (int bit = 15; bit >= 0; --bit) {
            const uint32_t cand = thr | (1u << bit);
            int c = 0;
#pragma unroll
            for (int i = 0; i < R; ++i) c += __popcll(__ballot(kv[i] >= cand));
            if (above_total + c >= K) thr = cand;
          }
        };
        if (inplay_total <= 64 * 4) {
          finish_regs(std::integral_constant<int, 4>());
        } else if (inplay_total <= 64 * MAXR) {
          finish_regs(std::integral_constant<int, MAXR>());
        } else {
#pragma unroll 1
          for (int bit = 15; bit >= 0; --bit) {
            const uint32_t cand = thr | (1u << bit);
            int c = 0;
            for (int i = lane; i < inplay_total; i += 64) c += s_c[i] >= cand ? 1 : 0;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
            if (above_total + c >= K) thr = cand;
          }
        }
        if (lane == 0) red[80] = (int)thr;
      }
      __syncthreads();
      thr = (uint32_t)red[80];
    } else {
      block_steps(15, 0);
    }
  }
  // keys above the threshold, and the first (lowest-index) ties up to K
  int gt = 0, eq = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    gt += (u[e] > thr) ? 1 : 0;
    eq += (u[e] == thr) ? 1 : 0;
  }
  int gt_total, eq_total, sel_total, eq_before;
  if constexpr (NG <= 8) {
    int gt_base;  // (only the total is used)
    block_exscan2(gt, eq, red, &gt_base, &eq_before, &gt_total, &eq_total);
  } else {
    (void)block_exscan(gt, red + 32, &gt_total);  // (only the total is used)
    eq_before = block_exscan(eq, red, &eq_total);
  }
  const int take = K - gt_total;  // >= 1 ties are selected
  const int my_eq = min(max(take - eq_before, 0), eq);
  int w = block_exscan(gt + my_eq, red + 32, &sel_total);
  int teq = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const bool sel = u[e] > thr || (u[e] == thr && teq < my_eq);
    teq += (u[e] == thr) ? 1 : 0;
    if (sel) {
      if constexpr (Src::kIds)
        out[w] = idv[e];
      else
        out[w] = src.id(i0 + e);
      if constexpr (KOUT) kout[w] = u[e];
      ++w;
    }
  }
}

// MAXNG: the largest row this instance takes is 4 MAXNG kSelThreads scores.
// Rows of up to 32768 scores are held to 64 VGPRs: two workgroups per CU, so
// one workgroup's barrier waits overlap the other's counting.  At that bound
// the compiler spills ~21 VGPRs to scratch; the spill-free build at one
// workgroup per CU (84 VGPRs) was measured 7 % slower on the whole call.
// Selection of the K best of n positions of `src` into out[0, K) (n > K),
// with the smallest run length per thread that holds n.
template <int MAXNG, bool KOUT, class Src>
__device__ __forceinline__ void select_dispatch(const Src& src, int n, int K, int32_t* out, uint32_t* kout, int* red,
                                                uint32_t* s_c) {
  constexpr int MAXR = MAXNG <= 8 ? 8 : 16;  // in-play keys per lane of the register finish
  const int ng = (n + 4 * kSelThreads - 1) / (4 * kSelThreads);
  if (ng <= 1)
    select_row<1, MAXR, KOUT>(src, n, K, out, kout, red, s_c);
  else if (ng <= 2)
    select_row<2, MAXR, KOUT>(src, n, K, out, kout, red, s_c);
  else if (ng <= 4)
    select_row<4, MAXR, KOUT>(src, n, K, out, kout, red, s_c);
  else if (MAXNG <= 8 || ng <= 8)
    select_row<8, MAXR, KOUT>(src, n, K, out, kout, red, s_c);
  else if constexpr (MAXNG > 8)
    select_row<16, MAXR, KOUT>(src, n, K, out, kout, red, s_c);
}

// MAXNG: the largest row this instance takes is 4 MAXNG kSelThreads scores.
// Rows of up to 32768 scores are held to 64 VGPRs: two workgroups per CU, so
// one workgroup's barrier waits overlap the other's counting.  At that bound
// the compiler spills ~21 VGPRs to scratch; the spill-free build at one
// workgroup per CU (84 VGPRs) was measured 7 % slower on the whole call.
template <int MAXNG>
// (second bound: minimum waves per SIMD; 8 = two 16-wave workgroups per CU)
__global__ __launch_bounds__(kSelThreads, MAXNG <= 8 ? 8 : 1) void topk_select_kernel(IndexerParams p, int t_begin,
                                                                                     int t_end) {
  __shared__ int red[96];
  __shared__ uint32_t s_c[kCompact];
  const int nt = t_end - t_begin;
  const int b = blockIdx.x / nt;
  const int t = t_begin + (int)(blockIdx.x % nt);
  const int tid = threadIdx.x;
  const int K = p.topk;
  const int n = __builtin_amdgcn_readfirstlane(key_end(p, b, t));
  int32_t* out = p.idx + b * p.i_sb + t * p.i_ss;

  if (n <= K) {  // every allowed key, ascending, then padding
    for (int i = tid; i < K; i += kSelThreads) out[i] = i < n ? i : -1;
    return;
  }
  const float* row = p.logits + b * p.g_sb + (int64_t)(t - p.g_t0) * p.g_ss;
  select_dispatch<MAXNG, false>(RowSrc{row, 0}, n, K, out, nullptr, red, s_c);
}

// Segmented selection, for launches with few long rows (a decode step: one
// workgroup per row would leave most CUs idle).  Phase 1: workgroup
// (row, s) selects the K best keys of segment s of the row, [s seglen,
// (s + 1) seglen) cut at the row's end, into the row's candidate list
// p.cand[row][s][0, K) in ascending key order (all of a segment's keys when
// it has at most K, then -1).  Phase 2 (topk_merge_kernel): one workgroup per
// row selects the K best of the row's nseg K candidates.  The union of the
// segments' selections holds the row's selection, ties included: a segment
// with at least K keys at or above the row's threshold would put K keys above
// it; so a segment's local threshold is at most the row's, and it keeps
// every key above the row's threshold and at least as many of its lowest
// equal keys as the row takes.  The candidates are in ascending key order
// (segment by segment), so the merge's equal-score rule (lower position
// first) is the row's (lower key first).
// (4 waves per SIMD: about 256 workgroups, one per CU)
__global__ __launch_bounds__(kSelThreads, 4) void topk_segment_kernel(IndexerParams p, int t_begin, int t_end) {
  __shared__ int red[96];
  __shared__ uint32_t s_c[kCompact];
  const int nt = t_end - t_begin;
  const int rowi = blockIdx.x / p.nseg;
  const int seg = (int)(blockIdx.x % p.nseg);
  const int b = rowi / nt;
  const int t = t_begin + rowi % nt;
  const int tid = threadIdx.x;
  const int K = p.topk;
  const int kpad = topk_list_stride(K);
  const int n = __builtin_amdgcn_readfirstlane(key_end(p, b, t));
  int32_t* out = p.cand + (int64_t)blockIdx.x * kpad;
  uint32_t* kout = p.cand_key + (int64_t)blockIdx.x * kpad;
  const int s0 = seg * p.seglen;
  const int ns = min(max(n - s0, 0), p.seglen);
  const float* row = p.logits + b * p.g_sb + (int64_t)(t - p.g_t0) * p.g_ss;
  if (ns <= K) {
    for (int i = tid; i < kpad; i += kSelThreads) {
      out[i] = i < ns ? s0 + i : -1;
      kout[i] = i < ns ? order_key(row[s0 + i]) : 0u;
    }
    return;
  }
  if (tid < kpad - K) {
    out[K + tid] = -1;
    kout[K + tid] = 0u;
  }
  select_dispatch<8, true>(RowSrc{row + s0, s0}, ns, K, out, kout, red, s_c);
}

// (4 waves per SIMD: one merge workgroup per row, few rows; the candidate
// gathers need more than the 64 VGPRs of two workgroups per CU)
__global__ __launch_bounds__(kSelThreads, 4) void topk_merge_kernel(IndexerParams p, int t_begin, int t_end) {
  __shared__ int red[96];
  __shared__ uint32_t s_c[kCompact];
  const int nt = t_end - t_begin;
  const int b = blockIdx.x / nt;
  const int t = t_begin + (int)(blockIdx.x % nt);
  const int tid = threadIdx.x;
  const int K = p.topk;
  const int n = __builtin_amdgcn_readfirstlane(key_end(p, b, t));
  int32_t* out = p.idx + b * p.i_sb + t * p.i_ss;
  if (n <= K) {
    for (int i = tid; i < K; i += kSelThreads) out[i] = i < n ? i : -1;
    return;
  }
  const int kpad = topk_list_stride(K);
  const int64_t c0 = (int64_t)blockIdx.x * p.nseg * kpad;
  select_dispatch<8, false>(CandSrc{p.cand + c0, p.cand_key + c0}, p.nseg * kpad, K, out, nullptr, red, s_c);
}

}  // namespace

int indexer_query_block(const IndexerParams& p) { return 4 * (128 / p.H); }

namespace {

// One-query scores launch: B x (t_end - t_begin) queries, each query's key
// tiles split over workgroups of at least kOneQMinSpan tiles (4 per wave) so
// that the launch holds about kOneQTargetWGs workgroups.
template <int H, bool F8>
hipError_t launch_logits_1q(const IndexerParams& p, int t_begin, int t_end, int ntiles_max, hipStream_t s) {
  constexpr int NB = 2;  // register tiles in flight per wave
  const int64_t nqry = (int64_t)p.B * (t_end - t_begin);
  int nks = 1;
  if (nqry < kOneQTargetWGs && ntiles_max > kOneQMinSpan) {
    const int64_t want = (kOneQTargetWGs + nqry - 1) / nqry;
    nks = (int)std::min<int64_t>(want, (ntiles_max + kOneQMinSpan - 1) / kOneQMinSpan);
  }
  const int span = std::max(1, (ntiles_max + nks - 1) / nks);
  hipLaunchKernelGGL((indexer_logits_1q_kernel<H, F8, NB>), dim3((unsigned)(nqry * nks)), dim3(kLogitThreads), 0, s,
                     p, t_begin, t_end, nks, span);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_indexer_logits(const IndexerParams& p, int t_begin, int t_end, hipStream_t s) {
  if (t_end <= t_begin || p.B == 0) return hipSuccess;
  if (p.Sq <= kOneQMaxSq) {
    const int kend_max = std::max(0, std::min(t_end + p.Skv - p.Sq, p.Skv));
    const int ntiles_max = (kend_max + kKT - 1) / kKT;
    if (p.fp8) {
      if (p.H == 64) return launch_logits_1q<64, true>(p, t_begin, t_end, ntiles_max, s);
      if (p.H == 32) return launch_logits_1q<32, true>(p, t_begin, t_end, ntiles_max, s);
      if (p.H == 128) return launch_logits_1q<128, true>(p, t_begin, t_end, ntiles_max, s);
    } else {
      if (p.H == 64) return launch_logits_1q<64, false>(p, t_begin, t_end, ntiles_max, s);
      if (p.H == 32) return launch_logits_1q<32, false>(p, t_begin, t_end, ntiles_max, s);
      if (p.H == 128) return launch_logits_1q<128, false>(p, t_begin, t_end, ntiles_max, s);
    }
    return hipErrorNotSupported;
  }
  const int qb = indexer_query_block(p);
  const int64_t nblk = (int64_t)p.B * ((t_end - t_begin + qb - 1) / qb);
  if (nblk == 0) return hipSuccess;
  // Key splits, for launches with fewer query blocks than workgroup slots (a
  // decode step: one query per sequence): a query block's key tiles are
  // shared by nks workgroups of span tiles each, so that the launch holds
  // about kLogitTargetWGs workgroups.  A split holds at least kLogitMinSpan
  // tiles.  Launches with more query blocks than slots are not split: every
  // split re-reads its block's q (128 KB for 64 heads) from HBM, which cost
  // more on the S = 32768 prefill than the balance it bought.
  const int kend_max = std::max(0, std::min(t_end + p.Skv - p.Sq, p.Skv));  // key_end of the last query, L = Skv
  const int ntiles_max = (kend_max + kKT - 1) / kKT;
  int nks = 1;
  if (nblk < kLogitSlots && ntiles_max > kLogitMinSpan) {
    const int64_t want = (kLogitTargetWGs + nblk - 1) / nblk;
    nks = (int)std::min<int64_t>(want, (ntiles_max + kLogitMinSpan - 1) / kLogitMinSpan);
  }
  const int span = std::max(1, (ntiles_max + nks - 1) / nks);
  const dim3 g((unsigned)(nblk * nks)), blk(kLogitThreads);
  if (p.fp8) {
    if (p.H == 64)
      hipLaunchKernelGGL((indexer_logits_kernel<64, true>), g, blk, 0, s, p, t_begin, t_end, nks, span);
    else if (p.H == 32)
      hipLaunchKernelGGL((indexer_logits_kernel<32, true>), g, blk, 0, s, p, t_begin, t_end, nks, span);
    else if (p.H == 128)
      hipLaunchKernelGGL((indexer_logits_kernel<128, true>), g, blk, 0, s, p, t_begin, t_end, nks, span);
    else
      return hipErrorNotSupported;
  } else {
    if (p.H == 64)
      hipLaunchKernelGGL((indexer_logits_kernel<64, false>), g, blk, 0, s, p, t_begin, t_end, nks, span);
    else if (p.H == 32)
      hipLaunchKernelGGL((indexer_logits_kernel<32, false>), g, blk, 0, s, p, t_begin, t_end, nks, span);
    else if (p.H == 128)
      hipLaunchKernelGGL((indexer_logits_kernel<128, false>), g, blk, 0, s, p, t_begin, t_end, nks, span);
    else
      return hipErrorNotSupported;
  }
  return hipGetLastError();
}

int topk_segments(const IndexerParams& p, int rows) {
  const int64_t nrow = (int64_t)p.B * rows;
  if (nrow <= 0 || nrow >= kSegMaxRows || p.Skv < kSegMinKeys) return 1;
  int nseg = (int)std::min<int64_t>(kSegMax, std::max<int64_t>(2, (kSegTargetWGs + nrow - 1) / nrow));
  // the candidates fill one merge row of at most 32768 (two workgroups per
  // CU), and a segment must be longer than K to cut anything
  while (nseg > 1 &&
         ((int64_t)nseg * topk_list_stride(p.topk) > 4 * 8 * kSelThreads || topk_seglen(p, nseg) <= p.topk))
    --nseg;
  return nseg;
}

int topk_seglen(const IndexerParams& p, int nseg) { return ((p.Skv + nseg - 1) / nseg + 31) / 32 * 32; }

hipError_t launch_topk_select(const IndexerParams& p, int t_begin, int t_end, hipStream_t s) {
  const int64_t n = (int64_t)p.B * (t_end - t_begin);
  if (n == 0) return hipSuccess;
  if (p.nseg > 1) {
    if (p.cand == nullptr || p.cand_key == nullptr || p.seglen <= 0 || p.seglen % 4 != 0 || (int64_t)p.seglen * p.nseg < p.Skv ||
        p.seglen > 4 * 8 * kSelThreads || (int64_t)p.nseg * topk_list_stride(p.topk) > 4 * 8 * kSelThreads)
      return hipErrorInvalidValue;
    // (Skv <= 65536 and at least 2 segments: a segment holds at most 32768)
    hipLaunchKernelGGL(topk_segment_kernel, dim3((unsigned)(n * p.nseg)), dim3(kSelThreads), 0, s, p, t_begin, t_end);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(topk_merge_kernel, dim3((unsigned)n), dim3(kSelThreads), 0, s, p, t_begin, t_end);
    return hipGetLastError();
  }
  // a row holds at most Skv scores
  if (p.Skv <= 4 * 8 * kSelThreads)
    hipLaunchKernelGGL(topk_select_kernel<8>, dim3((unsigned)n), dim3(kSelThreads), 0, s, p, t_begin, t_end);
  else
    hipLaunchKernelGGL(topk_select_kernel<16>, dim3((unsigned)n), dim3(kSelThreads), 0, s, p, t_begin, t_end);
  return hipGetLastError();
}

}  // namespace sfa

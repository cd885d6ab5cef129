// Index-row sort ahead of the persistent MLA prefill forward.
//
// The forward's result depends on the order of a row's slots only through
// the order of its floating-point sums (the reference, SFA.py:386-467, walks
// the slots in row order; any order gives the same softmax).  Walking the
// keys in ascending order is what makes the gathers share the L2: the
// persistent forward runs runs of consecutive queries together on one XCD,
// their rows select keys from nearly the same causal prefix, and with
// ascending rows they reach each region of that prefix at about the same
// time, so a row one workgroup gathered is often still in the XCD's L2 when
// the others reach it (MLA prefill, S = 32768, top-k 2048: about 2 % less
// kernel time).  sfa_fwd runs this pass unless the caller declares its rows
// ascending (SFA_FWD_IDX_SORTED), e.g. for rows of sfa_indexer_topk.
//
// One workgroup per index row at a time: the valid keys (0 <= key < bound,
// the forward's own rule) set bits of an LDS bitmap of the row's key range; a
// prefix count per bitmap word then gives every valid slot its rank among the
// row's keys (set bits of the lower words plus those below it in its word),
// the slot's key is written at that rank, and the slots after the last rank
// get -1.  Every thread ranks its own slots, so no thread loops over bits.  A
// row that selects some key twice (the forward counts every slot, so a
// repeated key contributes twice) is written back unchanged.  Each workgroup
// takes rows blockIdx.x, blockIdx.x + gridDim.x, ... and loads the next row's
// ids while it sorts the current one.

#include "sfa_common.h"

namespace sfa {
namespace {

constexpr int kSortMaxTopk = 2048;
constexpr int kSortThreads = 256;
constexpr int kSortPer = kSortMaxTopk / kSortThreads;  // slots per thread

// inclusive prefix sum over the 64 lanes of a wave
__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  return x;
}

// The ids of row r by buffer loads over its topk slots (slots past topk read
// 0; the users test the slot index), so the loads need no branches.
__device__ __forceinline__ void load_row(const Params& p, int r, int (&keys)[kSortPer], int tid) {
  const int g = r % p.Hkv;
  const int bt = r / p.Hkv;
  const int t = bt % p.Sq;
  const int b = bt / p.Sq;
  const int32_t* row = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(row, 4u * (uint32_t)p.topk);
#pragma unroll
  for (int j = 0; j < kSortPer; ++j)
    keys[j] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs, 4u * (uint32_t)(j * kSortThreads + tid), 0, 0);
}

// Workgroup barrier over LDS only: waits for this wave's LDS operations, not
// for its global loads and stores (the next row's loads and this row's
// stores stay in flight, which __syncthreads would wait for).
#define SORT_LDS_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

// NW: bitmap words, keys < 32 NW.
template <int NW>
__global__ __launch_bounds__(kSortThreads) void idx_sort_kernel(Params p, int32_t* __restrict__ out, int rows) {
  constexpr int WPT = NW / kSortThreads;  // bitmap words per thread in the prefix count
  static_assert(WPT == 4 || WPT == 8, "16-byte bitmap reads");
  __shared__ uint32_t bm[NW];
  __shared__ uint32_t pre[NW];  // set bits in the words before word w
  __shared__ int32_t srt[kSortMaxTopk];
  __shared__ int wsum[2][kSortThreads / 64];  // per wave: distinct keys, valid slots
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int keys[kSortPer];
  int r = blockIdx.x;
  if (r < rows) load_row(p, r, keys, tid);
  for (; r < rows; r += gridDim.x) {
    int cur[kSortPer];
#pragma unroll
    for (int j = 0; j < kSortPer; ++j) cur[j] = j * kSortThreads + tid < p.topk ? keys[j] : -1;
    if (r + (int)gridDim.x < rows) load_row(p, r + gridDim.x, keys, tid);
    const int b = r / (p.Hkv * p.Sq);
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(out + (int64_t)r * p.topk, 4u * (uint32_t)p.topk);
    const int bound = bound_of(p, b);
    const int nw = bound > 0 ? (bound + 31) >> 5 : 0;  // <= NW (the host checks Skv <= 32 NW)

    for (int w = tid; w < nw; w += kSortThreads) bm[w] = 0u;
    SORT_LDS_BARRIER();
    int nvalid = 0;
#pragma unroll
    for (int j = 0; j < kSortPer; ++j) {
      const int k = cur[j];
      if (k >= 0 && k < bound) {
        atomicOr(&bm[k >> 5], 1u << (k & 31));
        ++nvalid;
      }
    }
    SORT_LDS_BARRIER();
    // prefix counts: thread i sums its words [i WPT, (i + 1) WPT); a wave scan
    // and the lower waves' totals place them after every lower word
    uint32_t wd[WPT], loc[WPT];
    {
      const u32x4* b4 = reinterpret_cast<const u32x4*>(bm) + tid * (WPT / 4);
#pragma unroll
      for (int q = 0; q < WPT / 4; ++q) {
        const u32x4 x = b4[q];
        wd[4 * q] = x[0];
        wd[4 * q + 1] = x[1];
        wd[4 * q + 2] = x[2];
        wd[4 * q + 3] = x[3];
      }
    }
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
      loc[j] = (uint32_t)cnt;
      cnt += tid * WPT + j < nw ? __popc(wd[j]) : 0;
    }
    const int incl = wave_incl_scan(cnt, lane);
    const int vincl = wave_incl_scan(nvalid, lane);
    if (lane == 63) {
      wsum[0][wave] = incl;
      wsum[1][wave] = vincl;
    }
    SORT_LDS_BARRIER();
    int below = 0, total = 0, slots = 0;
#pragma unroll
    for (int w = 0; w < kSortThreads / 64; ++w) {
      const int x = wsum[0][w];
      below += w < wave ? x : 0;
      total += x;   // distinct valid keys
      slots += wsum[1][w];  // slots naming a valid key
    }
    const uint32_t excl = (uint32_t)(below + incl - cnt);
    // fewer distinct keys than valid slots: the row repeats a key
    const bool repeats = slots != total;
    if (!repeats) {
#pragma unroll
      for (int j = 0; j < WPT; ++j) pre[tid * WPT + j] = excl + loc[j];
      SORT_LDS_BARRIER();
#pragma unroll
      for (int j = 0; j < kSortPer; ++j) {
        const int k = cur[j];
        if (k >= 0 && k < bound) {
          const int w = k >> 5;
          srt[pre[w] + __popc(bm[w] & ((1u << (k & 31)) - 1u))] = k;
        }
      }
      SORT_LDS_BARRIER();
    }
    // (slots past topk: out-of-range offsets, the stores are dropped)
#pragma unroll
    for (int j = 0; j < kSortPer; ++j) {
      const int i = j * kSortThreads + tid;
      const int v = repeats ? cur[j] : (i < total ? srt[i] : -1);
      __builtin_amdgcn_raw_buffer_store_b32(v, ro, 4u * (uint32_t)i, 0, 0);
    }
    // (the next row's bitmap clear and wsum writes wait for every read here)
    SORT_LDS_BARRIER();
  }
}

}  // namespace

bool idx_sort_supported(const Params& p) { return p.topk <= kSortMaxTopk && p.Skv <= 32 * 2048; }

hipError_t launch_idx_sort(const Params& p, int32_t* out, hipStream_t s) {
  const int64_t rows = (int64_t)p.B * p.Sq * p.Hkv;
  if (!idx_sort_supported(p) || rows <= 0 || rows > INT32_MAX) return hipErrorInvalidValue;
  if ((int64_t)p.Sq * p.Hkv > INT32_MAX) return hipErrorInvalidValue;
  // 8 workgroups per CU (16 or 24 KB of LDS each), rows / 2048 rows each
  const unsigned grid = (unsigned)(rows < 2048 ? rows : 2048);
  if (p.Skv <= 32 * 1024)
    hipLaunchKernelGGL(idx_sort_kernel<1024>, dim3(grid), dim3(kSortThreads), 0, s, p, out, (int)rows);
  else
    hipLaunchKernelGGL(idx_sort_kernel<2048>, dim3(grid), dim3(kSortThreads), 0, s, p, out, (int)rows);
  return hipGetLastError();
}

}  // namespace sfa

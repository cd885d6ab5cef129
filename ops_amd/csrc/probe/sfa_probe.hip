// Measurement-only kernels (ops_amd/libsfa_probe.so; not part of libsfa.so
// and not behind include/sfa.h): what the split-k MLA decode's data movement
// costs on its own, without its MFMA work, so the floors of the work layouts
// the decode design compares can be measured from committed code
// (`python bench.py --probe decode_gather`).
//
// One launch gathers every valid top-k row of a [B][topk] index set (the
// decode: B sequences, one query each, a 576-dim bf16 latent row per key)
// exactly as fwd_mfma_kernel does -- the library's RowGather, 32-row
// swizzled tiles, buffer_load_dwordx4 ... lds, the next tile in flight while
// the current one is waited for, one workgroup barrier per tile -- in a
// layout of `splits` key splits x `hgroups` head groups per sequence (each
// workgroup gathers its split's rows; every head group of a split gathers
// them again).  Optional pieces of the real kernel's data movement:
//  * q_bytes: the workgroup first loads that many bytes of the sequence's Q
//    rows into LDS (the decode kernel loads its 128 heads x 576 dims, half
//    into LDS, half into registers);
//  * store_rows: after its last tile the workgroup writes that many 1 KB rows
//    (the bf16 partial O rows of its heads) to `part`.
// Nothing is computed; the tiles are overwritten in place.

#include "../sfa_common.h"
#include "../sfa_lds.h"

namespace sfa {
namespace {

constexpr int kPT = 32;             // rows per tile
constexpr int kPCH = 72;            // 16-byte chunks per 1152-byte row
constexpr int kPThreads = 256;      // 4 waves
constexpr int kPIdxCap = 2048;      // slots one workgroup stages
typedef RowGather<kPT, kPCH, 4, true, BufRows> PRG;

struct ProbeArgs {
  const void* kv;       // [B][Skv][576] bf16
  const void* q;        // [B][q_row_bytes] (only q_bytes of it are read)
  const int32_t* idx;   // [B][topk]
  void* part;           // [B * splits * hgroups][store_rows][1024 bytes]
  int B, Skv, topk, splits, hgroups, q_bytes, store_rows;
  int64_t q_row_bytes;
};

__global__ __launch_bounds__(kPThreads, 1) void probe_gather_kernel(ProbeArgs a) {
  __shared__ int s_idx[kPIdxCap];
  __shared__ u32x4 s_t[2][kPT * kPCH];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // workgroup -> (sequence, split, head group); the pieces of one sequence
  // run on one XCD (workgroup w goes to XCD w % 8), as in the decode kernel
  const int per = a.splits * a.hgroups;
  int vb = blockIdx.x, b, piece;
  if (a.B % 8 == 0) {
    const int x = vb % 8, r = vb / 8;
    piece = r % per;
    b = (r / per) * 8 + x;
  } else {
    piece = vb % per;
    b = vb / per;
  }
  const int split = piece % a.splits;
  const int len = (a.topk + a.splits - 1) / a.splits;
  const int s0 = split * len;
  const int nslots = max(0, min(a.topk - s0, len));
  // Q rows into LDS first (16-byte DMA per lane, into the tile buffers)
  if (a.q_bytes > 0) {
    const char* qb = reinterpret_cast<const char*>(a.q) + (int64_t)b * a.q_row_bytes;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(qb, (uint32_t)a.q_bytes);
    u32x4* dst = &s_t[0][0];
    constexpr int kSlots = 2 * kPT * kPCH;  // the two tile buffers
    for (int c = wave * 64; c * 16 < a.q_bytes; c += kPThreads) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void*)(dst + (c % kSlots)), 16, 16u * (uint32_t)(c + lane), 0,
                                               0, 0);
    }
  }
  // the split's index row, staged (slots past it: -1)
  const int32_t* irow = a.idx + (int64_t)b * a.topk + s0;
  for (int i = tid; i < kPIdxCap; i += kPThreads) s_idx[i] = i < nslots ? irow[i] : -1;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  BufRows src;
  src.rs = make_rsrc(reinterpret_cast<const char*>(a.kv) + (int64_t)b * a.Skv * 1152, (uint32_t)a.Skv * 1152u);
  src.row_bytes = 1152u;
  const int ntiles = (nslots + kPT - 1) / kPT;
  PRG rg;
  if (ntiles > 0) {
    rg.load_ids(s_idx, true, wave, src);
#pragma unroll
    for (int k = 0; k < PRG::NI; ++k) rg.issue(k, src, s_t[0], wave, lane);
  }
  for (int t = 0; t < ntiles; ++t) {
    if (t + 1 < ntiles) {
      rg.load_ids(s_idx + (t + 1) * kPT, true, wave, src);
#pragma unroll
      for (int k = 0; k < PRG::NI; ++k) rg.issue(k, src, s_t[(t + 1) & 1], wave, lane);
      // tile t landed; tile t + 1 still in flight
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PRG::NI) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
  }
  // the partial rows: 1 KB each, 16 bytes per lane, one row per instruction
  if (a.store_rows > 0) {
    u32x4* prow = reinterpret_cast<u32x4*>(a.part) + (int64_t)blockIdx.x * a.store_rows * 64;
    const u32x4* sv = &s_t[0][0];
    for (int r = wave; r < a.store_rows; r += 4) prow[(int64_t)r * 64 + lane] = sv[(r * 64 + lane) % (kPT * kPCH)];
  }
}

// The ceiling of the same rows' data movement: every valid row of the
// [B][topk] index set read once, 16 bytes per lane into registers (no LDS,
// no tiles, no barriers), with as many independent loads in flight as the
// grid allows: thread i of the grid takes 16-byte chunks i, i + nthreads,
// ... of the flattened list of (row, chunk) pairs, U at a time (the U index
// loads first, then the U row loads).  contiguous = 1 reads the same number
// of bytes from the start of the KV buffer instead (the streaming
// reference).  Each thread folds what it read into one word it writes to
// `sink`, so no load is dead.
template <int U>
__global__ __launch_bounds__(256) void probe_rowread_kernel(const u32x4* __restrict__ kv, const int32_t* __restrict__ idx,
                                                            uint32_t* __restrict__ sink, int B, int Skv, int topk,
                                                            int64_t nchunks, int contiguous) {
  constexpr int kCPR = 72;  // 16-byte chunks per 1152-byte row
  const int64_t nth = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (int64_t c0 = tid; c0 < nchunks; c0 += nth * U) {
    int64_t off[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + (int64_t)u * nth;
      if (contiguous) {
        off[u] = c < nchunks ? c : -1;
      } else {
        const int64_t r = c / kCPR;  // (sequence, slot) pair
        const int ch = (int)(c - r * kCPR);
        const int b = (int)(r / topk);
        const int key = c < nchunks ? idx[r] : -1;
        off[u] = key >= 0 && key < Skv ? ((int64_t)b * Skv + key) * kCPR + ch : -1;
      }
    }
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = off[u] >= 0 ? kv[off[u]] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  sink[tid] = acc;
}

}  // namespace
}  // namespace sfa

extern "C" {

// Launches probe_gather_kernel on `stream`: B * splits * hgroups workgroups.
// Returns 0, or -1 for arguments outside its limits (a split longer than the
// 2048 staged slots, a KV slice of 2 GiB or more), or the HIP error code of
// the launch.  (Q loads wrap around the two tile buffers: any q_bytes.)
__attribute__((visibility("default"))) int sfa_probe_gather(const void* kv, const void* q, int64_t q_row_bytes,
                                                            const int32_t* idx, void* part, int B, int Skv, int topk,
                                                            int splits, int hgroups, int q_bytes, int store_rows,
                                                            void* stream) {
  if (B <= 0 || Skv <= 0 || topk <= 0 || splits <= 0 || hgroups <= 0 || q_bytes < 0 || store_rows < 0) return -1;
  if ((topk + splits - 1) / splits > sfa::kPIdxCap) return -1;
  if (q_bytes > 0 && (q == nullptr || q_row_bytes < q_bytes)) return -1;
  if (store_rows > 0 && part == nullptr) return -1;
  if ((int64_t)Skv * 1152 >= ((int64_t)1 << 31)) return -1;
  sfa::ProbeArgs a{kv, q, idx, part, B, Skv, topk, splits, hgroups, q_bytes, store_rows, q_row_bytes};
  const unsigned grid = (unsigned)((int64_t)B * splits * hgroups);
  hipLaunchKernelGGL(sfa::probe_gather_kernel, dim3(grid), dim3(sfa::kPThreads), 0, (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

// Launches probe_rowread_kernel<8> on `stream`: `workgroups` x 256 threads
// read every valid row of idx ([B][topk]; a slot is valid iff 0 <= id < Skv,
// rows in order of the compacted list `rows` = the number of (b, slot) pairs
// to read, i.e. idx is read as a flat list of `rows` ids whose batch is
// position / topk) -- or, with contiguous, the same bytes from the start of
// kv.  sink: workgroups * 256 words.  Returns 0, -1 for bad arguments, or
// the HIP error of the launch.
__attribute__((visibility("default"))) int sfa_probe_rowread(const void* kv, const int32_t* idx, void* sink, int B,
                                                             int Skv, int topk, int workgroups, int contiguous,
                                                             void* stream) {
  if (kv == nullptr || sink == nullptr || B <= 0 || Skv <= 0 || topk <= 0 || workgroups <= 0) return -1;
  if (!contiguous && idx == nullptr) return -1;
  if (contiguous && topk > Skv) return -1;  // the contiguous bytes must lie in kv
  const int64_t nchunks = (int64_t)B * topk * 72;
  hipLaunchKernelGGL(sfa::probe_rowread_kernel<8>, dim3((unsigned)workgroups), dim3(256), 0, (hipStream_t)stream,
                     (const sfa::u32x4*)kv, idx, (uint32_t*)sink, B, Skv, topk, nchunks, contiguous);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

}  // extern "C"

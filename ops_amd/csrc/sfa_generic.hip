// Generic sparse flash attention kernels for any head dim / group size, in
// float32 or bfloat16.  They are the float32 path (the tiny fp32 workload) and
// the path for shapes the MFMA kernels do not cover.  One workgroup of 256
// threads (4 waves) owns one (batch, query, head) row; a wave evaluates one
// top-k slot at a time with a coalesced dot product over the feature dim.
//
// Math (reference SFA.py):  s = scale·<q, k[idx]>, masked to valid slots
// (SFA.py:392-404, 436); lse = log Σ exp(s) (+ exp(sink), SFA.py:469-474);
// out = Σ exp(s - lse)·v[idx] (SFA.py:441-480).  Backward: δ = Σ out·dout
// (SFA.py:590-610); dS = P(dP - δ); dq = scale·Σ dS·k (SFA.py:649-716);
// dk[idx] += scale·dS·q, dv[idx] += P·dout (SFA.py:757-853, fp32 atomics as
// SFA.py:853); dsink = -Σ exp(sink - lse)·δ (SFA.py:964-970), reduced per head in
// a fixed order by dsink_kernel.

#include "sfa_common.h"

namespace sfa {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ float block_reduce_max(float x, float* red) {
  x = wave_max(x);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = x;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) r = fmaxf(r, red[i]);
  return r;
}

__device__ __forceinline__ float block_reduce_sum(float x, float* red) {
  x = wave_sum(x);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = x;
  __syncthreads();
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r += red[i];
  return r;
}

// Shared memory: q row [Dqk] | per-slot score / probability [topk] | reduce [kWaves]
template <typename T>
__global__ __launch_bounds__(kThreads) void fwd_generic_kernel(Params p) {
  extern __shared__ float smem[];
  float* qs = smem;
  float* sc = smem + p.Dqk;
  float* red = sc + p.topk;

  const int row = blockIdx.x;  // (b, t, h) flattened as ((b*Sq)+t)*Hq+h
  const int h = row % p.Hq;
  const int t = (row / p.Hq) % p.Sq;
  const int b = row / (p.Hq * p.Sq);
  const int g = h / p.G;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  const T* qrow = reinterpret_cast<const T*>(p.q) + b * p.q_sb + t * p.q_ss + h * p.q_sh;
  for (int d = tid; d < p.Dqk; d += kThreads) qs[d] = to_f32(qrow[d]);
  __syncthreads();

  const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh;
  const int bound = bound_of(p, b);
  // paged KV: k / v are pools and the slot's pool row comes from the block
  // table (-1 for an invalid slot or an unmapped page)
  const bool paged = p.block_table != nullptr;
  const T* kb = reinterpret_cast<const T*>(p.k) + (paged ? 0 : b * p.k_sb) + g * p.k_sh;
  const T* vb = reinterpret_cast<const T*>(p.v) + (paged ? 0 : b * p.v_sb) + g * p.v_sh;
  const int pmask = (1 << p.page_shift) - 1;
  auto key_row = [&](const T* base, int id, int64_t sb, int64_t ss) -> const T* {
    if (paged) {
      const int r = paged_row(p, b, id, bound);
      return r < 0 ? nullptr : base + (int64_t)(r >> p.page_shift) * sb + (int64_t)(r & pmask) * ss;
    }
    return (id >= 0 && id < bound) ? base + (int64_t)id * ss : nullptr;
  };

  for (int j = wave; j < p.topk; j += kWaves) {
    const T* kr = key_row(kb, irow[j], p.k_sb, p.k_ss);
    float s = kNegInf;
    if (kr != nullptr) {
      float acc = 0.f;
      for (int d = lane; d < p.Dqk; d += 64) acc += qs[d] * to_f32(kr[d]);
      s = wave_sum(acc) * p.scale_log2;
    }
    if (lane == 0) sc[j] = s;
  }
  __syncthreads();

  float m = kNegInf;
  for (int j = tid; j < p.topk; j += kThreads) m = fmaxf(m, sc[j]);
  m = block_reduce_max(m, red);
  const float sink2 = p.sink ? p.sink[h] * kLog2e : kNegInf;
  const float mm = fmaxf(m, sink2);

  float l = 0.f;
  for (int j = tid; j < p.topk; j += kThreads) {
    const float s = sc[j];
    const float e = (s == kNegInf) ? 0.f : exp2f(s - mm);
    sc[j] = e;
    l += e;
  }
  l = block_reduce_sum(l, red);  // contains the barrier that publishes sc[]
  if (p.sink && mm != kNegInf) l += exp2f(sink2 - mm);
  const float inv = l > 0.f ? 1.f / l : 0.f;

  T* orow = reinterpret_cast<T*>(p.out) + b * p.o_sb + t * p.o_ss + h * p.o_sh;
  for (int d = tid; d < p.Dv; d += kThreads) {
    float acc = 0.f;
    for (int j = 0; j < p.topk; ++j) {
      const float e = sc[j];
      if (e != 0.f) acc += e * to_f32(key_row(vb, irow[j], p.v_sb, p.v_ss)[d]);
    }
    orow[d] = from_f32<T>(acc * inv);
  }
  if (tid == 0) {
    p.lse[b * p.l_sb + t * p.l_ss + h * p.l_sh] = (l > 0.f) ? (mm + log2f(l)) * kLn2 : kNegInf;
  }
}

// δ = Σ_d out·dout per (b, t, h) row (SFA.py:590-610), minus dlse when a
// gradient reaches the returned lse.  One wave per row.
template <typename T>
__global__ __launch_bounds__(kThreads) void delta_kernel(Params p) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + wave;
  const int64_t nrows = (int64_t)p.B * p.Sq * p.Hq;
  if (row >= nrows) return;
  const int h = row % p.Hq;
  const int t = (row / p.Hq) % p.Sq;
  const int b = row / ((int64_t)p.Hq * p.Sq);
  const T* o = reinterpret_cast<const T*>(p.out) + b * p.o_sb + t * p.o_ss + h * p.o_sh;
  const T* d = reinterpret_cast<const T*>(p.dout) + b * p.do_sb + t * p.do_ss + h * p.do_sh;
  float acc = 0.f;
  for (int i = lane; i < p.Dv; i += 64) acc += to_f32(o[i]) * to_f32(d[i]);
  acc = wave_sum(acc);
  // a gradient flowing into lse adds P·dlse to dS = P(dP - δ): fold it into δ
  if (p.dlse) acc -= p.dlse[b * p.l_sb + t * p.l_ss + h * p.l_sh];
  if (lane == 0) {
    p.delta[row] = acc;
    // key-major dK/dV: start values of its S and dP accumulators
    if (p.rowc) {
      p.rowc[row] = -p.lse[b * p.l_sb + t * p.l_ss + h * p.l_sh] / p.scale;
      p.rowc[nrows + row] = -acc;
    }
  }
}

// The same for bf16 rows of DV in {128, 256, 512} elements with 16-byte
// aligned rows: DV / 8 lanes per row, one 16-byte load of O and of dO each.
template <int DV>
__global__ __launch_bounds__(kThreads) void delta_vec_kernel(Params p) {
  constexpr int LPR = DV / 8;    // lanes per row
  constexpr int RPW = 64 / LPR;  // rows per wave
  static_assert(LPR * RPW == 64, "DV / 8 divides the wave");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t nrows = (int64_t)p.B * p.Sq * p.Hq;
  const int64_t row = ((int64_t)blockIdx.x * kWaves + wave) * RPW + lane / LPR;
  const bool live = row < nrows;
  const int h = live ? (int)(row % p.Hq) : 0;
  const int t = live ? (int)((row / p.Hq) % p.Sq) : 0;
  const int b = live ? (int)(row / ((int64_t)p.Hq * p.Sq)) : 0;
  float acc = 0.f;
  if (live) {
    const int c = 8 * (lane % LPR);
    const bf16x8 ov = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const bf16*>(p.out) + b * p.o_sb +
                                                       t * p.o_ss + h * p.o_sh + c);
    const bf16x8 dv = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const bf16*>(p.dout) + b * p.do_sb +
                                                       t * p.do_ss + h * p.do_sh + c);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += (float)ov[j] * (float)dv[j];
  }
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if (!live || lane % LPR != 0) return;
  if (p.dlse) acc -= p.dlse[b * p.l_sb + t * p.l_ss + h * p.l_sh];
  p.delta[row] = acc;
  if (p.rowc) {
    p.rowc[row] = -p.lse[b * p.l_sb + t * p.l_ss + h * p.l_sh] / p.scale;
    p.rowc[nrows + row] = -acc;
  }
}

// Shared memory: q row [Dqk] | dout row [Dv] | per-wave dq partial [kWaves][Dqk]
template <typename T>
__global__ __launch_bounds__(kThreads) void bwd_generic_kernel(Params p) {
  extern __shared__ float smem[];
  float* qs = smem;
  float* dos = qs + p.Dqk;
  float* dqw = dos + p.Dv;

  const int row = blockIdx.x;
  const int h = row % p.Hq;
  const int t = (row / p.Hq) % p.Sq;
  const int b = row / (p.Hq * p.Sq);
  const int g = h / p.G;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  const T* qrow = reinterpret_cast<const T*>(p.q) + b * p.q_sb + t * p.q_ss + h * p.q_sh;
  const T* dorow = reinterpret_cast<const T*>(p.dout) + b * p.do_sb + t * p.do_ss + h * p.do_sh;
  for (int d = tid; d < p.Dqk; d += kThreads) qs[d] = to_f32(qrow[d]);
  for (int d = tid; d < p.Dv; d += kThreads) dos[d] = to_f32(dorow[d]);
  for (int d = tid; d < kWaves * p.Dqk; d += kThreads) dqw[d] = 0.f;
  __syncthreads();

  const float lse = p.lse[b * p.l_sb + t * p.l_ss + h * p.l_sh];
  const float delta = p.delta[row];
  T* dqrow = reinterpret_cast<T*>(p.dq) + b * p.dq_sb + t * p.dq_ss + h * p.dq_sh;
  if (lse == kNegInf) {  // no valid slot and no sink: every gradient of this row is 0
    for (int d = tid; d < p.Dqk; d += kThreads) dqrow[d] = from_f32<T>(0.f);
    return;
  }
  const float lse2 = lse * kLog2e;

  const int32_t* irow = p.idx + b * p.i_sb + t * p.i_ss + g * p.i_sh;
  const int bound = bound_of(p, b);
  const T* kb = reinterpret_cast<const T*>(p.k) + b * p.k_sb + g * p.k_sh;
  const T* vb = reinterpret_cast<const T*>(p.v) + b * p.v_sb + g * p.v_sh;
  const int64_t acc_row_k = (int64_t)p.Hkv * p.Dqk, acc_row_v = (int64_t)p.Hkv * p.Dv;
  float* dkb = p.dk_acc + ((int64_t)b * p.Skv * p.Hkv + g) * p.Dqk;
  float* dvb = p.dv_acc + ((int64_t)b * p.Skv * p.Hkv + g) * p.Dv;
  float* mydq = dqw + wave * p.Dqk;

  for (int j = wave; j < p.topk; j += kWaves) {
    const int id = irow[j];
    if (id < 0 || id >= bound) continue;  // wave-uniform
    const T* kr = kb + (int64_t)id * p.k_ss;
    const T* vr = vb + (int64_t)id * p.v_ss;
    float s = 0.f, dp = 0.f;
    for (int d = lane; d < p.Dqk; d += 64) s += qs[d] * to_f32(kr[d]);
    for (int d = lane; d < p.Dv; d += 64) dp += dos[d] * to_f32(vr[d]);
    s = wave_sum(s);
    dp = wave_sum(dp);
    const float pr = exp2f(s * p.scale_log2 - lse2);
    const float ds = pr * (dp - delta);
    const float sds = p.scale * ds;
    float* dkr = dkb + (int64_t)id * acc_row_k;
    float* dvr = dvb + (int64_t)id * acc_row_v;
    for (int d = lane; d < p.Dqk; d += 64) {
      mydq[d] += sds * to_f32(kr[d]);
      atomicAdd(&dkr[d], sds * qs[d]);
    }
    for (int d = lane; d < p.Dv; d += 64) atomicAdd(&dvr[d], pr * dos[d]);
  }
  __syncthreads();
  for (int d = tid; d < p.Dqk; d += kThreads) {
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) acc += dqw[w * p.Dqk + d];
    dqrow[d] = from_f32<T>(acc);
  }
}

__global__ void zero_f32_kernel(float* ptr, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) ptr[i] = 0.f;
}

// fp32 accumulators [B, Skv, Hkv, D] -> output tensor with caller strides.
template <typename T>
__global__ void finish_kernel(const float* acc, int B, int Skv, int Hkv, int D, T* out, int64_t sb, int64_t ss,
                              int64_t sh) {
  const int64_t n = (int64_t)B * Skv * Hkv * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int d = i % D;
    const int64_t r = i / D;
    const int h = r % Hkv;
    const int s = (r / Hkv) % Skv;
    const int b = r / ((int64_t)Hkv * Skv);
    out[b * sb + s * ss + h * sh + d] = from_f32<T>(acc[i]);
  }
}

// Shared K/V rows (v = the first Dv dims of k): dk_acc[r][d] += dv_acc[r][d]
// for d < Dv, so one finish writes the gradient of the shared rows.
__global__ void add_rows_kernel(float* dk, const float* dv, int64_t rows, int Dk, int Dv) {
  const int64_t n = rows * Dv;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / Dv;
    dk[r * Dk + (i - r * Dv)] += dv[i];
  }
}

// Split-k combine: lse2 = log2 Σ_s 2^lse2_s, out = Σ_s 2^(lse2_s - lse2)·o_s
// (o_s the bf16 normalised partial of split s, accumulated in fp32),
// then the optional sink joins the denominator.  One wave per (b, t, h) row:
// the per-split weights are computed once per row (lane s), the partial rows
// are read as float4.
template <typename T>
__global__ __launch_bounds__(kThreads) void combine_kernel(Params p) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + wave;
  const int64_t nrows = (int64_t)p.B * p.Sq * p.Hq;
  if (row >= nrows) return;
  const int h = row % p.Hq;
  const int t = (row / p.Hq) % p.Sq;
  const int b = row / ((int64_t)p.Hq * p.Sq);
  const float ls = lane < p.num_splits ? p.part_lse[lane * nrows + row] : kNegInf;
  const float sink2 = p.sink ? p.sink[h] * kLog2e : kNegInf;
  const float m = wave_max(ls);
  const float mm = fmaxf(m, sink2);
  const float e = (ls == kNegInf || mm == kNegInf) ? 0.f : exp2f(ls - mm);
  float l = wave_sum(e);
  if (p.sink && mm != kNegInf) l += exp2f(sink2 - mm);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const float wl = e * inv;  // weight of split `lane`
  T* orow = reinterpret_cast<T*>(p.out) + b * p.o_sb + t * p.o_ss + h * p.o_sh;
  if ((p.Dv & 7) == 0) {
    for (int d = 8 * lane; d < p.Dv; d += 512) {
      float acc[8] = {};
      for (int s = 0; s < p.num_splits; ++s) {
        const float w = __shfl(wl, s, 64);
        if (w != 0.f) {
          const bf16x8 v = *reinterpret_cast<const bf16x8*>(p.part_o + (s * nrows + row) * p.Dv + d);
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[j] += w * (float)v[j];
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) orow[d + j] = from_f32<T>(acc[j]);
    }
  } else {
    for (int d = lane; d < p.Dv; d += 64) {
      float acc = 0.f;
      for (int s = 0; s < p.num_splits; ++s) {
        const float w = __shfl(wl, s, 64);
        if (w != 0.f) acc += w * (float)p.part_o[(s * nrows + row) * p.Dv + d];
      }
      orow[d] = from_f32<T>(acc);
    }
  }
  if (lane == 0) p.lse[b * p.l_sb + t * p.l_ss + h * p.l_sh] = (l > 0.f) ? (mm + log2f(l)) * kLn2 : kNegInf;
}

// The same merge for NS splits and d_v = 512 (the MLA decode): a wave
// issues its NS partial-row loads together with the LSE loads, before the
// weights that need the LSEs are formed, so it waits for one memory round
// trip instead of one per split.
//
// Placement: the forward puts the splits of work item i (a (b, t) row group,
// Hkv = 1) on XCD i % 8; when the item count and head count allow, the
// workgroups merging item i's rows are dispatched to the same XCD (workgroup
// w goes to XCD w % 8), whose L2 may still hold the partial rows just
// written.
template <typename T, int NS>
__global__ __launch_bounds__(kThreads) void combine512_kernel(Params p) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t nitems = (int64_t)p.B * p.Sq;
  int64_t row;
  if (nitems % 8 == 0 && p.Hq % kWaves == 0) {
    const int per = p.Hq / kWaves;  // workgroups per item
    const int x = blockIdx.x % 8, r = blockIdx.x / 8;
    row = ((int64_t)(r / per) * 8 + x) * p.Hq + (r % per) * kWaves + wave;
  } else {
    row = (int64_t)blockIdx.x * kWaves + wave;
  }
  const int64_t nrows = nitems * p.Hq;
  if (row >= nrows) return;
  const int h = row % p.Hq;
  const int t = (row / p.Hq) % p.Sq;
  const int b = row / ((int64_t)p.Hq * p.Sq);
  // The LSE and sink loads are buffer loads that read 0 out of range (lanes
  // >= NS, no sink) and whose values are selected only after the row loads
  // are issued: a conditional load or a value used at once makes the wave
  // wait for it before issuing the rows, a second memory round trip.
  const uint32_t lse_bytes = (uint32_t)((int64_t)NS * nrows * 4);
  const float ls_raw = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
      make_rsrc(p.part_lse, lse_bytes), lane < NS ? (uint32_t)((lane * nrows + row) * 4) : lse_bytes, 0, 0));
  const float sink_raw = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
      make_rsrc(p.sink, p.sink ? 4u * (uint32_t)p.Hq : 0u), 4u * (uint32_t)h, 0, 0));
  bf16x8 pv[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) pv[s] = *reinterpret_cast<const bf16x8*>(p.part_o + (s * nrows + row) * 512 + 8 * lane);
  // (keeps the row loads ahead of the selects below)
  __builtin_amdgcn_sched_barrier(0);
  const float ls = lane < NS ? ls_raw : kNegInf;
  const float sink2 = p.sink ? sink_raw * kLog2e : kNegInf;
  const float m = wave_max(ls);
  const float mm = fmaxf(m, sink2);
  const float e = (ls == kNegInf || mm == kNegInf) ? 0.f : exp2f(ls - mm);
  float l = wave_sum(e);
  if (p.sink && mm != kNegInf) l += exp2f(sink2 - mm);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const float wl = e * inv;  // weight of split `lane`
  float acc[8] = {};
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const float w = __shfl(wl, s, 64);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += w * (float)pv[s][j];
  }
  T* orow = reinterpret_cast<T*>(p.out) + b * p.o_sb + t * p.o_ss + h * p.o_sh;
#pragma unroll
  for (int j = 0; j < 8; ++j) orow[8 * lane + j] = from_f32<T>(acc[j]);
  if (lane == 0) p.lse[b * p.l_sb + t * p.l_ss + h * p.l_sh] = (l > 0.f) ? (mm + log2f(l)) * kLn2 : kNegInf;
}

// The same merge for NS splits and d_v = 128 (the d = 128 kernel splits a
// top-k set longer than its 1024-slot index window): four rows per wave, a
// 16-lane group per row, 8 dims (16 bytes) per lane; lane s of a group reads
// split s's LSE, and every lane its NS partial-row pieces, all issued before
// the weights are formed (one memory round trip).
template <typename T, int NS>
__global__ __launch_bounds__(kThreads) void combine128_kernel(Params p) {
  const int lane = threadIdx.x & 63, gl = lane & 15;
  const int64_t nrows = (int64_t)p.B * p.Sq * p.Hq;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 16) + (threadIdx.x >> 4);
  const bool ok = row < nrows;
  const int64_t r = ok ? row : nrows - 1;  // (rows past the end compute on the last row, store nothing)
  const int h = r % p.Hq;
  const int t = (r / p.Hq) % p.Sq;
  const int b = r / ((int64_t)p.Hq * p.Sq);
  const uint32_t lse_bytes = (uint32_t)((int64_t)NS * nrows * 4);
  const float ls_raw = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
      make_rsrc(p.part_lse, lse_bytes), gl < NS ? (uint32_t)((gl * nrows + r) * 4) : lse_bytes, 0, 0));
  const float sink_raw = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
      make_rsrc(p.sink, p.sink ? 4u * (uint32_t)p.Hq : 0u), 4u * (uint32_t)h, 0, 0));
  bf16x8 pv[NS];
#pragma unroll
  for (int sp = 0; sp < NS; ++sp) pv[sp] = *reinterpret_cast<const bf16x8*>(p.part_o + (sp * nrows + r) * 128 + 8 * gl);
  __builtin_amdgcn_sched_barrier(0);
  const float ls = gl < NS ? ls_raw : kNegInf;
  const float sink2 = p.sink ? sink_raw * kLog2e : kNegInf;
  float m = ls;
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 16));
  const float mm = fmaxf(m, sink2);
  const float e = (ls == kNegInf || mm == kNegInf) ? 0.f : exp2f(ls - mm);
  float l = e;
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) l += __shfl_xor(l, o, 16);
  if (p.sink && mm != kNegInf) l += exp2f(sink2 - mm);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const float wl = e * inv;  // weight of split gl of this row
  float acc[8] = {};
#pragma unroll
  for (int sp = 0; sp < NS; ++sp) {
    const float w = __shfl(wl, (lane & 48) | sp, 64);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += w * (float)pv[sp][j];
  }
  if (!ok) return;
  T* orow = reinterpret_cast<T*>(p.out) + b * p.o_sb + t * p.o_ss + h * p.o_sh;
  bf16x8 o;
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = (bf16)acc[j];
  *reinterpret_cast<bf16x8*>(orow + 8 * gl) = o;
  if (gl == 0) p.lse[b * p.l_sb + t * p.l_ss + h * p.l_sh] = (l > 0.f) ? (mm + log2f(l)) * kLn2 : kNegInf;
}

// dsink[h] = -Σ_{b,t} 2^(sink·log2e - lse2)·δ over the rows of head h
// (SFA.py:964-970).  One workgroup per head; each thread sums a fixed
// stride of rows and the block reduction adds in a fixed order, so the result
// is bitwise reproducible (no atomics).  Rows with lse = -inf contribute 0.
__global__ __launch_bounds__(kThreads) void dsink_kernel(Params p) {
  __shared__ float red[kWaves];
  const int h = blockIdx.x;
  const int64_t nbt = (int64_t)p.B * p.Sq;
  const float sink2 = p.sink[h] * kLog2e;
  float acc = 0.f;
  for (int64_t r = threadIdx.x; r < nbt; r += kThreads) {
    const int t = (int)(r % p.Sq);
    const int b = (int)(r / p.Sq);
    const float lse = p.lse[b * p.l_sb + t * p.l_ss + (int64_t)h * p.l_sh];
    if (lse != kNegInf) acc -= exp2f(sink2 - lse * kLog2e) * p.delta[r * p.Hq + h];
  }
  acc = block_reduce_sum(acc, red);
  if (threadIdx.x == 0) p.dsink[h] = acc;
}

inline int grid_for(int64_t n, int threads) {
  int64_t g = (n + threads - 1) / threads;
  if (g > 65535 * 16) g = 65535 * 16;
  if (g < 1) g = 1;
  return (int)g;
}

}  // namespace

hipError_t launch_fwd_generic(const Params& p, int dtype, hipStream_t s) {
  const size_t sh = sizeof(float) * ((size_t)p.Dqk + p.topk + kWaves);
  const dim3 grid((unsigned)((int64_t)p.B * p.Sq * p.Hq));
  if (dtype == SFA_DTYPE_F32)
    hipLaunchKernelGGL(fwd_generic_kernel<float>, grid, dim3(kThreads), sh, s, p);
  else
    hipLaunchKernelGGL(fwd_generic_kernel<bf16>, grid, dim3(kThreads), sh, s, p);
  return hipGetLastError();
}

hipError_t launch_bwd_delta(const Params& p, int dtype, hipStream_t s) {
  const int64_t rows = (int64_t)p.B * p.Sq * p.Hq;
  const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves));
  auto al16 = [](const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; };
  const bool vec = dtype == SFA_DTYPE_BF16 && (p.Dv == 128 || p.Dv == 256 || p.Dv == 512) && al16(p.out) &&
                   al16(p.dout) && p.o_sb % 8 == 0 && p.o_ss % 8 == 0 && p.o_sh % 8 == 0 && p.do_sb % 8 == 0 &&
                   p.do_ss % 8 == 0 && p.do_sh % 8 == 0;
  if (vec) {
    const int rpw = 64 / (p.Dv / 8);
    const dim3 vgrid((unsigned)((rows + (int64_t)kWaves * rpw - 1) / ((int64_t)kWaves * rpw)));
    if (p.Dv == 128)
      hipLaunchKernelGGL(delta_vec_kernel<128>, vgrid, dim3(kThreads), 0, s, p);
    else if (p.Dv == 256)
      hipLaunchKernelGGL(delta_vec_kernel<256>, vgrid, dim3(kThreads), 0, s, p);
    else
      hipLaunchKernelGGL(delta_vec_kernel<512>, vgrid, dim3(kThreads), 0, s, p);
    return hipGetLastError();
  }
  if (dtype == SFA_DTYPE_F32)
    hipLaunchKernelGGL(delta_kernel<float>, grid, dim3(kThreads), 0, s, p);
  else
    hipLaunchKernelGGL(delta_kernel<bf16>, grid, dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_bwd_dsink(const Params& p, hipStream_t s) {
  if (p.sink == nullptr || p.dsink == nullptr) return hipSuccess;
  hipLaunchKernelGGL(dsink_kernel, dim3((unsigned)p.Hq), dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_bwd_generic(const Params& p, int dtype, hipStream_t s) {
  const size_t sh = sizeof(float) * ((size_t)p.Dqk + p.Dv + (size_t)kWaves * p.Dqk);
  const dim3 grid((unsigned)((int64_t)p.B * p.Sq * p.Hq));
  if (dtype == SFA_DTYPE_F32)
    hipLaunchKernelGGL(bwd_generic_kernel<float>, grid, dim3(kThreads), sh, s, p);
  else
    hipLaunchKernelGGL(bwd_generic_kernel<bf16>, grid, dim3(kThreads), sh, s, p);
  return hipGetLastError();
}

hipError_t launch_zero_f32(float* ptr, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(zero_f32_kernel, dim3(grid_for((int64_t)n, 256 * 4)), dim3(256), 0, s, ptr, n);
  return hipGetLastError();
}

hipError_t launch_bwd_finish(const Params& p, int dtype, void* dk, int64_t dk_sb, int64_t dk_ss, int64_t dk_sh,
                             void* dv, int64_t dv_sb, int64_t dv_ss, int64_t dv_sh, hipStream_t s) {
  const int64_t nk = (int64_t)p.B * p.Skv * p.Hkv * p.Dqk, nv = (int64_t)p.B * p.Skv * p.Hkv * p.Dv;
  if (dtype == SFA_DTYPE_F32) {
    hipLaunchKernelGGL(finish_kernel<float>, dim3(grid_for(nk, 256 * 4)), dim3(256), 0, s, p.dk_acc, p.B, p.Skv,
                       p.Hkv, p.Dqk, (float*)dk, dk_sb, dk_ss, dk_sh);
    hipLaunchKernelGGL(finish_kernel<float>, dim3(grid_for(nv, 256 * 4)), dim3(256), 0, s, p.dv_acc, p.B, p.Skv,
                       p.Hkv, p.Dv, (float*)dv, dv_sb, dv_ss, dv_sh);
  } else {
    hipLaunchKernelGGL(finish_kernel<bf16>, dim3(grid_for(nk, 256 * 4)), dim3(256), 0, s, p.dk_acc, p.B, p.Skv,
                       p.Hkv, p.Dqk, (bf16*)dk, dk_sb, dk_ss, dk_sh);
    hipLaunchKernelGGL(finish_kernel<bf16>, dim3(grid_for(nv, 256 * 4)), dim3(256), 0, s, p.dv_acc, p.B, p.Skv,
                       p.Hkv, p.Dv, (bf16*)dv, dv_sb, dv_ss, dv_sh);
  }
  return hipGetLastError();
}

hipError_t launch_bwd_finish_merged(const Params& p, int dtype, void* dk, int64_t dk_sb, int64_t dk_ss,
                                    int64_t dk_sh, bool add_dv, hipStream_t s) {
  const int64_t rows = (int64_t)p.B * p.Skv * p.Hkv, nk = rows * p.Dqk;
  if (add_dv)
    hipLaunchKernelGGL(add_rows_kernel, dim3(grid_for(rows * p.Dv, 256 * 4)), dim3(256), 0, s, p.dk_acc, p.dv_acc, rows,
                       p.Dqk, p.Dv);
  if (dtype == SFA_DTYPE_F32)
    hipLaunchKernelGGL(finish_kernel<float>, dim3(grid_for(nk, 256 * 4)), dim3(256), 0, s, p.dk_acc, p.B, p.Skv,
                       p.Hkv, p.Dqk, (float*)dk, dk_sb, dk_ss, dk_sh);
  else
    hipLaunchKernelGGL(finish_kernel<bf16>, dim3(grid_for(nk, 256 * 4)), dim3(256), 0, s, p.dk_acc, p.B, p.Skv,
                       p.Hkv, p.Dqk, (bf16*)dk, dk_sb, dk_ss, dk_sh);
  return hipGetLastError();
}

hipError_t launch_combine(const Params& p, int dtype, hipStream_t s) {
  const int64_t rows = (int64_t)p.B * p.Sq * p.Hq;
  const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves));
  if (p.Dv == 512 && (p.num_splits == 2 || p.num_splits == 4 || p.num_splits == 8)) {
#define SFA_COMBINE512(NS)                                                              \
  if (p.num_splits == NS) {                                                               \
    if (dtype == SFA_DTYPE_F32)                                                           \
      hipLaunchKernelGGL((combine512_kernel<float, NS>), grid, dim3(kThreads), 0, s, p); \
    else                                                                                  \
      hipLaunchKernelGGL((combine512_kernel<bf16, NS>), grid, dim3(kThreads), 0, s, p);  \
    return hipGetLastError();                                                             \
  }
    SFA_COMBINE512(2)
    SFA_COMBINE512(4)
    SFA_COMBINE512(8)
#undef SFA_COMBINE512
  }
  if (p.Dv == 128 && dtype == SFA_DTYPE_BF16 && (p.num_splits == 2 || p.num_splits == 4 || p.num_splits == 8)) {
    const dim3 grid128((unsigned)((rows + kThreads / 16 - 1) / (kThreads / 16)));
    if (p.num_splits == 2)
      hipLaunchKernelGGL((combine128_kernel<bf16, 2>), grid128, dim3(kThreads), 0, s, p);
    else if (p.num_splits == 4)
      hipLaunchKernelGGL((combine128_kernel<bf16, 4>), grid128, dim3(kThreads), 0, s, p);
    else
      hipLaunchKernelGGL((combine128_kernel<bf16, 8>), grid128, dim3(kThreads), 0, s, p);
    return hipGetLastError();
  }
  if (dtype == SFA_DTYPE_F32)
    hipLaunchKernelGGL(combine_kernel<float>, grid, dim3(kThreads), 0, s, p);
  else
    hipLaunchKernelGGL(combine_kernel<bf16>, grid, dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

}  // namespace sfa

// LDS access helpers shared by the MFMA kernels (gfx950).
#pragma once

#include "sfa_common.h"

namespace sfa {

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// max / sum of x over lanes l and l ^ 32 (gfx950 v_permlane32_swap: no LDS trip)
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// LDS reads go through pointers derived from the __shared__ arrays themselves,
// so the compiler keeps per-array alias information and does not make reads of
// one tile buffer wait for the DMA still filling another.
__device__ __forceinline__ bf16x8 lds_read_b128(const void* base, uint32_t byte_off) {
  return *reinterpret_cast<const bf16x8*>(reinterpret_cast<const char*>(base) + byte_off);
}

__device__ __forceinline__ bf16x4 lds_read_tr16(const void* base, uint32_t byte_off) {
  typedef __attribute__((address_space(3))) const char lds_cchar;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      (lds_bf16x4*)((lds_cchar*)(base) + byte_off));
}

// Gather NKT rows of CH 16-byte chunks into an LDS tile with row pitch
// PITCH = CH + 1 slots, straight from global memory (buffer_load ... lds, no
// VGPR staging).  ib[r] is the row id of tile row r, or -1: such rows, and
// each row's pad slot, read from an out-of-range offset, so the hardware
// writes zeros.  Slot u of the tile holds chunk (u % PITCH) of row u / PITCH;
// thread tid owns slots tid, tid + THREADS, ... and walks (row, chunk)
// incrementally from two registers made opaque per call, so the compiler
// cannot hoist one offset per instruction out of the caller's tile loop.
// The LDS address of lane l of an instruction is the wave-uniform base plus
// 16 * l, so the destination of each instruction is 64 consecutive slots.
template <int NKT, int CH, int THREADS>
__device__ __forceinline__ void gather_tile(const int* ib, u32x4* dst, const __amdgpu_buffer_rsrc_t& rs,
                                            uint32_t row_bytes, int tid, int wave) {
  constexpr int PITCH = CH + 1;
  constexpr int NSLOT = NKT * PITCH;
  constexpr int NIT = (NSLOT + THREADS - 1) / THREADS;
  constexpr int DR = THREADS / PITCH, DC = THREADS % PITCH;
  int r = tid / PITCH, c = tid - (tid / PITCH) * PITCH;
  asm volatile("" : "+v"(r), "+v"(c));
  int ids[NIT], cs[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const bool live = (NSLOT % THREADS == 0) || (it * THREADS + tid < NSLOT);
    ids[it] = live ? ib[r] : -1;
    cs[it] = c;
    c += DC;
    r += DR;
    if (c >= PITCH) {
      c -= PITCH;
      r += 1;
    }
  }
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    if ((NSLOT % THREADS == 0) || (it * THREADS + tid < NSLOT)) {
      const uint32_t off =
          (ids[it] >= 0 && cs[it] < CH) ? __umul24((uint32_t)ids[it], row_bytes) + (uint32_t)cs[it] * 16u : kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + it * THREADS + wave * 64), 16, off, 0, 0, 0);
    }
  }
}

// Row-wise gather for wide rows (PITCH = CH + 1 >= 64 slots, so one 64-lane
// instruction spans at most two rows).  Wave w gathers tile rows
// [w * RPW, (w + 1) * RPW), i.e. the contiguous slot range [w * SPW, (w+1) * SPW).
// For instruction k every slot position is a compile-time constant, and the
// two row byte offsets it needs are wave-uniform scalars, so issuing one
// instruction costs two VALU operations and no per-lane index reads:
//   voffset(lane) = 16 * lane + (lane < bnd ? S0 : S1)
//   S0 = base[r0] + 16 * c0,  S1 = base[r0 + 1] + 16 * (c0 - PITCH)
// with r0, c0 the row / chunk of the instruction's first slot and bnd the
// lanes left in row r0.  base[r] is id * row_bytes, or kOOBRow for a padding
// row, which keeps every offset of that row above 2^31 (out of range, the
// hardware writes zeros).  The pad slot of a row reads the 16 bytes after the
// row (the next row's first chunk, or zeros past the end of the range); pad
// slots are never read.  Instructions can be issued one at a time (issue(k)),
// so a caller can spread them over its MFMA stream.
constexpr uint32_t kOOBRow = 0x80001000u;

template <int NKT, int CH, int NWAVES>
struct RowGather {
  static constexpr int PITCH = CH + 1;
  static constexpr int RPW = NKT / NWAVES;       // rows per wave
  static constexpr int SPW = RPW * PITCH;        // slots per wave
  static constexpr int NI = (SPW + 63) / 64;     // instructions per wave
  static_assert(PITCH >= 64, "an instruction must span at most two rows");
  static_assert(NKT % NWAVES == 0, "rows split evenly over the waves");

  uint32_t base[RPW];

  // ib: the tile's NKT staged row ids (-1 = padding row); wave-uniform reads.
  // valid == false makes every row a padding row (the instructions then move
  // no global data and write zeros); ib must still point into the array.
  // (No pointer select: the compiler keeps ib's array identity, so the read
  // does not wait for DMA into other LDS arrays.)
  __device__ __forceinline__ void load_ids(const int* ib, bool valid, int wave, uint32_t row_bytes) {
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int id = __builtin_amdgcn_readfirstlane(ib[wave * RPW + r]);
      base[r] = (valid && id >= 0) ? __umul24((uint32_t)id, row_bytes) : kOOBRow;
    }
  }

  __device__ __forceinline__ void issue(int k, const __amdgpu_buffer_rsrc_t& rs, u32x4* dst, int wave,
                                        int lane) const {
    const int s0 = 64 * k;
    const int r0 = s0 / PITCH, c0 = s0 % PITCH;
    const int bnd = PITCH - c0;
    const uint32_t S0 = base[r0] + 16u * (uint32_t)c0;
    uint32_t off = S0;
    if (bnd < 64 && r0 + 1 < RPW) {
      const uint32_t S1 = base[r0 + 1] + 16u * (uint32_t)c0 - 16u * (uint32_t)PITCH;
      off = lane < bnd ? S0 : S1;
    }
    off += 16u * (uint32_t)lane;
    u32x4* d = dst + wave * SPW + s0;
    if (s0 + 64 <= SPW) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)d, 16, off, 0, 0, 0);
    } else if (lane < SPW - s0) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)d, 16, off, 0, 0, 0);
    }
  }
};

}  // namespace sfa

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

}  // namespace sfa

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

// max of three floats as one v_max3_f32 (fmaxf on values the compiler cannot
// prove canonical, such as MFMA results from inline asm, adds a quieting
// v_max x, x per operand; NaN-free inputs here)
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

__device__ __forceinline__ float max_raw(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// xor32_max with raw maxes (see max3_raw)
__device__ __forceinline__ float xor32_max_raw(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_raw(__uint_as_float(r[0]), __uint_as_float(r[1]));
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

// Chunk swizzle of the MLA tile (row pitch 72 16-byte slots, no pad): row r
// stores its chunk c at slot position c ^ swz(r), swz(r) < 8 built from bits
// 1..3 of r.  With it both operand read patterns are bank-conflict free
// (64 banks x 4 bytes; 256 bytes per pass):
//  * S^T A operands (ds_read_b128): a 16-lane pass reads one chunk of 16
//    consecutive rows;
//  * O^T A operands (ds_read_b64_tr_b16): a 32-lane pass reads 4 consecutive
//    rows x 4 consecutive chunks (an aligned group of 4);
// the unswizzled pitch-73 layout makes the second pattern 2-way conflicted
// and a pitch of 72 without swizzle makes the first 8-way conflicted.  The
// swizzle never moves a chunk out of its aligned group of 8, so it commutes
// with adding multiples of 8 to a chunk index.
__device__ __forceinline__ int tile_swz(int r) {
  return (((r >> 1) & 1) << 2) ^ ((r >> 2) & 1) ^ (((r >> 3) & 1) << 1);
}

// Row-wise gather for wide rows (PITCH >= 64 slots, so one 64-lane
// instruction spans at most two rows).  Wave w gathers tile rows
// [w * RPW, (w + 1) * RPW), i.e. the contiguous slot range [w * SPW, (w+1) * SPW).
// For instruction k every slot position is a compile-time constant, and the
// two row byte offsets it needs are wave-uniform scalars, so issuing one
// instruction costs a few VALU operations and no per-lane index reads:
//   voffset(lane) = lane < bnd ? S0 + X0 : S1 + X1
//   S0 = base[r0] + 16 * c0,  S1 = base[r0 + 1] + 16 * (c0 - PITCH)
//   Xi = 16 * (lane ^ swz(row i))            (16 * lane without swizzle)
// with r0, c0 the row / slot of the instruction's first slot and bnd the
// lanes left in row r0 (with the swizzle c0 is a multiple of 8, so the lane at
// slot c0 + lane loads chunk c0 + (lane ^ swz)).  base[r] is id * row_bytes,
// or kOOBRow for a padding row, which keeps every offset of that row above
// 2^31 (out of range, the hardware writes zeros).  Without the swizzle the
// row has one pad slot (PITCH = CH + 1), which reads the 16 bytes after the
// row (the next row's first chunk, or zeros past the end of the range) and is
// never read.  Instructions can be issued one at a time (issue(k)), so a
// caller can spread them over its MFMA stream.
constexpr uint32_t kOOBRow = 0x80001000u;

// Row sources of RowGather.  base_t is what a row's base is held in; a
// padding row (id < 0 or !valid) gets a base whose every lane offset reads
// zeros.
// Contiguous rows of one (batch, kv head) slice: 32-bit offsets into a
// buffer resource, padding rows out of range.
struct BufRows {
  __amdgpu_buffer_rsrc_t rs;
  uint32_t row_bytes;
  typedef uint32_t base_t;
  __device__ __forceinline__ base_t row_base(int id, bool valid) const {
    return (valid && id >= 0) ? __umul24((uint32_t)id, row_bytes) : kOOBRow;
  }
  __device__ __forceinline__ void load_lds16(u32x4* dst, base_t off) const {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)dst, 16, off, 0, 0, 0);
  }
  static constexpr bool kUntrackedDma = false;  // the compiler tracks the DMA
};
// BufRows for staged entries that already are row byte offsets
// (IdxStage::store_offsets: kOOBRow for an invalid slot), so a row's base
// costs one select instead of a validity test and a multiply.
struct BufRowsOff : BufRows {
  __device__ __forceinline__ base_t row_base(int off, bool valid) const { return valid ? (uint32_t)off : kOOBRow; }
};
// One buffer_load_dwordx4 ... lds (M0 = the wave's LDS destination, lane l
// writes 16 bytes at M0 + 16 l) as inline asm: the compiler neither sees nor
// waits for it (its builtin form makes every later LDS read that the
// compiler cannot tell apart wait for vmcnt(0)).  The caller waits for
// vmcnt itself before the barrier that publishes the data.
__device__ __forceinline__ void dma_lds16_untracked(__amdgpu_buffer_rsrc_t rs, u32x4* dst, uint32_t off) {
  const uint32_t lds = (uint32_t)(uintptr_t)(lds_void*)dst;
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds), "v"(off), "s"(rs)
               : "memory", "m0");
}
// BufRows with untracked DMA (dma_lds16_untracked)
struct BufRowsUT : BufRows {
  __device__ __forceinline__ void load_lds16(u32x4* dst, base_t off) const { dma_lds16_untracked(rs, dst, off); }
  static constexpr bool kUntrackedDma = true;
};
// Rows of a paged pool (ids are the scaled pool offsets of staged_pool_off):
// 64-bit addresses, since a pool may exceed the 4 GiB a buffer offset
// reaches; padding rows read kZeroRow.
// The DMA (global_load_lds_dwordx4: M0 = the wave's LDS destination, lane l
// writes 16 bytes at M0 + 16 l) is issued as inline asm: the compiler counts
// its builtin form against the LDS counter too, which turns every later
// operand read's wait into lgkmcnt(0) and serialises the tile's LDS reads.
// The hardware counts it on vmcnt only, and the compiler does not see it, so
// the kernel waits for vmcnt(0) itself before the barrier that publishes a
// tile (waits the compiler inserts for other loads only get stricter).
struct PoolRows {
  const char* base;  // pool base + the kv head's offset
  int shift;         // staged offsets are in units of 2^shift bytes
  typedef uint64_t base_t;
  __device__ __forceinline__ base_t row_base(int off, bool valid) const {
    return (valid && off >= 0) ? (uint64_t)(uintptr_t)base + ((uint64_t)(uint32_t)off << shift)
                               : (uint64_t)(uintptr_t)kZeroRow;
  }
  __device__ __forceinline__ void load_lds16(u32x4* dst, base_t addr) const {
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_void*)dst;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(addr) : "memory", "m0");
  }
  static constexpr bool kUntrackedDma = true;  // the caller waits for vmcnt(0) before reading the tile
};

template <int NKT, int CH, int NWAVES, bool SWZ, class Src = BufRows>
struct RowGather {
  static constexpr int PITCH = SWZ ? CH : CH + 1;
  static constexpr int RPW = NKT / NWAVES;       // rows per wave
  static constexpr int SPW = RPW * PITCH;        // slots per wave
  static constexpr int NI = (SPW + 63) / 64;     // instructions per wave
  static_assert(PITCH >= 64, "an instruction must span at most two rows");
  static_assert(NKT % NWAVES == 0, "rows split evenly over the waves");
  static_assert(!SWZ || (PITCH % 8 == 0 && CH % 8 == 0), "swizzled rows are whole groups of 8 chunks");

  typename Src::base_t base[RPW];

  // ib: the tile's NKT staged row ids (-1 = padding row); wave-uniform reads.
  // valid == false makes every row a padding row (the instructions then move
  // no global data and write zeros); ib must still point into the array.
  // (No pointer select: the compiler keeps ib's array identity, so the read
  // does not wait for DMA into other LDS arrays.)
  __device__ __forceinline__ void load_ids(const int* ib, bool valid, int wave, const Src& src) {
    int raw[RPW];
    fetch(ib, wave, raw);
    set(raw, valid, src);
  }
  // load_ids in two halves, so a caller can issue the LDS reads early and
  // turn them into offsets once they have landed.
  __device__ __forceinline__ static void fetch(const int* ib, int wave, int (&raw)[RPW]) {
#pragma unroll
    for (int r = 0; r < RPW; ++r) raw[r] = ib[wave * RPW + r];
  }
  __device__ __forceinline__ void set_row(int r, int raw, bool valid, const Src& src) {
    const int id = __builtin_amdgcn_readfirstlane(raw);
    base[r] = src.row_base(id, valid);
  }
  __device__ __forceinline__ void set(const int (&raw)[RPW], bool valid, const Src& src) {
#pragma unroll
    for (int r = 0; r < RPW; ++r) set_row(r, raw[r], valid, src);
  }

  // (lanes past the first row's end read chunk c0 + lane' - PITCH of the
  // next row, lane' = lane or lane ^ swz; lane' >= bnd, so that offset is
  // non-negative)
  __device__ __forceinline__ void issue(int k, const Src& src, u32x4* dst, int wave, int lane) const {
    const int s0 = 64 * k;
    const int r0 = s0 / PITCH, c0 = s0 % PITCH;
    const int bnd = PITCH - c0;
    const uint32_t l16 = 16u * (uint32_t)lane;
    const uint32_t x0 = SWZ ? l16 ^ (16u * (uint32_t)tile_swz(wave * RPW + r0)) : l16;
    typename Src::base_t a = base[r0] + (16u * (uint32_t)c0 + x0);
    if (bnd < 64 && r0 + 1 < RPW) {
      const uint32_t x1 = SWZ ? l16 ^ (16u * (uint32_t)tile_swz(wave * RPW + r0 + 1)) : l16;
      const typename Src::base_t a1 = base[r0 + 1] + (16u * (uint32_t)c0 + x1 - 16u * (uint32_t)PITCH);
      a = lane < bnd ? a : a1;
    }
    u32x4* d = dst + wave * SPW + s0;
    if (s0 + 64 <= SPW) {
      src.load_lds16(d, a);
    } else if (lane < SPW - s0) {
      src.load_lds16(d, a);
    }
  }
};

}  // namespace sfa

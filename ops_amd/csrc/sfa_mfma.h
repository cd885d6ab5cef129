// MFMA wrappers shared by the MFMA kernels (gfx950, bf16 in, fp32 accumulate).
#pragma once

#include "sfa_common.h"

namespace sfa {

template <int T>
struct Mfma;

template <>
struct Mfma<32> {
  typedef f32x16 acc_t;
  static __device__ __forceinline__ acc_t mma(bf16x8 a, bf16x8 b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // Inline-asm MFMAs.  The O^T accumulators (256 registers per lane) must stay
  // in the AGPR file and the S^T accumulator in VGPRs; builtins leave that
  // choice to the compiler, which mixes the files and spills.  The compiler
  // does not model hazards inside inline asm, so the code provides them:
  //  * RAW VALU -> srcA/srcB needs 2 wait states: callers pass nop = true
  //    when an operand may have just been written by a VALU instruction;
  //  * WAR srcA/srcB -> later write: every MFMA also takes the operands of
  //    the previous MFMA (pa, pb) as inputs, so the compiler cannot reuse
  //    those registers before the next MFMA has issued; the last MFMA of a
  //    sequence is followed by tail(), which holds its operands for 8 more
  //    wait states;
  //  * RAW result -> VALU read needs up to 18 wait states: drain_*().
  // The "memory" clobber keeps the software-pipelined operand loads in
  // program order around the MFMAs.
  template <bool NOP>
  static __device__ __forceinline__ void mma_agpr(bf16x8 a, bf16x8 b, acc_t& c, const bf16x8& pa, const bf16x8& pb) {
    if constexpr (NOP)
      asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                   : "+a"(c) : "v"(a), "v"(b), "v"(pa), "v"(pb) : "memory");
    else
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                   : "+a"(c) : "v"(a), "v"(b), "v"(pa), "v"(pb) : "memory");
  }
  static __device__ __forceinline__ void mma_v(bf16x8 a, bf16x8 b, acc_t& c, const bf16x8& pa, const bf16x8& pb) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                 : "+v"(c) : "v"(a), "v"(b), "v"(pa), "v"(pb) : "memory");
  }
  static __device__ __forceinline__ void mma_v0(bf16x8 a, bf16x8 b, acc_t& c) {
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0"
                 : "=&v"(c) : "v"(a), "v"(b) : "memory");
  }
  // c += a b where c may just have been written by a VALU instruction
  static __device__ __forceinline__ void mma_vn(bf16x8 a, bf16x8 b, acc_t& c, const bf16x8& pa, const bf16x8& pb) {
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                 : "+v"(c) : "v"(a), "v"(b), "v"(pa), "v"(pb) : "memory");
  }
  // c = a b (fresh VGPR accumulator) with the previous MFMA's operands kept alive
  static __device__ __forceinline__ void mma_v0k(bf16x8 a, bf16x8 b, acc_t& c, const bf16x8& pa,
                                                 const bf16x8& pb) {
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0"
                 : "=&v"(c) : "v"(a), "v"(b), "v"(pa), "v"(pb) : "memory");
  }
  static __device__ __forceinline__ void tail(const bf16x8& a, const bf16x8& b) {
    asm volatile("s_nop 7" : : "v"(a), "v"(b));
  }
  // wait states between the last asm MFMA writing an accumulator and VALU reads
  static __device__ __forceinline__ void drain_v(acc_t& c, const bf16x8& a, const bf16x8& b) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(c) : "v"(a), "v"(b));
  }
  // both VGPR accumulators of two interleaved chains (the last MFMA used a, b)
  static __device__ __forceinline__ void drain_v2(acc_t& c0, acc_t& c1, const bf16x8& a, const bf16x8& b) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(c0), "+v"(c1) : "v"(a), "v"(b));
  }
  static __device__ __forceinline__ void drain(acc_t& c) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+a"(c));
  }
  // c *= s on an AGPR-resident accumulator without moving it to VGPRs.
  static __device__ __forceinline__ void scale_agpr(acc_t& c, float s) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float x = c[e];
      float tmp;
      asm volatile(
          "v_accvgpr_read_b32 %1, %0\n\t"
          "v_mul_f32 %1, %1, %2\n\t"
          "v_accvgpr_write_b32 %0, %1"
          : "+a"(x), "=&v"(tmp)
          : "v"(s));
      c[e] = x;
    }
  }
};

// Inline-asm 16x16x32 bf16 MFMAs with the accumulator pinned to AGPRs, for
// kernels whose accumulators do not fit next to their operands in the VGPR
// file.  The hazard rules are those of Mfma<32> above: NOP = true when an
// operand may just have been written by a VALU instruction, the previous
// MFMA's operands are passed along so their registers stay live until this
// one has issued, tail() after the last MFMA of a sequence, drain() before a
// VALU (or v_accvgpr_read) use of a result.  mma_b_agpr takes its B operand
// from AGPRs (gfx950 MFMAs read A/B from either file).
struct Mfma16A {
  typedef f32x4 acc_t;
  template <bool NOP>
  static __device__ __forceinline__ void mma(bf16x8 a, bf16x8 b, acc_t& c, const bf16x8& pa, const bf16x8& pb) {
    if constexpr (NOP)
      asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                   : "+a"(c) : "v"(a), "v"(b), "v"(pa), "v"(pb) : "memory");
    else
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                   : "+a"(c) : "v"(a), "v"(b), "v"(pa), "v"(pb) : "memory");
  }
  // c = a b: a fresh accumulator (srcC = 0), so no VALU write of c precedes it
  static __device__ __forceinline__ void mma0(bf16x8 a, bf16x8 b, acc_t& c, const bf16x8& pa, const bf16x8& pb) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0"
                 : "=&a"(c) : "v"(a), "v"(b), "v"(pa), "v"(pb) : "memory");
  }
  // A operand from AGPRs, B from VGPRs (pb: the previous MFMA's B, kept live)
  static __device__ __forceinline__ void mma_a_agpr(const bf16x8& a, bf16x8 b, acc_t& c, const bf16x8& pb) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "a"(a), "v"(b), "v"(pb) : "memory");
  }
  static __device__ __forceinline__ void mma_b_agpr(bf16x8 a, const bf16x8& b, acc_t& c, const bf16x8& pa) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "a"(b), "v"(pa) : "memory");
  }
  // VGPR accumulators: c = a b (fresh) and c += a b, with B in VGPRs or AGPRs
  static __device__ __forceinline__ void mma_v0(bf16x8 a, bf16x8 b, acc_t& c, const bf16x8& pa) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "v"(b), "v"(pa) : "memory");
  }
  static __device__ __forceinline__ void mma_v(bf16x8 a, bf16x8 b, acc_t& c, const bf16x8& pa) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b), "v"(pa) : "memory");
  }
  // c += a b with b just written by a VALU instruction
  static __device__ __forceinline__ void mma_vn(bf16x8 a, bf16x8 b, acc_t& c, const bf16x8& pa) {
    asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b), "v"(pa) : "memory");
  }
  static __device__ __forceinline__ void drain_v1(acc_t& c) { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(c)); }
  static __device__ __forceinline__ void mma_v0_ba(bf16x8 a, const bf16x8& b, acc_t& c, const bf16x8& pa) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "a"(b), "v"(pa) : "memory");
  }
  static __device__ __forceinline__ void mma_v_ba(bf16x8 a, const bf16x8& b, acc_t& c, const bf16x8& pa) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "a"(b), "v"(pa) : "memory");
  }
  // wait states between the last MFMA writing VGPR accumulators and VALU reads
  static __device__ __forceinline__ void drain_v4(acc_t& c0, acc_t& c1, acc_t& c2, acc_t& c3) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3));
  }
  static __device__ __forceinline__ void tail(const bf16x8& a, const bf16x8& b) {
    asm volatile("s_nop 7" : : "v"(a), "v"(b));
  }
  static __device__ __forceinline__ void tail1(const bf16x8& a) { asm volatile("s_nop 7" : : "v"(a)); }
  static __device__ __forceinline__ void drain(acc_t& c) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+a"(c));
  }
  // bf16x8 operand kept in AGPRs (v_accvgpr_write of a VGPR value)
  static __device__ __forceinline__ bf16x8 to_agpr(bf16x8 x) {
    asm volatile("" : "+a"(x));
    return x;
  }
};

template <>
struct Mfma<16> {
  typedef f32x4 acc_t;
  static __device__ __forceinline__ acc_t mma(bf16x8 a, bf16x8 b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  template <bool NOP>
  static __device__ __forceinline__ void mma_agpr(bf16x8 a, bf16x8 b, acc_t& c, const bf16x8&, const bf16x8&) {
    c = mma(a, b, c);
  }
  static __device__ __forceinline__ void mma_v(bf16x8 a, bf16x8 b, acc_t& c, const bf16x8&, const bf16x8&) {
    c = mma(a, b, c);
  }
  static __device__ __forceinline__ void mma_v0(bf16x8 a, bf16x8 b, acc_t& c) { c = mma(a, b, acc_t{}); }
  static __device__ __forceinline__ void tail(const bf16x8&, const bf16x8&) {}
  static __device__ __forceinline__ void drain_v(acc_t&, const bf16x8&, const bf16x8&) {}
  static __device__ __forceinline__ void scale_agpr(acc_t& c, float s) { c *= s; }
  static __device__ __forceinline__ void drain(acc_t&) {}
};

}  // namespace sfa

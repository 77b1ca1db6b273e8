// mfma_pipe.hpp -- device building blocks shared by the gfx950 MFMA
// attention kernels (decode_mfma.hip, prefill_mfma.hip): explicit
// vector-memory / LDS waits, inline-asm LDS operand traffic, direct-to-LDS
// DMA with an SGPR base, the VGPR-resident S^T MFMA chain and helpers that
// steer register allocation.
#pragma once

#include "internal.hpp"

namespace qmla {
namespace pipe {

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void wait_vmcnt_dyn(int n) {
  // n is wave-uniform (scalar); dispatch to an immediate.
  switch (n) {
#define QMLA_W(k) case k: wait_vmcnt<k>(); break;
    QMLA_W(0) QMLA_W(1) QMLA_W(2) QMLA_W(3) QMLA_W(4) QMLA_W(5) QMLA_W(6) QMLA_W(7)
    QMLA_W(8) QMLA_W(9) QMLA_W(10) QMLA_W(11) QMLA_W(12) QMLA_W(13) QMLA_W(14) QMLA_W(15)
    QMLA_W(16) QMLA_W(17) QMLA_W(18) QMLA_W(19) QMLA_W(20) QMLA_W(21) QMLA_W(22) QMLA_W(23)
    QMLA_W(24) QMLA_W(25) QMLA_W(26) QMLA_W(27) QMLA_W(28) QMLA_W(29) QMLA_W(30) QMLA_W(31)
    QMLA_W(32) QMLA_W(33) QMLA_W(34) QMLA_W(35) QMLA_W(36) QMLA_W(37) QMLA_W(38) QMLA_W(39)
    QMLA_W(40) QMLA_W(41) QMLA_W(42) QMLA_W(43) QMLA_W(44) QMLA_W(45) QMLA_W(46) QMLA_W(47)
    QMLA_W(48) QMLA_W(49) QMLA_W(50) QMLA_W(51) QMLA_W(52) QMLA_W(53) QMLA_W(54) QMLA_W(55)
    QMLA_W(56) QMLA_W(57) QMLA_W(58) QMLA_W(59) QMLA_W(60) QMLA_W(61) QMLA_W(62)
#undef QMLA_W
    default: wait_vmcnt<0>(); break;
  }
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4;
typedef __attribute__((address_space(3))) bf16x8_t lds_bf16x8;

// S^T accumulation chain in arch VGPRs.  Any AGPR operand in a function makes
// the compiler pick the AGPR form for every MFMA builtin, which would put
// this 16-register accumulator next to the 256 O^T accumulators in the AGPR
// file and spill Q; issuing the S^T MFMAs through inline asm with "v"
// constraints keeps it in VGPRs.  Hazards: the first MFMA of a chain takes
// srcC = 0 (no VALU -> MFMA srcC dependence); each following one reads the
// previous result as srcC with exactly the same registers (forwarded, no
// wait states); VALU reads of the result are preceded by s_nop padding
// (mfma_s_drain) longer than the MFMA's 8 passes.
__device__ __forceinline__ floatx16_t mfma_s_first(const bf16x8_t &a, const bf16x8_t &b) {
  floatx16_t d;
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
  return d;
}
__device__ __forceinline__ void mfma_s_acc(floatx16_t &d, const bf16x8_t &a, const bf16x8_t &b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_s_drain(floatx16_t &d) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(d));
}

__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v;
  v[0] = (__bf16)a;  // v_cvt_pk_bf16_f32: round to nearest even
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// LDS traffic of the hot loop is issued through inline asm with explicit
// lgkmcnt waits.  The compiler cannot tell the tile reads from the
// direct-to-LDS DMA writes still in flight into other stages, so for
// ordinary loads it drains the vector-memory counter (vmcnt(0): every tile
// in flight) and the LDS counter before each group of reads, which
// serialises the pipeline.  Ordering is explicit instead: a stage is read
// only after wait_tiles + barrier, and each operand after the lgkmcnt wait
// that covers it (LDS operations complete in issue order; any other
// counted operation only makes a wait stricter).
__device__ __forceinline__ uint32_t lds_u32(const lds_char *p) {
  return (uint32_t)(uintptr_t)p;
}
template <int OFF>
__device__ __forceinline__ bf16x8_t ds_b128(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset");
  bf16x8_t r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
  return r;
}
// V^T operand: two transposing 8-byte reads (tokens t and t + 8)
template <int OFF, int HI>
__device__ __forceinline__ bf16x8_t ds_tr2(uint32_t addr) {
  static_assert(OFF >= 0 && OFF + HI < 65536, "ds offset");
  u32x2_t lo, hi;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(lo) : "v"(addr), "n"(OFF));
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(hi) : "v"(addr), "n"(OFF + HI));
  return __builtin_bit_cast(bf16x8_t, (u32x4_t){lo[0], lo[1], hi[0], hi[1]});
}
template <int OFF>
__device__ __forceinline__ void ds_w128(uint32_t addr, const bf16x8_t &v) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "v"(v), "n"(OFF));
}
template <int N>
__device__ __forceinline__ void wait_lgkm() {
  static_assert(N >= 0 && N <= 15, "lgkmcnt");
  asm volatile("s_waitcnt lgkmcnt(%0)" : : "n"(N) : "memory");
}
// Marks x as produced here: placed right after the wait that covers the
// asm read of x, it keeps every use of x (compiler MFMAs, copies) after
// that wait.  Emits no code.
__device__ __forceinline__ void arrived(bf16x8_t &x) { asm volatile("" : "+v"(x)); }

// One direct-to-LDS DMA instruction: 64 lanes x 16 B from sbase + voff
// (uniform base, 32-bit per-lane offset) to LDS address lds + 16 * lane.
// Issued through asm in the SGPR-base form, so no 64-bit per-lane address
// is formed; M0 (the LDS destination) is saved and restored around it, and
// the wait states after the M0 write are covered by the s_nop.  The compiler
// does not track this load: vmcnt is waited on explicitly (wait_tiles).
__device__ __forceinline__ void dma16(const uint8_t *sbase, uint32_t voff, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(sbase), "s"(lds)
      : "memory");
}

// Hides a uniform value from loop-invariant code motion: addresses derived
// from it are formed right where they are used instead of being hoisted
// (dozens of per-instruction DMA addresses would otherwise occupy SGPRs).
template <class T>
__device__ __forceinline__ T fresh(T x) {
  asm volatile("" : "+s"(x));
  return x;
}
// Per-lane counterpart: values derived from it after the hot loop are not
// computed before the loop (and then kept, or spilled, across it).
__device__ __forceinline__ int vfresh(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Block-wide flags and per-row floats in LDS, accessed through asm like
// the rest of the kernel's LDS traffic.
__device__ __forceinline__ void ds_w32(uint32_t addr, uint32_t v) {
  asm volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v));
}
__device__ __forceinline__ uint32_t ds_r32(uint32_t addr) {
  uint32_t r;
  asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}
__device__ __forceinline__ void arrived32(uint32_t &x) { asm volatile("" : "+v"(x)); }


}  // namespace pipe
}  // namespace qmla

// common.hpp -- shared plumbing of libqmla: error reporting, HIP checks,
// bf16 helpers and vector types for gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "qmla.h"

namespace qmla {

// Per-thread message of the last failed call (qmla_last_error).
void set_error_msg(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
const char *error_msg();
void clear_error();

inline qmla_status fail(qmla_status s, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
inline qmla_status fail(qmla_status s, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  set_error_msg("%s: %s", qmla_status_string(s), buf);
  return s;
}

// Wraps a HIP call: on failure records the message and returns QMLA_ERR_HIP
// (QMLA_ERR_OOM for allocation failures) from the enclosing function.
#define QMLA_HIP(call)                                                                     \
  do {                                                                                     \
    hipError_t e_ = (call);                                                                \
    if (e_ != hipSuccess) {                                                                \
      (void)hipGetLastError();                                                             \
      return ::qmla::fail(e_ == hipErrorOutOfMemory ? QMLA_ERR_OOM : QMLA_ERR_HIP,         \
                          "%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, \
                          __LINE__);                                                       \
    }                                                                                      \
  } while (0)

// Checks the launch that was just enqueued.
#define QMLA_LAUNCH_CHECK(name)                                                           \
  do {                                                                                    \
    hipError_t e_ = hipGetLastError();                                                    \
    if (e_ != hipSuccess)                                                                 \
      return ::qmla::fail(QMLA_ERR_HIP, "launch of %s failed: %s", name,                  \
                          hipGetErrorString(e_));                                         \
  } while (0)

#define QMLA_REQUIRE(cond, status, ...)               \
  do {                                                \
    if (!(cond)) return ::qmla::fail(status, __VA_ARGS__); \
  } while (0)

#define QMLA_TRY(expr)                 \
  do {                                 \
    qmla_status s_ = (expr);           \
    if (s_ != QMLA_OK) return s_;      \
  } while (0)

inline hipStream_t as_stream(qmla_stream s) { return reinterpret_cast<hipStream_t>(s); }

// Number of compute units of the current device (cached per device).
int device_cu_count();

// Raises the dynamic LDS limit of kernel `fn` on the current device to at
// least `bytes`; the attribute call is made once per (kernel, device).
qmla_status ensure_dynamic_lds(const void *fn, size_t bytes);

// ------------------------------------------------------------- device side

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// f32 -> bf16 bits, round to nearest even, NaN kept quiet.
__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__host__ __device__ inline float bf16_bits_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}

// Two f32 -> packed bf16x2 (low half = a), round to nearest even.
__device__ inline uint32_t pack_bf16x2(float a, float b) {
  return static_cast<uint32_t>(f32_to_bf16_bits(a)) |
         (static_cast<uint32_t>(f32_to_bf16_bits(b)) << 16);
}

// cos(ang) * mscale and sin(ang) * mscale of a RoPE angle (src/model.rs:
// 63-64): one shared argument reduction for both.
__device__ __forceinline__ void rope_cs(float ang, float mscale, float &cs, float &sn) {
  float s, c;
  sincosf(ang, &s, &c);
  cs = c * mscale;
  sn = s * mscale;
}

constexpr int kWave = 64;

// Combines a value with the one held by lane (l ^ 32): returns own and
// partner value as (r0, r1) in some order -- callers reduce the pair with a
// symmetric op (max, +).  v_permlane32_swap a, b swaps a[32:63] with
// b[0:31]; with a = b = x, lanes 0-31 end with (x, x[l+32]) and lanes 32-63
// with (x[l-32], x).  Issued through inline asm: this compiler's
// __builtin_amdgcn_permlane32_swap returns the first result for both halves
// of its pair in some contexts (observed in generated code), so it is not
// used.  The s_nop covers the VALU-write -> permlane-read hazard.
__device__ __forceinline__ void xor32_pair(float x, float &r0, float &r1) {
  float a = x, b = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  r0 = a;
  r1 = b;
}

__device__ __forceinline__ float xor32_max(float x) {
  float a, b;
  xor32_pair(x, a, b);
  return fmaxf(a, b);
}

__device__ __forceinline__ float xor32_sum(float x) {
  float a, b;
  xor32_pair(x, a, b);
  return a + b;
}

}  // namespace qmla

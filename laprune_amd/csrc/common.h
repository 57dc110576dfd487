// common.h — shared helpers for the gfx950 retrieval-path kernels and the
// C ABI: thread-local error state, argument checks, fp16/bf16 bit helpers,
// cached device facts.  Everything is written for wave64 CDNA (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>
#include <cstdio>
#include <cstdarg>

#include "../../include/laprune_hip.h"

namespace lap {

// lap_row_plan as seen by kernels: kPlanInts int32 fields per sequence, in
// declaration order (t_codes, t_total, cand_start, cand_end, k, sink,
// tail_start, tail_count).
constexpr int kPlanInts = 8;
static_assert(sizeof(lap_row_plan) == kPlanInts * sizeof(int32_t), "lap_row_plan layout");

// ---------------------------------------------------------------- errors
void set_error(const char* fmt, ...);
void clear_error();

// Return LAP_ERR_INVALID with a formatted message when cond is false.
#define LAP_CHECK(cond, ...)                                                  \
  do {                                                                        \
    if (!(cond)) {                                                            \
      ::lap::set_error(__VA_ARGS__);                                          \
      return LAP_ERR_INVALID;                                                 \
    }                                                                         \
  } while (0)

#define LAP_CHECK_CODE(cond, code, ...)                                       \
  do {                                                                        \
    if (!(cond)) {                                                            \
      ::lap::set_error(__VA_ARGS__);                                          \
      return (code);                                                          \
    }                                                                         \
  } while (0)

// Check a HIP call; on failure record "<what>: <hip error>".
#define LAP_HIP(call, what)                                                   \
  do {                                                                        \
    hipError_t e__ = (call);                                                  \
    if (e__ != hipSuccess) {                                                  \
      ::lap::set_error("%s: %s", (what), hipGetErrorString(e__));             \
      return LAP_ERR_HIP;                                                     \
    }                                                                         \
  } while (0)

// After a launch: surface launch-configuration errors immediately (does not
// synchronise).
#define LAP_LAUNCH_CHECK(what)                                                \
  do {                                                                        \
    hipError_t e__ = hipGetLastError();                                       \
    if (e__ != hipSuccess) {                                                  \
      ::lap::set_error("%s launch: %s", (what), hipGetErrorString(e__));      \
      return LAP_ERR_HIP;                                                     \
    }                                                                         \
  } while (0)

inline hipStream_t as_stream(lap_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------- device
struct DevInfo {
  int cu_count = 0;
  int lds_per_block = 0;
  int wave_size = 0;
};
// Facts of the current device, queried once per device.
int device_info(DevInfo* out);

inline int dtype_size(int dt) {
  switch (dt) {
    case LAP_DTYPE_F32: return 4;
    case LAP_DTYPE_F16: return 2;
    case LAP_DTYPE_BF16: return 2;
    case LAP_DTYPE_U8: return 1;
    case LAP_DTYPE_I8: return 1;
    case LAP_DTYPE_I32: return 4;
    case LAP_DTYPE_I64: return 8;
    default: return 0;
  }
}

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// ------------------------------------------------- fp16 / bf16 bit helpers
// fp16 bits -> fp32 (exact).
__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
// fp32 -> fp16 bits, round to nearest even (v_cvt_f16_f32, default mode),
// from the fp32 value as rounded.  The empty asm keeps the compiler from
// folding the instruction that produced f into the conversion: it turns
// fp16(fmaf(a, b, c)) into v_fma_mixlo_f16, which rounds the exact result to
// fp16 once, and so differs from fp16(fp32(a * b + c)) where the fp32
// rounding lands on an fp16 midpoint.
__device__ __forceinline__ uint16_t f2h(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
// bf16 bits -> fp32 (exact: the bf16 pattern is the high half of the fp32).
__device__ __forceinline__ float bf2f(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}
// fp32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Load one element of dtype dt (f32/f16/bf16) as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dt) {
  if (dt == LAP_DTYPE_F32) return static_cast<const float*>(p)[i];
  uint16_t v = static_cast<const uint16_t*>(p)[i];
  return dt == LAP_DTYPE_F16 ? h2f(v) : bf2f(v);
}

// Orderable 16-bit key of fp16 / bf16 bits b: larger value -> larger key;
// -0 and +0 map to the same key.  Written with selects (no branches), as it
// runs once or four times per scored token.
__device__ __forceinline__ uint32_t orderable16(uint32_t b) {
  b = (b & 0x7fffu) == 0 ? 0u : b;
  return b ^ ((b & 0x8000u) ? 0xffffu : 0x8000u);
}
// Orderable key of a fp16 score.
__device__ __forceinline__ uint32_t f16_key(uint16_t h) { return orderable16(h); }
// Orderable key of bf16(fp16 score) (the model-dtype cast before top-k): the
// f2bf rounding of the exact fp32 value of h, NaN kept quiet.
__device__ __forceinline__ uint32_t bf16_key_of_f16(uint16_t h) {
  const uint32_t u = __builtin_bit_cast(uint32_t, h2f(h));
  const bool nan = (u & 0x7fffffffu) > 0x7f800000u;
  const uint32_t b = nan ? ((u >> 16) | 0x40u) : ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  return orderable16(b);
}

// Exact fp32 accumulate of an fp16 value: acc + (float)h with one rounding.
// Written as fma(fpext(h), fpext(one), acc) so gfx950 issues a single
// v_fma_mix_f32; `one` must be a runtime fp16 1.0 (a literal would be folded
// into cvt + add).
__device__ __forceinline__ float acc_f16(float acc, _Float16 h, _Float16 one) {
  return __builtin_fmaf((float)h, (float)one, acc);
}

// ---------------------------------------------------------- wave helpers
__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Workgroup barrier that orders LDS only.  __syncthreads() is a fence over
// all address spaces, which on gfx9 waits for every outstanding global load
// (vmcnt(0)) before the barrier and so cancels any prefetch in flight; this
// barrier waits only for the LDS counter, letting global loads stay in
// flight across it.  Use it only where no global-memory ordering between the
// threads of the workgroup is needed.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace lap

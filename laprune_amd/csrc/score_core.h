// score_core.h — the G = 4 scorer's inner pieces, shared by the scorer
// kernels (score.hip) and the fused decode step (step.hip).
#pragma once

#include "common.h"

namespace lap {
namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

constexpr int kG = 4, kM = 32, kK = 256;
constexpr int kLutBytes = kG * kM * kK * 2;  // 65536

// Level-1 histograms in LDS: HC copies per selection row, at a pitch of 257
// words so that the copies of one bin sit in different banks; lane l adds to
// copy l % HC.  Keys of nearby scores share a few high bytes, and the LDS
// serialises atomics that a wave aims at one address.
constexpr int kHPitch = 257;
template <int HC>
using HistRows = uint32_t (*)[HC * kHPitch];

// Byte j of code word w times 8 (the table offset of that code within its
// codebook's 2 KiB slice), one SDWA shift: the compiler extracts bytes 1-3
// this way by itself but byte 0 with a shift and a mask.  `three` holds 3 in
// a VGPR (SDWA takes no literal operand).
template <int J>
__device__ __forceinline__ uint32_t code_off(uint32_t w, uint32_t three) {
  uint32_t r;
  if constexpr (J == 0)
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
        : "=v"(r) : "v"(three), "v"(w));
  else if constexpr (J == 1)
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
        : "=v"(r) : "v"(three), "v"(w));
  else if constexpr (J == 2)
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
        : "=v"(r) : "v"(three), "v"(w));
  else
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
        : "=v"(r) : "v"(three), "v"(w));
  return r;
}

// Accumulate one token's 32 lookups into four fp32 head sums.
__device__ __forceinline__ void score_token(const char* __restrict__ lds, const uint4 c0,
                                            const uint4 c1, _Float16 one, float& a0,
                                            float& a1, float& a2, float& a3) {
  const uint32_t w[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  uint32_t three = 3u;
  asm("" : "+v"(three));
#pragma unroll
  for (int m = 0; m < kM; ++m) {
    uint32_t off;
    switch (m & 3) {
      case 0: off = code_off<0>(w[m >> 2], three); break;
      case 1: off = code_off<1>(w[m >> 2], three); break;
      case 2: off = code_off<2>(w[m >> 2], three); break;
      default: off = code_off<3>(w[m >> 2], three); break;
    }
    const half4_t v = *reinterpret_cast<const half4_t*>(lds + m * (kK * kG * 2) + off);
    a0 = acc_f16(a0, v.x, one);
    a1 = acc_f16(a1, v.y, one);
    a2 = acc_f16(a2, v.z, one);
    a3 = acc_f16(a3, v.w, one);
  }
}

// The loads are issued from inline asm because their order is the point and
// the compiler may reorder independent loads; every loaded value is tied to
// the s_waitcnt that covers it, so no instruction reads it early.  A wait
// for n outstanding operations is safe with stores in flight too: stores
// only add to the count, which makes the wait longer, never shorter.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 gload16_ordered(const void* p) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p));
  return v;
}
// The same load marked non-temporal: code rows are read once per launch, and
// the hint keeps the stream from displacing what the caches hold for longer
// (measured on MI355X: the C2 scorer 0.3 us faster per launch).
__device__ __forceinline__ u32x4 gload16_stream(const void* p) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(v) : "v"(p));
  return v;
}

// Wave priority for stage j of TOK: the stages still ahead, at most 3.  A
// SIMD serves its waves oldest first, so without it some waves finish their
// last stage well before others and the table lookups of the last stage
// run on a few waves with the LDS half idle; lowering a wave's priority as
// it advances keeps the waves of a workgroup within about one stage.
__device__ __forceinline__ void stage_prio(int j, int TOK) {
  const int p = TOK - 1 - j;
  if (p >= 3) __builtin_amdgcn_s_setprio(3);
  else if (p == 2) __builtin_amdgcn_s_setprio(2);
  else if (p == 1) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

template <int N>
__device__ __forceinline__ void vmw1(u32x4& a) {
  asm volatile("s_waitcnt vmcnt(%1)" : "+v"(a) : "n"(N));
}
template <int N>
__device__ __forceinline__ void vmw2(u32x4& a, u32x4& b) {
  asm volatile("s_waitcnt vmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N));
}
// Wait until at most n vector-memory operations are outstanding; n is a
// compile-time constant after unrolling, so the switch folds away.
__device__ __forceinline__ void vm_wait(int n, u32x4& a) {
  switch (n) {
#define LAP_VW(N) case N: vmw1<N>(a); break;
    LAP_VW(0) LAP_VW(1) LAP_VW(2) LAP_VW(3) LAP_VW(4) LAP_VW(5) LAP_VW(6) LAP_VW(7)
    LAP_VW(8) LAP_VW(9) LAP_VW(10) LAP_VW(11) LAP_VW(12) LAP_VW(13) LAP_VW(14) LAP_VW(15)
    LAP_VW(16) LAP_VW(17) LAP_VW(18) LAP_VW(19) LAP_VW(20) LAP_VW(21) LAP_VW(22) LAP_VW(23)
#undef LAP_VW
    default: vmw1<0>(a);
  }
}
__device__ __forceinline__ void vm_wait(int n, u32x4& a, u32x4& b) {
  switch (n) {
#define LAP_VW(N) case N: vmw2<N>(a, b); break;
    LAP_VW(0) LAP_VW(2) LAP_VW(4) LAP_VW(6) LAP_VW(8) LAP_VW(10) LAP_VW(12) LAP_VW(14)
    LAP_VW(16)
#undef LAP_VW
    default: vmw2<0>(a, b);
  }
}

template <int N>
__device__ __forceinline__ void vmw4(u32x4& a, u32x4& b, u32x4& c, u32x4& d) {
  asm volatile("s_waitcnt vmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N));
}
__device__ __forceinline__ void vm_wait(int n, u32x4& a, u32x4& b, u32x4& c, u32x4& d) {
  switch (n) {
#define LAP_VW(N) case N: vmw4<N>(a, b, c, d); break;
    LAP_VW(0) LAP_VW(1) LAP_VW(2) LAP_VW(3) LAP_VW(4) LAP_VW(5) LAP_VW(6) LAP_VW(7)
    LAP_VW(8) LAP_VW(9) LAP_VW(10) LAP_VW(11) LAP_VW(12) LAP_VW(13) LAP_VW(14) LAP_VW(15)
    LAP_VW(16) LAP_VW(17) LAP_VW(18) LAP_VW(19) LAP_VW(20) LAP_VW(21) LAP_VW(22) LAP_VW(23)
#undef LAP_VW
    default: vmw4<0>(a, b, c, d);
  }
}

__device__ __forceinline__ uint4 as_uint4(const u32x4 v) { return make_uint4(v.x, v.y, v.z, v.w); }

// Entries k0 .. k0+7 of one (m, k-block) for the four heads of a KV group,
// from the reference layout (one u32x4 of 8 fp16 per head), as the four
// uint4 of the [M][K][4] table: entry k = (h0, h1 | h2, h3) in 8 bytes.
__device__ __forceinline__ void interleave_heads(const u32x4& h0, const u32x4& h1,
                                                 const u32x4& h2, const u32x4& h3,
                                                 uint4* __restrict__ dst) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t a = h0[q], b = h1[q], c = h2[q], d = h3[q];
    // even entry: low halves; odd entry: high halves
    dst[q] = make_uint4(__builtin_amdgcn_perm(b, a, 0x05040100u),
                        __builtin_amdgcn_perm(d, c, 0x05040100u),
                        __builtin_amdgcn_perm(b, a, 0x07060302u),
                        __builtin_amdgcn_perm(d, c, 0x07060302u));
  }
}

}  // namespace
}  // namespace lap

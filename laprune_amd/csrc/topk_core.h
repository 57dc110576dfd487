// topk_core.h — wave and workgroup scans and the radix bin pick, shared
// by the top-k kernels (topk.hip) and the fused decode step (step.hip).
#pragma once

#include "common.h"

namespace lap {
namespace {

// Inclusive prefix sum over the 64 lanes of a wave (DPP row shifts, then the
// row broadcasts of lanes 15 and 31).
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t x) {
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, true);  // row_shr:1
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, true);  // row_shr:2
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, true);  // row_shr:4
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, true);  // row_shr:8
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Suffix sums S(i) = sum_{j>=i} h[j] over 256 LDS bins (waves 0..3 scan the
// reversed bins), then the unique bin b with S(b) >= target > S(b+1).
// s_res = {b, S(b+1)}; every thread of the block synchronises.  target must
// satisfy 1 <= target <= S(0); the block has at least 256 threads.
[[maybe_unused]] __device__ void select_bin(const uint32_t* s_h, uint32_t target, uint32_t* s_wsum,
                                            uint32_t* s_res) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t x = 0, h = 0;
  if (wave < 4) {
    h = s_h[255 - tid];
    x = wave_inclusive_scan(h);
    if (lane == 63) s_wsum[wave] = x;
  }
  __syncthreads();
  if (wave < 4) {
    uint32_t add = 0;
    for (int w = 0; w < wave; ++w) add += s_wsum[w];
    const uint32_t S_i = x + add;  // keys in bins >= 255 - tid
    const uint32_t S_next = S_i - h;
    if (S_i >= target && S_next < target) {
      s_res[0] = 255 - tid;
      s_res[1] = S_next;
    }
  }
  __syncthreads();
}

// Exclusive prefix sum over the TH threads of the block; returns the
// thread's prefix and writes the block total to *total.
template <int TH>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t x, uint32_t* s_wsum,
                                                         uint32_t* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t inc = wave_inclusive_scan(x);
  if (lane == 63) s_wsum[wave] = inc;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < TH / 64; ++w) {
    const uint32_t v = s_wsum[w];
    before += w < wave ? v : 0u;
    all += v;
  }
  __syncthreads();
  *total = all;
  return before + inc - x;
}

}  // namespace
}  // namespace lap

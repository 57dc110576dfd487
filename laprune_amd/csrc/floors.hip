// floors.hip — measurement kernels for the fused scorer's floors.
//
// They have no counterpart in the reference and are not on the retrieval
// path: bench.py times them next to score_g4p_kernel<1024, 4, 1> to show what
// its launch shape costs before any scoring.
//   * floor_empty_kernel: the scorer's grid, workgroup size and LDS
//     footprint, no work (dispatch and drain of 1024-thread workgroups that
//     each hold 68 KiB of LDS).
//   * floor_stream_kernel<AHEAD>: the scorer's data movement without its
//     lookups and adds.  Workgroup i takes KV row i % R and 4096 consecutive
//     tokens of it; thread tid reads its 64 KiB table slice (the GMKG table of
//     that row) into LDS, then the 32-byte code rows of tokens
//     t0 + j * 1024 + tid for j < 4, with AHEAD stages in flight (1: the
//     scorer's schedule; 4: every stage requested up front), through the same
//     ordered loads.  Everything read is XOR-folded into one word per
//     workgroup, so no load is dead and a test can check the result.
#include "common.h"
#include "score_core.h"

namespace lap {
namespace {

constexpr int kFloorTH = 1024, kFloorTok = 4;
constexpr int kFloorChunk = kFloorTH * kFloorTok;
constexpr int kFloorHist = 4 * kHPitch;  // the scorer's level-1 histogram words

__global__ __launch_bounds__(kFloorTH) void floor_empty_kernel(uint32_t* sink, int flag) {
  __shared__ uint4 s_lut[kLutBytes / 16];
  __shared__ uint32_t s_hist[kFloorHist];
  // flag is 0 at run time; the stores keep the LDS allocation in the kernel
  if (flag) {
    s_lut[threadIdx.x] = make_uint4(flag, 0, 0, 0);
    s_hist[threadIdx.x] = flag;
    __syncthreads();
    sink[threadIdx.x] = s_lut[(threadIdx.x + 1) % kFloorTH].x + s_hist[(threadIdx.x + 7) % kFloorTH];
  }
}

template <int AHEAD>
__global__ __launch_bounds__(kFloorTH) void floor_stream_kernel(const uint16_t* __restrict__ lut,
                                                                const uint8_t* __restrict__ codes,
                                                                int64_t cs_r, int64_t cs_t, int R,
                                                                int T, uint32_t* __restrict__ out) {
  constexpr int kFill = kLutBytes / 16 / kFloorTH;  // 4 table uint4s per thread
  static_assert(kFill + 2 * AHEAD <= 23 && 2 * AHEAD <= 16, "vmcnt range");
  __shared__ __attribute__((aligned(16))) uint4 s_lut[kLutBytes / 16];
  __shared__ uint32_t s_x[kFloorTH / 64];
  const int r = blockIdx.x % R, chunk = blockIdx.x / R, tid = threadIdx.x;
  const int t0 = chunk * kFloorChunk;
  const int t1 = min(T, t0 + kFloorChunk);  // > t0 by the grid

  const uint4* src = reinterpret_cast<const uint4*>(lut + (int64_t)r * (kLutBytes / 2));
  u32x4 f[kFill];
#pragma unroll
  for (int i = 0; i < kFill; ++i) f[i] = gload16_ordered(src + i * kFloorTH + tid);
  const uint8_t* crow = codes + (int64_t)r * cs_r;
  u32x4 c[kFloorTok][2];
  auto request = [&](int j) {
    const int t = min(t0 + j * kFloorTH + tid, t1 - 1);
    const uint8_t* p = crow + (int64_t)t * cs_t;
    c[j][0] = gload16_ordered(p);
    c[j][1] = gload16_ordered(p + 16);
  };
#pragma unroll
  for (int j = 0; j < AHEAD; ++j) request(j);
#pragma unroll
  for (int i = 0; i < kFill; ++i) {
    vm_wait(kFill - 1 - i + 2 * AHEAD, f[i]);
    s_lut[i * kFloorTH + tid] = as_uint4(f[i]);
  }
  lds_barrier();

  uint32_t x = 0;
#pragma unroll
  for (int j = 0; j < kFloorTok; ++j) {
    const int later = (j + AHEAD - 1 < kFloorTok - 1 ? j + AHEAD - 1 : kFloorTok - 1) - j;
    vm_wait(2 * later, c[j][0], c[j][1]);
    if (j + AHEAD < kFloorTok) request(j + AHEAD);
    x ^= c[j][0].x ^ c[j][0].y ^ c[j][0].z ^ c[j][0].w ^ c[j][1].x ^ c[j][1].y ^ c[j][1].z ^
         c[j][1].w;
  }
  // the table as read back from LDS (another thread's slice)
#pragma unroll
  for (int i = 0; i < kFill; ++i) {
    const uint4 v = s_lut[i * kFloorTH + (tid ^ 1)];
    x ^= v.x ^ v.y ^ v.z ^ v.w;
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) x ^= (uint32_t)__shfl_xor((int)x, d, 64);
  if ((tid & 63) == 0) s_x[tid >> 6] = x;
  __syncthreads();
  if (tid == 0) {
    uint32_t y = 0;
#pragma unroll
    for (int w = 0; w < kFloorTH / 64; ++w) y ^= s_x[w];
    out[blockIdx.x] = y;
  }
}

}  // namespace
}  // namespace lap

extern "C" int lap_floor_empty(int R, int T, lap_stream_t stream) {
  using namespace lap;
  clear_error();
  LAP_CHECK(R > 0 && T > 0, "lap_floor_empty: R and T must be positive");
  const int64_t grid = (int64_t)R * ((T + kFloorChunk - 1) / kFloorChunk);
  LAP_CHECK(grid <= (1 << 30), "lap_floor_empty: grid too large");
  hipLaunchKernelGGL(floor_empty_kernel, dim3((unsigned)grid), dim3(kFloorTH), 0,
                     as_stream(stream), nullptr, 0);
  LAP_LAUNCH_CHECK("floor_empty_kernel");
  return LAP_OK;
}

extern "C" int lap_floor_stream(const void* lut, const void* codes, int64_t cs_r, int64_t cs_t,
                                int R, int T, int ahead, uint32_t* out, lap_stream_t stream) {
  using namespace lap;
  clear_error();
  LAP_CHECK(lut && codes && out, "lap_floor_stream: null pointer");
  LAP_CHECK(R > 0 && T > 0, "lap_floor_stream: R and T must be positive");
  LAP_CHECK(ahead == 1 || ahead == 4, "lap_floor_stream: ahead must be 1 or 4 (got %d)", ahead);
  LAP_CHECK(cs_t >= 32 && cs_r >= 0, "lap_floor_stream: code rows are 32 bytes apart or more");
  LAP_CHECK(reinterpret_cast<uintptr_t>(codes) % 16 == 0 && cs_t % 16 == 0 && cs_r % 16 == 0 &&
                reinterpret_cast<uintptr_t>(lut) % 16 == 0,
            "lap_floor_stream: code rows and the table must be 16-byte aligned");
  const int64_t grid = (int64_t)R * ((T + kFloorChunk - 1) / kFloorChunk);
  LAP_CHECK(grid <= (1 << 30), "lap_floor_stream: grid too large");
  const uint16_t* l = static_cast<const uint16_t*>(lut);
  const uint8_t* c = static_cast<const uint8_t*>(codes);
  if (ahead == 1)
    hipLaunchKernelGGL(floor_stream_kernel<1>, dim3((unsigned)grid), dim3(kFloorTH), 0,
                       as_stream(stream), l, c, cs_r, cs_t, R, T, out);
  else
    hipLaunchKernelGGL(floor_stream_kernel<4>, dim3((unsigned)grid), dim3(kFloorTH), 0,
                       as_stream(stream), l, c, cs_r, cs_t, R, T, out);
  LAP_LAUNCH_CHECK("floor_stream_kernel");
  return LAP_OK;
}

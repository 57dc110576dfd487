// lut.hip — A1: per-query-head AQ lookup table.
//
//   lut[h, m, k] = fp16_rne( sum_d q[h, d] * C[m, k, d] )
//
// with the sum taken as one fp32 fmaf chain over d = 0..D-1 starting from 0
// (the order the CPU oracle restates).  The reference forms this LUT with a
// vendor GEMM (laprune/llm/aq_kv.py:681-682) or an fp32 einsum (:620).
//
// Work shape: a 256-thread workgroup owns a tile of 32 codebook rows
// (row = m*K + k) x 32 query heads; each thread produces 1 row x 4 heads.
// The codebook tile and the query tile are staged in LDS as fp32 with padded
// rows so that the eight row-pairs (and eight head-quads) read by one wave
// fall in distinct banks.  The interleaved layout [Hq/G][M][K][G] is written
// directly so the scorer can fill its LDS table with a linear copy.
#include "common.h"

namespace lap {
namespace {

constexpr int kRowsPerTile = 32;
constexpr int kHeadsPerTile = 32;
constexpr int kThreads = 256;

// Load 4 consecutive elements of dtype DT at element offset i as fp32.
template <int DT>
__device__ __forceinline__ float4 load4(const void* p, int64_t i) {
  if (DT == LAP_DTYPE_F32) return *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
  const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
  if (DT == LAP_DTYPE_F16)
    return make_float4(h2f(w.x & 0xffffu), h2f(w.x >> 16), h2f(w.y & 0xffffu), h2f(w.y >> 16));
  return make_float4(bf2f(w.x & 0xffffu), bf2f(w.x >> 16), bf2f(w.y & 0xffffu), bf2f(w.y >> 16));
}

// LDS layout (floats):
//   s_cb [32 rows][D + 4]                 rows padded by 4 banks
//   s_q  [8 quads][4 heads][D] + 4 per quad  quads padded by 4 banks
// so the 8 row reads and the 8 head-quad reads of one wave hit distinct banks.
template <int QDT, int CDT>
__global__ __launch_bounds__(kThreads) void lut_build_kernel(
    const void* __restrict__ q, int64_t q_row_stride,
    const void* __restrict__ cb, int Hq, int D, int MK, int G, int layout,
    uint16_t* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int ldc = D + 4;
  const int ldq = 4 * D + 4;
  float* s_cb = smem;                         // [32][ldc]
  float* s_q = smem + kRowsPerTile * ldc;     // [8][ldq]

  const int row0 = blockIdx.x * kRowsPerTile;
  const int head0 = blockIdx.y * kHeadsPerTile;
  const int tid = threadIdx.x;
  const int D4 = D / 4;

  // Stage both tiles with all loads issued before the LDS stores.
  {
    constexpr int kMaxIt = (kRowsPerTile * 256 / 4 + kThreads - 1) / kThreads;  // D <= 256
    float4 cv[kMaxIt], qv[kMaxIt];
    const int n4 = kRowsPerTile * D4;  // float4 slots per tile (same for q: 32 heads)
#pragma unroll
    for (int it = 0; it < kMaxIt; ++it) {
      const int i = tid + it * kThreads;
      cv[it] = make_float4(0.f, 0.f, 0.f, 0.f);
      qv[it] = cv[it];
      if (i < n4) {
        const int r = i / D4, d = (i - r * D4) * 4;
        if (row0 + r < MK) cv[it] = load4<CDT>(cb, (int64_t)(row0 + r) * D + d);
        if (head0 + r < Hq) qv[it] = load4<QDT>(q, (int64_t)(head0 + r) * q_row_stride + d);
      }
    }
#pragma unroll
    for (int it = 0; it < kMaxIt; ++it) {
      const int i = tid + it * kThreads;
      if (i < n4) {
        const int r = i / D4, d = (i - r * D4) * 4;
        *reinterpret_cast<float4*>(s_cb + r * ldc + d) = cv[it];
        *reinterpret_cast<float4*>(s_q + (r >> 2) * ldq + (r & 3) * D + d) = qv[it];
      }
    }
  }
  __syncthreads();

  const int hq4 = tid & 7;   // heads 4*hq4 .. 4*hq4+3 of the tile
  const int rr = tid >> 3;   // row rr of the tile
  const float* c0 = s_cb + rr * ldc;
  const float* qa = s_q + hq4 * ldq;

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  // One fmaf chain over d per output, d ascending.
  for (int d = 0; d < D; d += 4) {
    const float4 x = *reinterpret_cast<const float4*>(c0 + d);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const float4 qv = *reinterpret_cast<const float4*>(qa + h * D + d);
      acc[h] = __builtin_fmaf(qv.x, x.x, acc[h]);
      acc[h] = __builtin_fmaf(qv.y, x.y, acc[h]);
      acc[h] = __builtin_fmaf(qv.z, x.z, acc[h]);
      acc[h] = __builtin_fmaf(qv.w, x.w, acc[h]);
    }
  }

  const int row = row0 + rr;
  const int headA = head0 + 4 * hq4;
  if (row >= MK) return;
  if (layout == LAP_LUT_GMKG && G == 4 && headA + 3 < Hq) {
    // Four heads of one KV group for one row: 8 contiguous bytes.
    const int hkv = headA >> 2;
    const uint32_t w0 = (uint32_t)f2h(acc[0]) | ((uint32_t)f2h(acc[1]) << 16);
    const uint32_t w1 = (uint32_t)f2h(acc[2]) | ((uint32_t)f2h(acc[3]) << 16);
    *reinterpret_cast<uint2*>(out + ((int64_t)hkv * MK + row) * 4) = make_uint2(w0, w1);
    return;
  }
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const int head = headA + h;
    if (head >= Hq) continue;
    int64_t idx;
    if (layout == LAP_LUT_HMK) idx = (int64_t)head * MK + row;
    else idx = ((int64_t)(head / G) * MK + row) * G + (head % G);
    out[idx] = f2h(acc[h]);
  }
}

size_t lut_smem_bytes(int D) {
  return ((size_t)kRowsPerTile * (D + 4) + (size_t)8 * (4 * D + 4)) * sizeof(float);
}

template <int QDT>
hipError_t launch_lut(const void* q, int64_t qs, const void* cb, int cb_dtype, int Hq,
                      int D, int MK, int G, int layout, uint16_t* out, hipStream_t st) {
  dim3 grid((MK + kRowsPerTile - 1) / kRowsPerTile, (Hq + kHeadsPerTile - 1) / kHeadsPerTile);
  const size_t smem = lut_smem_bytes(D);
  if (cb_dtype == LAP_DTYPE_F32) {
    hipLaunchKernelGGL((lut_build_kernel<QDT, LAP_DTYPE_F32>), grid, dim3(kThreads), smem, st,
                       q, qs, cb, Hq, D, MK, G, layout, out);
  } else {
    hipLaunchKernelGGL((lut_build_kernel<QDT, LAP_DTYPE_F16>), grid, dim3(kThreads), smem, st,
                       q, qs, cb, Hq, D, MK, G, layout, out);
  }
  return hipGetLastError();
}

}  // namespace
}  // namespace lap

extern "C" int lap_lut_build(const void* q, int q_dtype, int64_t q_row_stride,
                             const void* codebooks, int cb_dtype, int Hq, int D, int M,
                             int K, int G, int layout, void* lut_out, lap_stream_t stream) {
  using namespace lap;
  clear_error();
  LAP_CHECK(q && codebooks && lut_out, "lap_lut_build: null pointer");
  LAP_CHECK(q_dtype == LAP_DTYPE_F32 || q_dtype == LAP_DTYPE_F16 || q_dtype == LAP_DTYPE_BF16,
            "lap_lut_build: q dtype must be f32/f16/bf16");
  LAP_CHECK(cb_dtype == LAP_DTYPE_F32 || cb_dtype == LAP_DTYPE_F16,
            "lap_lut_build: codebook dtype must be f32/f16");
  LAP_CHECK(Hq > 0 && M > 0 && K > 0 && D > 0, "lap_lut_build: sizes must be positive");
  LAP_CHECK(D % 4 == 0, "lap_lut_build: D must be a multiple of 4 (got %d)", D);
  LAP_CHECK_CODE(D <= 256, LAP_ERR_UNSUPPORTED, "lap_lut_build: D=%d > 256 unsupported", D);
  LAP_CHECK(q_row_stride >= D, "lap_lut_build: q row stride %lld < D", (long long)q_row_stride);
  LAP_CHECK(layout == LAP_LUT_HMK || layout == LAP_LUT_GMKG, "lap_lut_build: bad layout");
  if (layout == LAP_LUT_GMKG)
    LAP_CHECK(G > 0 && Hq % G == 0, "lap_lut_build: Hq=%d not divisible by G=%d", Hq, G);
  LAP_CHECK((int64_t)M * K <= (1 << 30), "lap_lut_build: M*K too large");
  DevInfo di;
  int ds = device_info(&di);
  if (ds != LAP_OK) return ds;
  const size_t smem = lut_smem_bytes(D);
  LAP_CHECK_CODE(smem <= (size_t)di.lds_per_block, LAP_ERR_UNSUPPORTED,
                 "lap_lut_build: D=%d needs %zu bytes of LDS", D, smem);
  hipError_t e;
  const int MK = M * K;
  uint16_t* out = static_cast<uint16_t*>(lut_out);
  hipStream_t st = as_stream(stream);
  switch (q_dtype) {
    case LAP_DTYPE_F32:
      e = launch_lut<LAP_DTYPE_F32>(q, q_row_stride, codebooks, cb_dtype, Hq, D, MK, G, layout, out, st);
      break;
    case LAP_DTYPE_F16:
      e = launch_lut<LAP_DTYPE_F16>(q, q_row_stride, codebooks, cb_dtype, Hq, D, MK, G, layout, out, st);
      break;
    default:
      e = launch_lut<LAP_DTYPE_BF16>(q, q_row_stride, codebooks, cb_dtype, Hq, D, MK, G, layout, out, st);
      break;
  }
  LAP_HIP(e, "lap_lut_build launch");
  return LAP_OK;
}

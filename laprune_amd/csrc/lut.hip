// lut.hip — A1: per-query-head AQ lookup table.
//
//   lut[h, m, k] = fp16_rne( sum_d q[h, d] * C[m, k, d] )
//
// with the sum taken as one fp32 fmaf chain over d = 0..D-1 starting from 0
// (the order the CPU oracle restates).  The reference forms this LUT with a
// vendor GEMM (laprune/llm/aq_kv.py:681-682) or an fp32 einsum (:620).
//
// Work shape: one lane per codebook row (row = m*K + k), four query heads per
// wave, 64 rows x 16 heads per workgroup (1024 waves at Hq = 32, M*K = 8192).
// The interleaved layout [Hq/G][M][K][G] is written directly so the scorer can
// fill its LDS table with a linear copy.
#include "common.h"

namespace lap {
namespace {

constexpr int kRows = 64;        // codebook rows per workgroup (one per lane)
constexpr int kHeadsPerWG = 16;  // query heads per workgroup (4 per wave)
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

// Workgroup = 64 codebook rows x 16 query heads; wave w owns heads
// head0 + 4w .. head0 + 4w + 3 and lane l owns row row0 + l, so each lane runs
// four independent fmaf chains over d.  The query slice is staged once in LDS
// as fp32 and read as wave-wide broadcasts (one address per instruction, no
// bank conflicts); the codebook row is read straight from L1/L2.
template <int QDT, int CDT>
__global__ __launch_bounds__(kThreads) void lut_build_kernel(
    const void* __restrict__ q, int64_t q_row_stride,
    const void* __restrict__ cb, int Hq, int D, int MK, int G, int layout,
    uint16_t* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) float s_q[];  // [16][D]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * kRows;
  const int head0 = blockIdx.y * kHeadsPerWG;
  const int D4 = D / 4;

  for (int i = tid; i < kHeadsPerWG * D4; i += kThreads) {
    const int h = i / D4, d = (i - h * D4) * 4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (head0 + h < Hq) v = load4<QDT>(q, (int64_t)(head0 + h) * q_row_stride + d);
    *reinterpret_cast<float4*>(s_q + h * D + d) = v;
  }
  __syncthreads();

  const int row = row0 + lane;
  const int rowc = row < MK ? row : MK - 1;  // clamped for the loads
  const float* qw = s_q + (4 * wave) * D;
  float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
#pragma unroll 4
  for (int d = 0; d < D; d += 4) {
    const float4 c = load4<CDT>(cb, (int64_t)rowc * D + d);
    const float4 q0 = *reinterpret_cast<const float4*>(qw + d);
    const float4 q1 = *reinterpret_cast<const float4*>(qw + D + d);
    const float4 q2 = *reinterpret_cast<const float4*>(qw + 2 * D + d);
    const float4 q3 = *reinterpret_cast<const float4*>(qw + 3 * D + d);
    acc0 = __builtin_fmaf(q0.x, c.x, acc0);
    acc1 = __builtin_fmaf(q1.x, c.x, acc1);
    acc2 = __builtin_fmaf(q2.x, c.x, acc2);
    acc3 = __builtin_fmaf(q3.x, c.x, acc3);
    acc0 = __builtin_fmaf(q0.y, c.y, acc0);
    acc1 = __builtin_fmaf(q1.y, c.y, acc1);
    acc2 = __builtin_fmaf(q2.y, c.y, acc2);
    acc3 = __builtin_fmaf(q3.y, c.y, acc3);
    acc0 = __builtin_fmaf(q0.z, c.z, acc0);
    acc1 = __builtin_fmaf(q1.z, c.z, acc1);
    acc2 = __builtin_fmaf(q2.z, c.z, acc2);
    acc3 = __builtin_fmaf(q3.z, c.z, acc3);
    acc0 = __builtin_fmaf(q0.w, c.w, acc0);
    acc1 = __builtin_fmaf(q1.w, c.w, acc1);
    acc2 = __builtin_fmaf(q2.w, c.w, acc2);
    acc3 = __builtin_fmaf(q3.w, c.w, acc3);
  }
  if (row >= MK) return;
  const int headA = head0 + 4 * wave;
  const float acc[4] = {acc0, acc1, acc2, acc3};
  if (layout == LAP_LUT_GMKG && G == 4 && headA + 3 < Hq) {
    // The four heads of one KV group for this row: 8 contiguous bytes; a
    // wave writes 512 contiguous bytes.
    const uint32_t w0 = (uint32_t)f2h(acc0) | ((uint32_t)f2h(acc1) << 16);
    const uint32_t w1 = (uint32_t)f2h(acc2) | ((uint32_t)f2h(acc3) << 16);
    *reinterpret_cast<uint2*>(out + ((int64_t)(headA >> 2) * MK + row) * 4) = make_uint2(w0, w1);
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

size_t lut_smem_bytes(int D) { return (size_t)kHeadsPerWG * D * sizeof(float); }

template <int QDT>
hipError_t launch_lut(const void* q, int64_t qs, const void* cb, int cb_dtype, int Hq,
                      int D, int MK, int G, int layout, uint16_t* out, hipStream_t st) {
  dim3 grid((MK + kRows - 1) / kRows, (Hq + kHeadsPerWG - 1) / kHeadsPerWG);
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

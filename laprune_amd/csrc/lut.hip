// lut.hip — A1: per-query-head AQ lookup table.
//
//   lut[h, m, k] = fp16_rne( sum_d q[h, d] * C[m, k, d] )
//
// with the sum taken as one fp32 fmaf chain over d = 0..D-1 starting from 0
// (the order the CPU oracle restates).  The reference forms this LUT with a
// vendor GEMM (laprune/llm/aq_kv.py:681-682) or an fp32 einsum (:620).
//
// Work shape: a 256-thread workgroup owns a tile of 64 codebook rows
// (row = m*K + k) x 32 query heads; each thread produces 2 rows x 4 heads.
// The codebook tile and the query tile are staged in LDS as fp32 with padded
// rows so that the eight row-pairs (and eight head-quads) read by one wave
// fall in distinct banks.  The interleaved layout [Hq/G][M][K][G] is written
// directly so the scorer can fill its LDS table with a linear copy.
#include "common.h"

namespace lap {
namespace {

constexpr int kRowsPerTile = 64;
constexpr int kHeadsPerTile = 32;
constexpr int kThreads = 256;

template <int QDT, int CDT>
__global__ __launch_bounds__(kThreads) void lut_build_kernel(
    const void* __restrict__ q, int64_t q_row_stride,
    const void* __restrict__ cb, int Hq, int D, int MK, int G, int layout,
    uint16_t* __restrict__ out) {
  extern __shared__ float smem[];
  const int ld = D + 4;  // padded row length (floats)
  float* s_cb = smem;                        // [64][ld]
  float* s_q = smem + kRowsPerTile * ld;     // [32][ld]

  const int row0 = blockIdx.x * kRowsPerTile;
  const int head0 = blockIdx.y * kHeadsPerTile;
  const int tid = threadIdx.x;

  // Stage the codebook tile (fp32) and the query tile (fp32).
  for (int i = tid; i < kRowsPerTile * D; i += kThreads) {
    const int r = i / D, d = i - r * D;
    const int row = row0 + r;
    float v = 0.f;
    if (row < MK) v = load_as_f32(cb, (int64_t)row * D + d, CDT);
    s_cb[r * ld + d] = v;
  }
  for (int i = tid; i < kHeadsPerTile * D; i += kThreads) {
    const int h = i / D, d = i - h * D;
    const int head = head0 + h;
    float v = 0.f;
    if (head < Hq) v = load_as_f32(q, (int64_t)head * q_row_stride + d, QDT);
    s_q[h * ld + d] = v;
  }
  __syncthreads();

  const int hq4 = tid & 7;    // heads 4*hq4 .. 4*hq4+3 of the tile
  const int rp = tid >> 3;    // rows 2*rp, 2*rp+1 of the tile
  const float* c0 = s_cb + (2 * rp) * ld;
  const float* c1 = c0 + ld;
  const float* qa = s_q + (4 * hq4) * ld;

  float acc[2][4];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int h = 0; h < 4; ++h) acc[r][h] = 0.f;

  // Sequential fmaf chain over d for each of the 8 outputs.
  for (int d = 0; d < D; d += 4) {
    const float4 x0 = *reinterpret_cast<const float4*>(c0 + d);
    const float4 x1 = *reinterpret_cast<const float4*>(c1 + d);
    float4 qv[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) qv[h] = *reinterpret_cast<const float4*>(qa + h * ld + d);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      acc[0][h] = __builtin_fmaf(qv[h].x, x0.x, acc[0][h]);
      acc[0][h] = __builtin_fmaf(qv[h].y, x0.y, acc[0][h]);
      acc[0][h] = __builtin_fmaf(qv[h].z, x0.z, acc[0][h]);
      acc[0][h] = __builtin_fmaf(qv[h].w, x0.w, acc[0][h]);
      acc[1][h] = __builtin_fmaf(qv[h].x, x1.x, acc[1][h]);
      acc[1][h] = __builtin_fmaf(qv[h].y, x1.y, acc[1][h]);
      acc[1][h] = __builtin_fmaf(qv[h].z, x1.z, acc[1][h]);
      acc[1][h] = __builtin_fmaf(qv[h].w, x1.w, acc[1][h]);
    }
  }

  const int rowA = row0 + 2 * rp;
  const int headA = head0 + 4 * hq4;
  if (layout == LAP_LUT_GMKG && G == 4 && headA + 3 < Hq && (headA & 3) == 0 &&
      rowA + 1 < MK) {
    // Four heads of one KV group for two consecutive rows: 16 contiguous bytes.
    const int hkv = headA >> 2;
    uint32_t w[4];
    w[0] = (uint32_t)f2h(acc[0][0]) | ((uint32_t)f2h(acc[0][1]) << 16);
    w[1] = (uint32_t)f2h(acc[0][2]) | ((uint32_t)f2h(acc[0][3]) << 16);
    w[2] = (uint32_t)f2h(acc[1][0]) | ((uint32_t)f2h(acc[1][1]) << 16);
    w[3] = (uint32_t)f2h(acc[1][2]) | ((uint32_t)f2h(acc[1][3]) << 16);
    uint4* dst = reinterpret_cast<uint4*>(out + ((int64_t)hkv * MK + rowA) * 4);
    *dst = make_uint4(w[0], w[1], w[2], w[3]);
    return;
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int row = rowA + r;
    if (row >= MK) continue;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int head = headA + h;
      if (head >= Hq) continue;
      int64_t idx;
      if (layout == LAP_LUT_HMK) {
        idx = (int64_t)head * MK + row;
      } else {
        idx = ((int64_t)(head / G) * MK + row) * G + (head % G);
      }
      out[idx] = f2h(acc[r][h]);
    }
  }
}

template <int QDT>
hipError_t launch_lut(const void* q, int64_t qs, const void* cb, int cb_dtype, int Hq,
                      int D, int MK, int G, int layout, uint16_t* out, hipStream_t st) {
  dim3 grid((MK + kRowsPerTile - 1) / kRowsPerTile, (Hq + kHeadsPerTile - 1) / kHeadsPerTile);
  const size_t smem = (size_t)(kRowsPerTile + kHeadsPerTile) * (D + 4) * sizeof(float);
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
  const size_t smem = (size_t)(kRowsPerTile + kHeadsPerTile) * (D + 4) * sizeof(float);
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

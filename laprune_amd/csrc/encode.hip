// encode.hip — A6: greedy additive-quantization encode of new keys.
//
// Contract (the fp32 greedy path of laprune/quantizer.py:346-355 with
// iters = 0, written out in an explicit order):
//   r = x
//   for m = 0..M-1:
//     rn     = dot16(r, r)
//     dist_k = (rn + cn[m,k]) - 2 * dot16(r, C[m,k])      k = 0..K-1
//     code_m = lowest k attaining min_k dist_k
//     r      = r - C[m, code_m]                            (elementwise fp32)
//   resid_norm = sqrtf(dot16(r, r))
// with cn[m,k] = dot16(C[m,k], C[m,k]) and
//   dot16(a, b): s_j = fmaf-chain over d = jL .. jL+L-1 from 0 (L = D/16),
//                then s_j += s_{j+w} for w = 8, 4, 2, 1; result s_0.
// The reference GPU kernel (aq_kernels/fused_linear_encode.cu:34-102) keeps
// an fp16 residual and an argmax of r.c - |c|^2/2; the fp32 path is the one
// followed here.
//
// lap_encode_prepare builds, once per codebook: Ct[m][d][k] (the codebook
// transposed so that lane-contiguous k is memory-contiguous) and cn[m][k].
// lap_encode_greedy: one wave per row; lane l owns entries k = 4l..4l+3 and
// keeps their 16 chain sums in registers while d streams through; the row's
// residual lives in LDS and is read as a broadcast.
#include "common.h"

namespace lap {
namespace {

struct Prep {
  float* ct;  // [M][D][K]
  float* cn;  // [M][K]
  size_t bytes;
};

Prep carve_prep(void* base, int M, int K, int D) {
  Prep p{};
  char* b = static_cast<char*>(base);
  size_t off = 0;
  p.ct = reinterpret_cast<float*>(b ? b + off : nullptr);
  off = align_up(off + (size_t)M * D * K * 4, 256);
  p.cn = reinterpret_cast<float*>(b ? b + off : nullptr);
  off = align_up(off + (size_t)M * K * 4, 256);
  p.bytes = off;
  return p;
}

// Fold 16 chain sums in the contract order.
__device__ __forceinline__ float fold16(float s[16]) {
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
    for (int j = 0; j < w; ++j) s[j] = s[j] + s[j + w];
  return s[0];
}

__global__ __launch_bounds__(256) void encode_prep_transpose(const float* __restrict__ cb,
                                                             int M, int K, int D,
                                                             float* __restrict__ ct) {
  __shared__ float tile[32][33];
  const int m = blockIdx.z;
  const int k0 = blockIdx.x * 32, d0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int i = ty; i < 32; i += 8) {
    const int k = k0 + i, d = d0 + tx;
    tile[i][tx] = (k < K && d < D) ? cb[((int64_t)m * K + k) * D + d] : 0.f;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int d = d0 + i, k = k0 + tx;
    if (k < K && d < D) ct[((int64_t)m * D + d) * K + k] = tile[tx][i];
  }
}

__global__ __launch_bounds__(256) void encode_prep_norms(const float* __restrict__ cb, int M,
                                                         int K, int D, float* __restrict__ cn) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= M * K) return;
  const float* row = cb + (int64_t)i * D;
  const int L = D / 16;
  float s[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    float a = 0.f;
    for (int t = 0; t < L; ++t) a = __builtin_fmaf(row[j * L + t], row[j * L + t], a);
    s[j] = a;
  }
  cn[i] = fold16(s);
}

// dot16(r, r) over a row held in LDS: lanes 0..15 each run one chain, the
// fold is an xor butterfly within 16 lanes (lane j < w pairs with j + w).
__device__ __forceinline__ float wave_self_dot16(const float* r, int D, int lane) {
  const int L = D / 16;
  const int j = lane & 15;
  float a = 0.f;
  for (int t = 0; t < L; ++t) {
    const float v = r[j * L + t];
    a = __builtin_fmaf(v, v, a);
  }
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1) a = a + __shfl_xor(a, w, 16);
  return __shfl(a, 0, 64);
}

template <int D>
__global__ __launch_bounds__(256) void encode_greedy_kernel(
    const float* __restrict__ x, int64_t x_rs, int N, const float* __restrict__ cb, int M,
    int K, const float* __restrict__ ct, const float* __restrict__ cn,
    uint8_t* __restrict__ codes, int64_t c_rs, float* __restrict__ rnorm) {
  constexpr int L = D / 16;
  __shared__ __attribute__((aligned(16))) float s_r[4][D];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + wave;
  const bool live = row < N;
  float* r = s_r[wave];
  for (int d = lane; d < D; d += 64) r[d] = live ? x[(int64_t)row * x_rs + d] : 0.f;
  __syncthreads();

  const int k0 = 4 * lane;
  const bool own = k0 < K;  // K % 4 == 0
  for (int m = 0; m < M; ++m) {
    const float rn = wave_self_dot16(r, D, lane);
    float acc[4][16];
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[e][j] = 0.f;
    const float* ctm = ct + (int64_t)m * D * K + k0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
#pragma unroll
      for (int t = 0; t < L; ++t) {
        const int d = j * L + t;
        const float rv = r[d];
        const float4 c = own ? *reinterpret_cast<const float4*>(ctm + (int64_t)d * K)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
        acc[0][j] = __builtin_fmaf(rv, c.x, acc[0][j]);
        acc[1][j] = __builtin_fmaf(rv, c.y, acc[1][j]);
        acc[2][j] = __builtin_fmaf(rv, c.z, acc[2][j]);
        acc[3][j] = __builtin_fmaf(rv, c.w, acc[3][j]);
      }
    }
    float best = INFINITY;
    int bk = 0x7fffffff;
    if (own) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float dot = fold16(acc[e]);
        const float dist = (rn + cn[(int64_t)m * K + k0 + e]) - 2.0f * dot;
        if (dist < best) {
          best = dist;
          bk = k0 + e;
        }
      }
    }
#pragma unroll
    for (int w = 32; w >= 1; w >>= 1) {
      const float ob = __shfl_xor(best, w, 64);
      const int ok = __shfl_xor(bk, w, 64);
      if (ob < best || (ob == best && ok < bk)) {
        best = ob;
        bk = ok;
      }
    }
    // No finite winner (all distances NaN): code 0, as the oracle's strict-<
    // scan from +inf leaves it.
    if (bk >= K) bk = 0;
    if (live && lane == 0) codes[(int64_t)row * c_rs + m] = (uint8_t)bk;
    const float* crow = cb + ((int64_t)m * K + bk) * D;
    for (int d = lane; d < D; d += 64) r[d] = r[d] - crow[d];
    __syncthreads();
  }
  const float rn = wave_self_dot16(r, D, lane);
  if (live && lane == 0 && rnorm) rnorm[row] = sqrtf(rn);
}

}  // namespace
}  // namespace lap

using namespace lap;

extern "C" int lap_encode_prep_size(int M, int K, int D, size_t* bytes) {
  clear_error();
  LAP_CHECK(bytes, "lap_encode_prep_size: null output");
  LAP_CHECK(M > 0 && K > 0 && D > 0, "lap_encode_prep_size: bad sizes");
  *bytes = carve_prep(nullptr, M, K, D).bytes;
  return LAP_OK;
}

extern "C" int lap_encode_prepare(const float* codebooks, int M, int K, int D, void* prep,
                                  size_t prep_bytes, lap_stream_t stream) {
  clear_error();
  LAP_CHECK(codebooks && prep, "lap_encode_prepare: null pointer");
  LAP_CHECK(M > 0 && K > 0 && D > 0, "lap_encode_prepare: bad sizes");
  LAP_CHECK(D % 16 == 0, "lap_encode_prepare: D=%d must be a multiple of 16", D);
  Prep p = carve_prep(prep, M, K, D);
  LAP_CHECK_CODE(prep_bytes >= p.bytes, LAP_ERR_WORKSPACE,
                 "lap_encode_prepare: prep buffer of %zu bytes needed", p.bytes);
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(encode_prep_transpose, dim3((K + 31) / 32, (D + 31) / 32, M), dim3(256), 0,
                     st, codebooks, M, K, D, p.ct);
  LAP_LAUNCH_CHECK("encode_prep_transpose");
  hipLaunchKernelGGL(encode_prep_norms, dim3((M * K + 255) / 256), dim3(256), 0, st, codebooks,
                     M, K, D, p.cn);
  LAP_LAUNCH_CHECK("encode_prep_norms");
  return LAP_OK;
}

extern "C" int lap_encode_greedy(const float* x, int64_t x_row_stride, int N, int D,
                                 const float* codebooks, int M, int K, const void* prep,
                                 size_t prep_bytes, uint8_t* codes_out, int64_t codes_row_stride,
                                 float* resid_norm, lap_stream_t stream) {
  clear_error();
  LAP_CHECK(x && codebooks && prep && codes_out, "lap_encode_greedy: null pointer");
  LAP_CHECK(N >= 0 && M > 0 && K > 0 && D > 0, "lap_encode_greedy: bad sizes");
  LAP_CHECK(K <= 256, "lap_encode_greedy: K=%d exceeds 256 (uint8 codes)", K);
  LAP_CHECK_CODE(K % 4 == 0, LAP_ERR_UNSUPPORTED, "lap_encode_greedy: K must be a multiple of 4");
  LAP_CHECK_CODE(D == 64 || D == 128 || D == 256, LAP_ERR_UNSUPPORTED,
                 "lap_encode_greedy: D=%d unsupported (64/128/256)", D);
  LAP_CHECK(x_row_stride >= D && codes_row_stride >= M, "lap_encode_greedy: bad row strides");
  Prep p = carve_prep(const_cast<void*>(prep), M, K, D);
  LAP_CHECK_CODE(prep_bytes >= p.bytes, LAP_ERR_WORKSPACE,
                 "lap_encode_greedy: prep buffer of %zu bytes needed", p.bytes);
  LAP_CHECK((reinterpret_cast<uintptr_t>(p.ct) & 15) == 0, "lap_encode_greedy: prep misaligned");
  if (N == 0) return LAP_OK;
  hipStream_t st = as_stream(stream);
  dim3 grid((N + 3) / 4);
#define LAP_ENC(D_)                                                                          \
  hipLaunchKernelGGL(encode_greedy_kernel<D_>, grid, dim3(256), 0, st, x, x_row_stride, N,   \
                     codebooks, M, K, p.ct, p.cn, codes_out, codes_row_stride, resid_norm)
  if (D == 64) LAP_ENC(64);
  else if (D == 128) LAP_ENC(128);
  else LAP_ENC(256);
#undef LAP_ENC
  LAP_LAUNCH_CHECK("encode_greedy_kernel");
  return LAP_OK;
}

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

#include <algorithm>
#include <cstdlib>
#include <cstring>

namespace lap {
namespace {

struct Prep {
  float* ct;       // [M][D][K]
  float* cn;       // [M][K]
  float* scn;      // [M][K] sqrtf(cn)
  uint16_t* frag;  // bf16 MFMA B fragments [M][K/16][D/16][64 lanes][4] (K % 16 == 0)
  uint16_t* frag4; // 4x4x4 B operands [M][ceil(K/64)][D/8][64 lanes][8] (K % 16 == 0)
  float4* c4;      // [M][D/4][K] float4: entry k's d = 4q .. 4q+3 (the exact kernel's rows)
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
  p.scn = reinterpret_cast<float*>(b ? b + off : nullptr);
  off = align_up(off + (size_t)M * K * 4, 256);
  p.frag = reinterpret_cast<uint16_t*>(b ? b + off : nullptr);
  if (K % 16 == 0) off = align_up(off + (size_t)M * K * D * 2, 256);
  p.frag4 = reinterpret_cast<uint16_t*>(b ? b + off : nullptr);
  if (K % 16 == 0) off = align_up(off + (size_t)M * ((K + 63) / 64) * 64 * D * 2, 256);
  p.c4 = reinterpret_cast<float4*>(b ? b + off : nullptr);
  off = align_up(off + (size_t)M * K * D * 4, 256);
  p.bytes = off;
  return p;
}

// Row addressing of an encode call.  Row i of the N rows is token
// t0 + i % L of segment s = i / L, and segment s is (b, h) = (s / Hs, s % Hs):
// a block of L consecutive tokens of every (batch, KV head) pair of a
// strided [B][H][T][D] key cache, and the same position in a strided
// [B][H][Tcap][M] code cache.  A plain [N][D] input is L = N, Hs = 1.
// With per-batch ranges (device [B][2] = t0_b, t1_b), segment s covers
// tokens t0_b + j for j < min(t1_b - t0_b, L); rows past that are not live.
struct RowMap {
  const void* x;
  int x_dtype;  // f32 / f16 / bf16 (widened exactly to fp32)
  int64_t x_sb, x_sh, x_st;
  uint8_t* codes;
  int64_t c_sb, c_sh, c_st;
  int L, Hs, t0;
  const int32_t* ranges;  // [B][2] or null
  int t_cap;              // with ranges: rows outside [0, t_cap) are not live
  __device__ __forceinline__ int64_t off(int i, int64_t sb, int64_t sh, int64_t st) const {
    const int sg = i / L, j = i - sg * L;
    const int b = sg / Hs, h = sg - b * Hs;
    const int t = (ranges ? ranges[2 * b] : t0) + j;
    return (int64_t)b * sb + (int64_t)h * sh + (int64_t)t * st;
  }
  __device__ __forceinline__ bool live(int i) const {
    if (!ranges) return true;
    const int sg = i / L, b = sg / Hs, j = i - sg * L;
    const int lo = ranges[2 * b], hi = min(ranges[2 * b + 1], t_cap);
    return lo >= 0 && lo + j < hi;
  }
  __device__ __forceinline__ float xval(int i, int d) const {
    return load_as_f32(x, off(i, x_sb, x_sh, x_st) + d, x_dtype);
  }
  __device__ __forceinline__ uint8_t* crow(int i) const { return codes + off(i, c_sb, c_sh, c_st); }
};

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

// c4[m][q][k] = (C[m,k,4q], .., C[m,k,4q+3]): lane k of a wave reads 16 bytes
// and the 64 lanes one contiguous kilobyte.
__global__ __launch_bounds__(256) void encode_prep_c4(const float* __restrict__ cb, int M, int K,
                                                      int D, float4* __restrict__ c4) {
  const int Q = D / 4;
  const int64_t n = (int64_t)M * Q * K;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int k = (int)(i % K);
    const int64_t mq = i / K;
    const int q = (int)(mq % Q), m = (int)(mq / Q);
    c4[i] = *reinterpret_cast<const float4*>(cb + ((int64_t)m * K + k) * D + 4 * q);
  }
}

__global__ __launch_bounds__(256) void encode_prep_norms(const float* __restrict__ cb, int M,
                                                         int K, int D, float* __restrict__ cn,
                                                         float* __restrict__ scn) {
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
  scn[i] = sqrtf(cn[i]);
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
    RowMap rm, int N, const float* __restrict__ cb, int M,
    int K, const float* __restrict__ ct, const float* __restrict__ cn,
    float* __restrict__ rnorm) {
  constexpr int L = D / 16;
  __shared__ __attribute__((aligned(16))) float s_r[4][D];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + wave;
  const bool live = row < N && rm.live(row);
  float* r = s_r[wave];
  for (int d = lane; d < D; d += 64) r[d] = live ? rm.xval(row, d) : 0.f;
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
    if (live && lane == 0) rm.crow(row)[m] = (uint8_t)bk;
    const float* crow = cb + ((int64_t)m * K + bk) * D;
    for (int d = lane; d < D; d += 64) r[d] = r[d] - crow[d];
    __syncthreads();
  }
  const float rn = wave_self_dot16(r, D, lane);
  if (live && lane == 0 && rnorm) rnorm[row] = sqrtf(rn);
}

// ------------------------------------------------------------------ MFMA path
// The same greedy recurrence with the distance search split in two:
//   coarse: G_k = (rn + cn_k) - 2 * Dm_k, where Dm_k = r . C_k from
//           v_mfma_f32_16x16x16_bf16 on bf16-rounded inputs;
//   exact:  E_k = (rn + cn_k) - 2 * dot16(r, C_k) (the contract) for every k
//           that the coarse pass cannot rule out.
// Error bound.  With S_k = sum_d |r_d C_k,d| <= sqrt(rn * cn_k) (up to the
// relative error of the fp32 norms), bf16 rounding of both inputs moves each
// product by at most 2^-8 (1 + 2^-10) |r_d C_d|, fp32 accumulation of the 128
// exact products adds at most 128 * 2^-24 S_k, and dot16 differs from the
// exact dot by at most 12 * 2^-24 S_k; so |Dm_k - dot16_k| < 1.02 * 2^-8 S_k
// and |G_k - E_k| < 2^-7 * 1.03 * S_k + 2u (|A_k| + 2 |Dm_k|) (u = 2^-24, the
// two roundings of the final subtraction).  eps_k doubles both terms and adds
// an absolute term for flushed subnormals.  Entry k is ruled out only when
//   fl(G_k - eps_k) > U,  U = min_j fl(G_j + eps_j),
// which implies E_k > E_j for the entry j attaining U, so the exact minimum
// and all its ties survive; written as !(G_k - eps_k > U), non-finite
// values are never ruled out (NaN rows fall back to a full exact scan).
// The exact pass keeps the contract's lowest-index tie rule; NaN and +inf
// never win, as in the strict-< scan, and a row with no finite distance gets
// code 0.
//
// A workgroup owns 16 rows and runs all M stages; wave w covers N-tiles
// w, w + WAVES, ...  Stage m + 1's B fragments and norms are loaded while
// stage m runs.
typedef short bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <int D>
struct EncCfg {
  static constexpr int KS = D / 16;             // MFMA k-steps per tile
  static constexpr int TPW = D == 256 ? 2 : 4;  // N-tiles per wave
  static constexpr int WAVES = 16 / TPW;        // covers K <= 256 (16 tiles)
  static constexpr int THREADS = WAVES * 64;
  static constexpr int L = D / 16;              // dot16 chain length
  static constexpr int CAP = D == 256 ? 2 : 4;  // exact rechecks loaded per batch
};

__global__ __launch_bounds__(256) void encode_prep_frag(const float* __restrict__ cb, int M,
                                                        int K, int D,
                                                        uint16_t* __restrict__ frag) {
  // One thread per (m, tile, ks, lane): four bf16 of C[m][tile*16 + l%16][ks*16 + 4*(l/16) ..].
  const int KS = D / 16, NT = K / 16;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)M * NT * KS * 64;
  if (i >= total) return;
  const int l = (int)(i % 64);
  int64_t q = i / 64;
  const int ks = (int)(q % KS);
  q /= KS;
  const int tile = (int)(q % NT);
  const int m = (int)(q / NT);
  const int k = tile * 16 + (l & 15);
  const int d = ks * 16 + 4 * (l >> 4);
  const float* src = cb + ((int64_t)m * K + k) * D + d;
  uint16_t* dst = frag + i * 4;
#pragma unroll
  for (int e = 0; e < 4; ++e) dst[e] = f2bf(src[e]);
}

// One thread per (m, quarter q, step pair p, lane l): the eight bf16 of
// C[m][64q + l][8p .. 8p+7] (zeros past K), the B operands of two 4x4x4 steps.
__global__ __launch_bounds__(256) void encode_prep_frag4(const float* __restrict__ cb, int M,
                                                         int K, int D,
                                                         uint16_t* __restrict__ frag4) {
  const int NQ = (K + 63) / 64, NP = D / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)M * NQ * NP * 64;
  if (i >= total) return;
  const int l = (int)(i % 64);
  int64_t q = i / 64;
  const int pp = (int)(q % NP);
  q /= NP;
  const int qq = (int)(q % NQ);
  const int m = (int)(q / NQ);
  const int k = qq * 64 + l;
  uint16_t* dst = frag4 + i * 8;
  const float* src = cb + ((int64_t)m * K + k) * D + 8 * pp;
#pragma unroll
  for (int e = 0; e < 8; ++e) dst[e] = k < K ? f2bf(src[e]) : (uint16_t)0;
}

// Cross-lane moves within a row of 16 lanes (DPP, no LDS round trip).
// row_shl:n gives lane i the value of lane i + n of its row (0 past the end).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
// dot16 fold of the 16 chain sums held by the lanes of a row, leaving s_0 in
// every lane.  Step w adds the value rotated by w within the row.  After the
// steps for 8, ..., 2w the row's values repeat with period 2w, so the lane at
// rotation distance w holds the value of lane j ^ w: lanes j < w compute
// s_j + s_{j+w} (the contract's pairing) and every other lane a copy of one
// of those sums (fp32 addition is commutative).
__device__ __forceinline__ float row_fold16(float a) {
  a = a + dpp_f<0x128>(a);  // row_ror:8
  a = a + dpp_f<0x124>(a);  // row_ror:4
  a = a + dpp_f<0x122>(a);  // row_ror:2
  a = a + dpp_f<0x121>(a);  // row_ror:1
  return a;
}
// Minimum over the 16 lanes of a row, in every lane (row_ror rotations).
__device__ __forceinline__ float row_min16(float a) {
  a = fminf(a, dpp_f<0x128>(a));  // row_ror:8
  a = fminf(a, dpp_f<0x124>(a));  // row_ror:4
  a = fminf(a, dpp_f<0x122>(a));  // row_ror:2
  a = fminf(a, dpp_f<0x121>(a));  // row_ror:1
  return a;
}

template <int D>
struct EncStage {
  uint2 b[EncCfg<D>::TPW][EncCfg<D>::KS];
  float cn[EncCfg<D>::TPW];
  float scn[EncCfg<D>::TPW];
};

// Stage m's fragments and norms for this wave's tiles.  Tiles past K load
// tile NT - 1 (in bounds, results ignored), so the loads are branch-free and
// the compiler's wait counts stay exact.
template <int D>
__device__ __forceinline__ void enc_load_stage(EncStage<D>& st, const uint2* __restrict__ frag,
                                               const float* __restrict__ cn,
                                               const float* __restrict__ scn, int m, int NT,
                                               int K, int wave, int lane) {
  using C = EncCfg<D>;
#pragma unroll
  for (int i = 0; i < C::TPW; ++i) {
    const int tile = min(wave + i * C::WAVES, NT - 1);
    const uint2* f = frag + (((int64_t)m * NT + tile) * C::KS) * 64 + lane;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) st.b[i][ks] = f[ks * 64];
    const int64_t ci = (int64_t)m * K + tile * 16 + (lane & 15);
    st.cn[i] = cn[ci];
    st.scn[i] = scn[ci];
  }
}

// Four fp32 -> bf16 (round to nearest even; v_cvt_pk_bf16_f32) packed in 8 bytes.
__device__ __forceinline__ uint2 bf16x4_bits(const float4 v) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t lo = {(__bf16)v.x, (__bf16)v.y};
  const bf16x2_t hi = {(__bf16)v.z, (__bf16)v.w};
  return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
}

template <int D>
struct EncShared {
  float r[16][D];
  // bf16(r): the MFMA A operand.  The pitch (D + 8) puts the 16 rows of one
  // operand read in different banks (a pitch of D, a multiple of 64 banks,
  // would put them all in the same two)
  uint16_t rb[16][D + 8];
  float rn[16];
  float u[16][EncCfg<D>::WAVES];  // per row, per wave: min of the upper bounds
  uint16_t mask[16][16];          // per row, per 16-entry tile: coarse-pass survivors
  uint8_t list[16][256];          // survivors of a row, ascending
  uint8_t code[16][64];           // codes of stages < 64, stored after the last stage
};

// Pull this workgroup's quarter of codebook m (fp32) into L2 ahead of the
// exact recheck: one dword per 128-byte line.  Workgroups are dealt
// round-robin to the 8 XCDs, so the four workgroups b, b + 8, b + 16, b + 24
// share an L2 and each takes a different quarter.  The value is consumed a
// stage later (folded into a sink the kernel keeps alive), so the compiler
// waits for it only then.
template <int D>
__device__ __forceinline__ uint32_t enc_prefetch_l2(const float* __restrict__ cb, int m, int K,
                                                    int wave, int lane) {
  using C = EncCfg<D>;
  const int64_t words = (int64_t)K * D;     // fp32 words of codebook m
  const int64_t q = words / 4;              // this workgroup's quarter
  const int64_t lo = ((blockIdx.x >> 3) & 3) * q;
  // one word per 32 bytes of the quarter (a wave's four lanes on one line
  // share a request)
  int64_t w = lo + ((int64_t)wave * 64 + lane) * (q / C::THREADS > 8 ? q / C::THREADS : 8);
  w = w < words - 1 ? w : words - 1;
  return __builtin_bit_cast(uint32_t, cb[(int64_t)m * words + w]);
}

// One greedy stage for the workgroup's 16 rows.  On entry s.r holds the
// residuals and s.rn their dot16 norms; on exit both are updated and codes
// for stage m are written.  The barriers order LDS only, so the next stage's
// fragment loads stay in flight across them.
template <int D>
__device__ __forceinline__ void enc_stage(EncShared<D>& s, const EncStage<D>& st,
                                          const float* __restrict__ cb,
                                          const float* __restrict__ cn, int m, int K, int NT,
                                          int row0, int N, const RowMap& rm, int wave,
                                          int lane, int tid) {
  using C = EncCfg<D>;
  // A fragments: row l%16, d = ks*16 + 4*(l/16) + e, from the bf16 copy.
  bf16x4_t a[C::KS];
  {
    const uint16_t* rr = s.rb[lane & 15] + 4 * (lane >> 4);
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks)
      a[ks] = __builtin_bit_cast(bf16x4_t, *reinterpret_cast<const uint2*>(rr + ks * 16));
  }
  f32x4_t acc[C::TPW];
#pragma unroll
  for (int i = 0; i < C::TPW; ++i) {
    acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks)
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
          a[ks], __builtin_bit_cast(bf16x4_t, st.b[i][ks]), acc[i], 0, 0, 0);
  }
  // acc[i][e]: row 4*(lane/16) + e, entry k = (wave + i*WAVES)*16 + lane%16.
  float g_lo[C::TPW][4], g_hi[C::TPW][4];
  float umin[4] = {INFINITY, INFINITY, INFINITY, INFINITY};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int row = 4 * (lane >> 4) + e;
    const float rn = s.rn[row];
    // v_sqrt_f32 (within an ulp or so): the 1.0078 factor of the first eps
    // term absorbs the rounding of both square roots and their product.
    const float srn = __builtin_amdgcn_sqrtf(rn);
#pragma unroll
    for (int i = 0; i < C::TPW; ++i) {
      const float cnk = st.cn[i];
      const float A = rn + cnk;
      const float dm = acc[i][e];
      const float g = A - 2.0f * dm;
      const float eps = 0x1.02p-6f * (srn * st.scn[i]) + 0x1p-21f * (fabsf(A) + 2.0f * fabsf(dm)) +
                        0x1p-116f * (1.0f + srn + st.scn[i]);
      const bool live = wave + i * C::WAVES < NT;
      g_lo[i][e] = live ? g - eps : INFINITY;
      g_hi[i][e] = live ? g + eps : INFINITY;
      umin[e] = fminf(umin[e], g_hi[i][e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) umin[e] = row_min16(umin[e]);
  if ((lane & 15) == 0)
#pragma unroll
    for (int e = 0; e < 4; ++e) s.u[4 * (lane >> 4) + e][wave] = umin[e];
  lds_barrier();
  // Survivors: entries whose lower bound does not exceed the row's least
  // upper bound U.  One ballot per (tile, row slot) gives the four rows'
  // 16-entry masks; lane 16g writes row 4g + e's (no atomics, no returns).
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int row = 4 * (lane >> 4) + e;
    const float4* up = reinterpret_cast<const float4*>(s.u[row]);
    float U = INFINITY;
#pragma unroll
    for (int w = 0; w < C::WAVES / 4; ++w) {
      const float4 v = up[w];
      U = fminf(U, fminf(fminf(v.x, v.y), fminf(v.z, v.w)));
    }
#pragma unroll
    for (int i = 0; i < C::TPW; ++i) {
      const int tile = wave + i * C::WAVES;
      const uint64_t b = __ballot(tile < NT && !(g_lo[i][e] > U));
      if ((lane & 15) == 0) s.mask[row][tile] = (uint16_t)(b >> (lane & 48));
    }
  }
  lds_barrier();
  // Group g < 16 (16 lanes) owns row g: it rechecks the row's survivors with
  // the exact dot16 (lane j runs chain j), keeps the winner's fp32 chunk in
  // registers, and updates its residual chunk and norm without another
  // barrier.  Ties go to the lowest entry; NaN and +inf never win; no finite
  // distance leaves code 0.
  const int grp = wave * 4 + (lane >> 4), j = lane & 15;
  if (grp < 16) {
    const int row = grp;
    float rc[C::L];
#pragma unroll
    for (int t = 0; t < C::L; t += 4) {
      const float4 v = *reinterpret_cast<const float4*>(&s.r[row][j * C::L + t]);
      rc[t] = v.x;
      rc[t + 1] = v.y;
      rc[t + 2] = v.z;
      rc[t + 3] = v.w;
    }
    const float rn = s.rn[row];
    // The row's survivor list: lane j takes tile j's mask, an inclusive scan
    // over the group's 16 lanes gives each tile its offset, and the lanes
    // write their entries in ascending order.  The group reads the list
    // back in the same wave, so LDS order is all that is needed.
    uint32_t n;
    {
      const uint32_t mk = s.mask[row][j];
      const uint32_t c = (uint32_t)__builtin_popcount(mk);
      uint32_t inc = c;
      inc += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)inc, 0x111, 0xf, 0xf, true);  // row_shr:1
      inc += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)inc, 0x112, 0xf, 0xf, true);  // row_shr:2
      inc += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)inc, 0x114, 0xf, 0xf, true);  // row_shr:4
      inc += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)inc, 0x118, 0xf, 0xf, true);  // row_shr:8
      n = (uint32_t)__builtin_amdgcn_ds_bpermute((lane | 15) << 2, (int)inc);
      uint32_t o = inc - c, mm = mk;
      while (mm) {
        s.list[row][o++] = (uint8_t)(j * 16 + __builtin_ctz(mm));
        mm &= mm - 1;
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
    float bc[C::L];
#pragma unroll
    for (int t = 0; t < C::L; ++t) bc[t] = 0.f;
    float best = 0.f;
    int bk = -1;
    // Batches of CAP survivors: all their loads are issued before any
    // is used, so a batch costs one memory latency.
    for (uint32_t base = 0; base < n; base += C::CAP) {
      const uint32_t word = C::CAP == 4 ? *reinterpret_cast<const uint32_t*>(&s.list[row][base])
                                        : *reinterpret_cast<const uint16_t*>(&s.list[row][base]);
      int kq[C::CAP];
      float c[C::CAP][C::L], cnk[C::CAP];
#pragma unroll
      for (int q = 0; q < C::CAP; ++q) {
        // entries past n repeat the batch's first (in bounds; not evaluated)
        kq[q] = base + q < n ? (int)((word >> (8 * q)) & 0xffu) : (int)(word & 0xffu);
        const float* cr = cb + ((int64_t)m * K + kq[q]) * D + j * C::L;
#pragma unroll
        for (int t = 0; t < C::L; t += 4) {
          const float4 v = *reinterpret_cast<const float4*>(cr + t);
          c[q][t] = v.x;
          c[q][t + 1] = v.y;
          c[q][t + 2] = v.z;
          c[q][t + 3] = v.w;
        }
        cnk[q] = cn[(int64_t)m * K + kq[q]];
      }
#pragma unroll
      for (int q = 0; q < C::CAP; ++q) {
        float dot = 0.f;
#pragma unroll
        for (int t = 0; t < C::L; ++t) dot = __builtin_fmaf(rc[t], c[q][t], dot);
        dot = row_fold16(dot);
        const float E = (rn + cnk[q]) - 2.0f * dot;
        const int k = kq[q];
        if (base + q < n && !(E != E) && E != INFINITY &&
            (bk < 0 || E < best || (E == best && k < bk))) {
          best = E;
          bk = k;
#pragma unroll
          for (int t = 0; t < C::L; ++t) bc[t] = c[q][t];
        }
      }
    }
    const int code = bk < 0 ? 0 : bk;
    if (bk < 0) {
      const float* cr = cb + (int64_t)m * K * D + j * C::L;
#pragma unroll
      for (int t = 0; t < C::L; ++t) bc[t] = cr[t];
    }
    float a2 = 0.f;
#pragma unroll
    for (int t = 0; t < C::L; t += 4) {
      float4 r4;
      r4.x = rc[t] - bc[t];
      r4.y = rc[t + 1] - bc[t + 1];
      r4.z = rc[t + 2] - bc[t + 2];
      r4.w = rc[t + 3] - bc[t + 3];
      *reinterpret_cast<float4*>(&s.r[row][j * C::L + t]) = r4;
      *reinterpret_cast<uint2*>(&s.rb[row][j * C::L + t]) = bf16x4_bits(r4);
      a2 = __builtin_fmaf(r4.x, r4.x, a2);
      a2 = __builtin_fmaf(r4.y, r4.y, a2);
      a2 = __builtin_fmaf(r4.z, r4.z, a2);
      a2 = __builtin_fmaf(r4.w, r4.w, a2);
    }
    a2 = row_fold16(a2);
    if (j == 0) {
      s.rn[row] = a2;
      // held in LDS: a store here would hold up the next stage's operand wait
      if (m < 64) s.code[row][m] = (uint8_t)code;
      else if (row0 + row < N && rm.live(row0 + row)) rm.crow(row0 + row)[m] = (uint8_t)code;
    }
  }
  lds_barrier();
}

template <int D>
__global__ __launch_bounds__(EncCfg<D>::THREADS) void encode_mfma_kernel(
    RowMap rm, int N, const float* __restrict__ cb, int M,
    int K, const uint2* __restrict__ frag, const float* __restrict__ cn,
    const float* __restrict__ scn, float* __restrict__ rnorm) {
  using C = EncCfg<D>;
  __shared__ __attribute__((aligned(16))) EncShared<D> s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * 16;
  const int NT = K / 16;
  if (rm.ranges) {  // a workgroup with no live row leaves at once (same test in every thread)
    bool any = false;
    for (int r = 0; r < 16; ++r) any = any || (row0 + r < N && rm.live(row0 + r));
    if (!any) return;
  }
  // Stage 0's fragments are requested first, so that they arrive with the
  // rows.  Stage m + 1's are requested before stage m runs.  The request is
  // unconditional (the last stage re-requests itself) so that no branch
  // joins paths with different numbers of loads in flight, which would force
  // the compiler to wait for all of them before the first MFMA.
  EncStage<D> st0, st1;
  enc_load_stage<D>(st0, frag, cn, scn, 0, NT, K, wave, lane);
  for (int i = tid; i < 16 * D; i += C::THREADS) {
    const int r = i / D, d = i - r * D;
    const float v = (row0 + r < N && rm.live(row0 + r)) ? rm.xval(row0 + r, d) : 0.f;
    s.r[r][d] = v;
    s.rb[r][d] = __builtin_bit_cast(uint16_t, (__bf16)v);
  }
  lds_barrier();
  const int grp = wave * 4 + (lane >> 4), j = lane & 15;
  if (grp < 16) {
    const float* rr = s.r[grp] + j * C::L;
    float a2 = 0.f;
#pragma unroll
    for (int t = 0; t < C::L; ++t) a2 = __builtin_fmaf(rr[t], rr[t], a2);
    a2 = row_fold16(a2);
    if (j == 0) s.rn[grp] = a2;
  }
  lds_barrier();

  uint32_t sink = 0, pfa = 0, pfb = 0;
  for (int m = 0; m < M; m += 2) {
    enc_load_stage<D>(st1, frag, cn, scn, min(m + 1, M - 1), NT, K, wave, lane);
    pfb = enc_prefetch_l2<D>(cb, min(m + 1, M - 1), K, wave, lane);
    enc_stage<D>(s, st0, cb, cn, m, K, NT, row0, N, rm, wave, lane, tid);
    sink ^= pfa;
    if (m + 1 >= M) break;
    enc_load_stage<D>(st0, frag, cn, scn, min(m + 2, M - 1), NT, K, wave, lane);
    pfa = enc_prefetch_l2<D>(cb, min(m + 2, M - 1), K, wave, lane);
    enc_stage<D>(s, st1, cb, cn, m + 1, K, NT, row0, N, rm, wave, lane, tid);
    sink ^= pfb;
  }
  sink ^= pfa ^ pfb;
  if (sink == 0x9e3779b9u && N < 0) rm.codes[0] = 0;  // never true: keeps the prefetch loads
  const int mc = M < 64 ? M : 64;
  for (int i = tid; i < 16 * mc; i += C::THREADS) {
    const int r = i / mc, mm = i - r * mc;
    if (row0 + r < N && rm.live(row0 + r)) rm.crow(row0 + r)[mm] = s.code[r][mm];
  }
  if (tid < 16 && rnorm && row0 + tid < N && rm.live(row0 + tid))
    rnorm[row0 + tid] = sqrtf(s.rn[tid]);
}

// ------------------------------------------ four rows per workgroup (flushes)
// The stage of enc_stage for 4 rows, so that a decode flush (8 KV heads x 64
// tokens = 512 rows) spreads over 128 CUs instead of 32.  The stage chain is
// latency-bound: a 16-row workgroup has one wave per SIMD, each running 16
// rows' bound arithmetic, list building and recheck back to back.  Here the
// coarse dots come from v_mfma_f32_4x4x4bf16_1k (16 blocks of 4x4x4); in
// block b (lanes 4b .. 4b+3)
//     D[lane l][v] = sum_k A[lane 4b+v][k] * B[lane l][k]
// over the four bf16 k terms of a register.  With lane l supplying residual
// row l % 4 as A and codebook entry 64w + l (wave w) as B, lane l ends with the
// dots of its entry with all four rows.  The error bound of the 16-row kernel
// holds as it stands: it covers any fp32 accumulation order of the D exact
// bf16 products.  After one barrier wave v owns row v: its survivors are four
// wave-uniform ballots over the row's 256 lower bounds, rechecked four at a
// time (one candidate per 16-lane group, dot16 chain j in lane j), and the
// group holding the winner updates the row's residual.  B operands come from
// the 16x16x16 fragment layout of the prep: entry k's 4 bf16 at d = 4s are
// fragment lane (k % 16) + 16 (s % 4) of tile k / 16, k-step s / 4, i.e.
// 16 s uint2 past its step-0 slot.
constexpr int kR4 = 4;
// Codes of the first kCodeStage stages are kept in LDS and stored once at
// the end: a global store inside the stage loop would make the next stage's
// wait for its operands also wait for the store's acknowledgement.
constexpr int kCodeStage = 64;

template <int D>
struct Enc4Shared {
  float r[kR4][D];
  uint16_t rb[kR4][D + 8];  // bf16(r); the pitch puts the four rows in different banks
  float rn[kR4];
  float2 gb[kR4][256];      // per row, per entry: (lower, upper) bound of the coarse distance
  uint8_t code[kR4][kCodeStage];  // the rows' codes, written out after the last stage
};

template <int D>
struct Enc4Stage {
  uint4 b[D / 8];  // B operands of steps 2p (x, y) and 2p + 1 (z, w)
  float cn, scn;
};

// Stage m's operands of lane l of wave q: entry 64q + l (quarters past K load
// the last quarter, results ignored), one coalesced 16-byte load per step pair.
template <int D>
__device__ __forceinline__ void enc4_load_stage(Enc4Stage<D>& st, const uint4* __restrict__ frag4,
                                                const float* __restrict__ cn,
                                                const float* __restrict__ scn, int m, int NQ,
                                                int K, int qc, int kc, int lane) {
  const uint4* f = frag4 + (((int64_t)m * NQ + qc) * (D / 8)) * 64 + lane;
#pragma unroll
  for (int pp = 0; pp < D / 8; ++pp) st.b[pp] = f[64 * pp];
  st.cn = cn[(int64_t)m * K + kc];
  st.scn = scn[(int64_t)m * K + kc];
}

// Minimum over the 64 lanes of a wave (wave-uniform).
__device__ __forceinline__ float wave_min64(float a) {
  a = row_min16(a);
  const float a0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 0));
  const float a1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 16));
  const float a2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 32));
  const float a3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 48));
  return fminf(fminf(a0, a1), fminf(a2, a3));
}

// Lowest set bit of the 256-bit mask m[0..3] (wave-uniform), cleared; -1 if empty.
__device__ __forceinline__ int pop_lowest(uint64_t& m0, uint64_t& m1, uint64_t& m2, uint64_t& m3) {
  if (m0) { const int b = __builtin_ctzll(m0); m0 &= m0 - 1; return b; }
  if (m1) { const int b = __builtin_ctzll(m1); m1 &= m1 - 1; return 64 + b; }
  if (m2) { const int b = __builtin_ctzll(m2); m2 &= m2 - 1; return 128 + b; }
  if (m3) { const int b = __builtin_ctzll(m3); m3 &= m3 - 1; return 192 + b; }
  return -1;
}

// Pull slice (block / 8) % 16 of codebook m (fp32) into L2 ahead of the exact
// recheck: the workgroups of one XCD (block ids equal mod 8) take different
// slices.  One word per 32 bytes; consumed a stage later through a sink.
template <int D>
__device__ __forceinline__ uint32_t enc4_prefetch_l2(const float* __restrict__ cb, int m, int K,
                                                     int tid) {
  const int64_t words = (int64_t)K * D;
  const int64_t slice = (words + 15) / 16;
  const int64_t stride = slice / 256 > 8 ? slice / 256 : 8;
  int64_t w = ((blockIdx.x >> 3) & 15) * slice + (int64_t)tid * stride;
  w = w < words - 1 ? w : words - 1;
  return __builtin_bit_cast(uint32_t, cb[(int64_t)m * words + w]);
}

template <int D>
__device__ __forceinline__ void enc4_stage(Enc4Shared<D>& s, const Enc4Stage<D>& st,
                                           const float* __restrict__ cb,
                                           const float* __restrict__ cn, int m, int K, int row0,
                                           int N, const RowMap& rm, bool own, int k, int wave,
                                           int lane) {
  constexpr int S4 = D / 4, L = D / 16;
  // ---- coarse pass: lane l, entry k = 64 wave + l, all four rows
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  {
    const uint16_t* ar = s.rb[lane & 3];
#pragma unroll
    for (int t = 0; t < S4; t += 2) {
      const uint4 aa = *reinterpret_cast<const uint4*>(ar + 4 * t);
      const uint4 bb = st.b[t / 2];
      acc0 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(
          __builtin_bit_cast(bf16x4_t, make_uint2(aa.x, aa.y)),
          __builtin_bit_cast(bf16x4_t, make_uint2(bb.x, bb.y)), acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(
          __builtin_bit_cast(bf16x4_t, make_uint2(aa.z, aa.w)),
          __builtin_bit_cast(bf16x4_t, make_uint2(bb.z, bb.w)), acc1, 0, 0, 0);
    }
  }
#pragma unroll
  for (int v = 0; v < kR4; ++v) {
    const float rn = s.rn[v];
    const float srn = __builtin_amdgcn_sqrtf(rn);
    const float A = rn + st.cn;
    const float dm = acc0[v] + acc1[v];
    const float g = A - 2.0f * dm;
    const float eps = 0x1.02p-6f * (srn * st.scn) + 0x1p-21f * (fabsf(A) + 2.0f * fabsf(dm)) +
                      0x1p-116f * (1.0f + srn + st.scn);
    s.gb[v][k] = own ? make_float2(g - eps, g + eps) : make_float2(INFINITY, INFINITY);
  }
  lds_barrier();

  // ---- exact recheck of row v = wave: U = least upper bound over the row
  const int v = wave, j = lane & 15, grp = lane >> 4;
  const float2 b0 = s.gb[v][lane], b1 = s.gb[v][64 + lane];
  const float2 b2 = s.gb[v][128 + lane], b3 = s.gb[v][192 + lane];
  const float U = wave_min64(fminf(fminf(b0.y, b1.y), fminf(b2.y, b3.y)));
  uint64_t mk0 = __ballot(lane < K && !(b0.x > U));
  uint64_t mk1 = __ballot(64 + lane < K && !(b1.x > U));
  uint64_t mk2 = __ballot(128 + lane < K && !(b2.x > U));
  uint64_t mk3 = __ballot(192 + lane < K && !(b3.x > U));
  float rc[L];
#pragma unroll
  for (int t = 0; t < L; t += 4) {
    const float4 x = *reinterpret_cast<const float4*>(&s.r[v][j * L + t]);
    rc[t] = x.x;
    rc[t + 1] = x.y;
    rc[t + 2] = x.z;
    rc[t + 3] = x.w;
  }
  const float rn = s.rn[v];
  float bc[L];
#pragma unroll
  for (int t = 0; t < L; ++t) bc[t] = 0.f;
  float best = 0.f;
  int bk = -1;
  // Batches of four survivors, one per group, lowest entries first.  Ties go
  // to the lowest entry; NaN and +inf never win.
  while (mk0 | mk1 | mk2 | mk3) {
    const int q0 = pop_lowest(mk0, mk1, mk2, mk3);
    const int q1 = pop_lowest(mk0, mk1, mk2, mk3);
    const int q2 = pop_lowest(mk0, mk1, mk2, mk3);
    const int q3 = pop_lowest(mk0, mk1, mk2, mk3);
    const int kq = grp == 0 ? q0 : grp == 1 ? q1 : grp == 2 ? q2 : q3;
    if (kq >= 0) {
      const float* cr = cb + ((int64_t)m * K + kq) * D + j * L;
      float c[L];
#pragma unroll
      for (int t = 0; t < L; t += 4) {
        const float4 x = *reinterpret_cast<const float4*>(cr + t);
        c[t] = x.x;
        c[t + 1] = x.y;
        c[t + 2] = x.z;
        c[t + 3] = x.w;
      }
      const float cnk = cn[(int64_t)m * K + kq];
      float dot = 0.f;
#pragma unroll
      for (int t = 0; t < L; ++t) dot = __builtin_fmaf(rc[t], c[t], dot);
      dot = row_fold16(dot);
      const float E = (rn + cnk) - 2.0f * dot;
      if (!(E != E) && E != INFINITY && (bk < 0 || E < best || (E == best && kq < bk))) {
        best = E;
        bk = kq;
#pragma unroll
        for (int t = 0; t < L; ++t) bc[t] = c[t];
      }
    }
  }
  // the winning group: lowest (E, entry) over the four groups' bests
  int gw = -1, code = 0;
  float ew = 0.f;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int kg = __builtin_amdgcn_readlane(bk, 16 * g);
    const float eg = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, best), 16 * g));
    if (kg >= 0 && (gw < 0 || eg < ew || (eg == ew && kg < code))) {
      gw = g;
      ew = eg;
      code = kg;
    }
  }
  if (gw < 0) {  // no finite distance: code 0, as the strict-< scan from +inf leaves it
    gw = 0;
    if (grp == 0) {
      const float* cr = cb + (int64_t)m * K * D + j * L;
#pragma unroll
      for (int t = 0; t < L; ++t) bc[t] = cr[t];
    }
  }
  if (grp == gw) {
    float a2 = 0.f;
#pragma unroll
    for (int t = 0; t < L; t += 4) {
      float4 r4;
      r4.x = rc[t] - bc[t];
      r4.y = rc[t + 1] - bc[t + 1];
      r4.z = rc[t + 2] - bc[t + 2];
      r4.w = rc[t + 3] - bc[t + 3];
      *reinterpret_cast<float4*>(&s.r[v][j * L + t]) = r4;
      *reinterpret_cast<uint2*>(&s.rb[v][j * L + t]) = bf16x4_bits(r4);
      a2 = __builtin_fmaf(r4.x, r4.x, a2);
      a2 = __builtin_fmaf(r4.y, r4.y, a2);
      a2 = __builtin_fmaf(r4.z, r4.z, a2);
      a2 = __builtin_fmaf(r4.w, r4.w, a2);
    }
    a2 = row_fold16(a2);
    if (j == 0) {
      s.rn[v] = a2;
      if (m < kCodeStage) s.code[v][m] = (uint8_t)code;
      else if (row0 + v < N && rm.live(row0 + v)) rm.crow(row0 + v)[m] = (uint8_t)code;
    }
  }
  lds_barrier();
}

template <int D>
__global__ __launch_bounds__(256) void encode_mfma4_kernel(
    RowMap rm, int N, const float* __restrict__ cb, int M, int K,
    const uint4* __restrict__ frag4, const float* __restrict__ cn,
    const float* __restrict__ scn, float* __restrict__ rnorm) {
  constexpr int L = D / 16;
  __shared__ __attribute__((aligned(16))) Enc4Shared<D> s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * kR4;
  const int NQ = (K + 63) / 64;
  const int qc = wave < NQ ? wave : NQ - 1;
  if (rm.ranges) {  // a workgroup with no live row leaves at once (same test in every thread)
    bool any = false;
    for (int r = 0; r < kR4; ++r) any = any || (row0 + r < N && rm.live(row0 + r));
    if (!any) return;
  }
  const int k = wave * 64 + lane;
  const bool own = k < K;
  const int kc = own ? k : K - 1;  // dead lanes load entry K - 1 (in bounds, ignored)
  // Stage 0's operands are requested first, so that they arrive with the
  // rows; stage m + 1's before stage m runs (unconditionally, the last stage
  // re-requesting itself, so that the compiler's wait counts stay exact).
  Enc4Stage<D> st0, st1;
  enc4_load_stage<D>(st0, frag4, cn, scn, 0, NQ, K, qc, kc, lane);
  for (int i = tid; i < kR4 * D; i += 256) {
    const int r = i / D, d = i - r * D;
    const float x = (row0 + r < N && rm.live(row0 + r)) ? rm.xval(row0 + r, d) : 0.f;
    s.r[r][d] = x;
    s.rb[r][d] = __builtin_bit_cast(uint16_t, (__bf16)x);
  }
  lds_barrier();
  if (lane < 16) {  // wave v: dot16 norm of row v
    const float* rr = s.r[wave] + lane * L;
    float a2 = 0.f;
#pragma unroll
    for (int t = 0; t < L; ++t) a2 = __builtin_fmaf(rr[t], rr[t], a2);
    a2 = row_fold16(a2);
    if (lane == 0) s.rn[wave] = a2;
  }
  lds_barrier();

  for (int m = 0; m < M; m += 2) {
    enc4_load_stage<D>(st1, frag4, cn, scn, min(m + 1, M - 1), NQ, K, qc, kc, lane);
    enc4_stage<D>(s, st0, cb, cn, m, K, row0, N, rm, own, k, wave, lane);
    if (m + 1 >= M) break;
    enc4_load_stage<D>(st0, frag4, cn, scn, min(m + 2, M - 1), NQ, K, qc, kc, lane);
    enc4_stage<D>(s, st1, cb, cn, m + 1, K, row0, N, rm, own, k, wave, lane);
  }
  const int mc = M < kCodeStage ? M : kCodeStage;
  for (int i = tid; i < kR4 * mc; i += 256) {
    const int r = i / mc, mm = i - r * mc;
    if (row0 + r < N && rm.live(row0 + r)) rm.crow(row0 + r)[mm] = s.code[r][mm];
  }
  if (tid < kR4 && rnorm && row0 + tid < N && rm.live(row0 + tid))
    rnorm[row0 + tid] = sqrtf(s.rn[tid]);
}

// ------------------------------------------ exact distances (flushes)
// A decode flush (8 KV heads x 64 tokens = 512 rows) has few rows per CU, and
// the bf16-MFMA kernels above pay a chain of dependent latencies per stage:
// coarse pass, survivor ballots, an L2 round trip for each survivor's fp32
// row, the exact recheck, the residual update.  Here every stage computes
// the contract's distance exactly for all K entries, with no coarse pass and
// no survivors: thread k of the 256 owns entry k and holds that entry's fp32
// row in registers (D values), loaded from the [M][D/4][K] float4 layout of
// the prep (each wave instruction reads one contiguous kilobyte).  A stage:
//   A. every thread runs the contract's dot16 (16 fmaf chains of D/16 and
//      the fold) of its entry against each of the R residuals, read from LDS
//      as broadcasts; each block of its row is reloaded with the next
//      stage's as soon as its products are done, so that the codebook
//      stream (every workgroup reads all of it) runs under the arithmetic;
//      each wave then takes its minimum of (orderable distance, entry) with
//      DPP and a ballot.  At C3 (two rows) the products' residual reads and
//      the stream each take about 0.9 us of a stage's 2 us;
//   B. (after a barrier) wave v picks row v's winner among the four wave
//      minima (lowest distance, then lowest entry; NaN and +inf never win;
//      none finite: entry 0), reads that entry's row from the fp32
//      codebook, subtracts it from the residual and forms the new
//      dot16(r, r) in 16 lanes; a second barrier ends the stage.
template <int D, int R>
struct ExactShared {
  float r[R][D];
  unsigned long long part[R][4];  // (distance key << 32) | entry, per wave
  float rn[R];
  uint8_t code[R][kCodeStage];
};

// Block q of entry kc's row in stage m: a uniform base per block and one
// 32-bit lane offset (the scalar-base address form: no 64-bit address per
// load in registers).
template <int D>
__device__ __forceinline__ float4 exact_block(const float4* __restrict__ c4, int m, int q, int K,
                                              uint32_t off) {
  const char* base = reinterpret_cast<const char*>(c4 + ((int64_t)m * (D / 4) + q) * K);
  return *reinterpret_cast<const float4*>(base + off);
}

// Orderable 32-bit key of a distance that may win (-0 as +0); 0xffffffff,
// above every such key, marks one that may not.
__device__ __forceinline__ uint32_t dist_key(float E, bool valid) {
  uint32_t u = __builtin_bit_cast(uint32_t, E == 0.0f ? 0.0f : E);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return valid ? u : 0xffffffffu;
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xf, 0xf, false);
}
// Minimum over the wave, uniform: rotations within each row of 16 lanes, then
// the four row minima through scalar registers.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  x = min(x, dpp_u<0x128>(x));  // row_ror:8
  x = min(x, dpp_u<0x124>(x));  // row_ror:4
  x = min(x, dpp_u<0x122>(x));  // row_ror:2
  x = min(x, dpp_u<0x121>(x));  // row_ror:1
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)x, 0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)x, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)x, 32);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)x, 48);
  return min(min(a, b), min(c, d));
}

template <int D, int R>
__global__ __launch_bounds__(256) void encode_exact_kernel(
    RowMap rm, int N, const float* __restrict__ cb, const float4* __restrict__ c4,
    const float* __restrict__ cn, int M, int K, float* __restrict__ rnorm) {
  static_assert(R >= 1 && R <= 4, "one wave per row for the residual update");
  constexpr int Q = D / 4, L = D / 16, QC = L / 4;  // float4 per chain
  constexpr int P = R >= 4 ? 3 : 4;  // residual reads in flight per row (LDS counter: 15)
  static_assert(L % 4 == 0, "chains of whole float4 blocks");
  __shared__ __attribute__((aligned(16))) ExactShared<D, R> s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * R;
  if (rm.ranges) {  // a workgroup with no live row leaves at once (same test in every thread)
    bool any = false;
    for (int r = 0; r < R; ++r) any = any || (row0 + r < N && rm.live(row0 + r));
    if (!any) return;
  }
  const bool own = tid < K;
  const int kc = own ? tid : K - 1;  // dead threads load entry K - 1 (in bounds, never chosen)
  const uint32_t off = (uint32_t)kc * 16u;
  float4 c[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) c[q] = exact_block<D>(c4, 0, q, K, off);
  float cnk = cn[kc];
  for (int i = tid; i < R * D; i += 256) {
    const int r = i / D, d = i - r * D;
    s.r[r][d] = (row0 + r < N && rm.live(row0 + r)) ? rm.xval(row0 + r, d) : 0.f;
  }
  lds_barrier();
  if (wave < R && lane < 16) {
    const float* rr = s.r[wave] + lane * L;
    float a2 = 0.f;
#pragma unroll
    for (int t = 0; t < L; ++t) a2 = __builtin_fmaf(rr[t], rr[t], a2);
    a2 = row_fold16(a2);
    if (lane == 0) s.rn[wave] = a2;
  }
  lds_barrier();
  for (int m = 0; m < M; ++m) {
    // the stage whose rows are requested behind this one's (the last stage
    // re-requests itself: every load is unconditional)
    const int mn = min(m + 1, M - 1);
    // A: exact distances of this thread's entry to every row
    float a[R][16];
#pragma unroll
    for (int v = 0; v < R; ++v)
#pragma unroll
      for (int j = 0; j < 16; ++j) a[v][j] = 0.f;
    // The residual blocks are read P blocks ahead, in a ring; the scheduling
    // barriers keep the compiler from hoisting every read to the top, which
    // costs a register per value and pushes the entry rows out of registers.
    float4 rb[P][R];
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int v = 0; v < R; ++v) rb[p][v] = *reinterpret_cast<const float4*>(&s.r[v][4 * p]);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      __builtin_amdgcn_sched_barrier(0);
      const int j = q / QC;
#pragma unroll
      for (int v = 0; v < R; ++v) {
        const float4 r4 = rb[q % P][v];
        a[v][j] = __builtin_fmaf(r4.x, c[q].x, a[v][j]);
        a[v][j] = __builtin_fmaf(r4.y, c[q].y, a[v][j]);
        a[v][j] = __builtin_fmaf(r4.z, c[q].z, a[v][j]);
        a[v][j] = __builtin_fmaf(r4.w, c[q].w, a[v][j]);
        // pins the chain's progress here: without it the compiler sinks
        // the later rows' products below the first row's selection and
        // keeps their residual blocks live meanwhile
        asm volatile("" : "+v"(a[v][j]));
      }
      c[q] = exact_block<D>(c4, mn, q, K, off);
      if (q + P < Q) {
#pragma unroll
        for (int v = 0; v < R; ++v)
          rb[q % P][v] = *reinterpret_cast<const float4*>(&s.r[v][4 * (q + P)]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int v = 0; v < R; ++v) {
      const float E = (s.rn[v] + cnk) - 2.0f * fold16(a[v]);
      const uint32_t key = dist_key(E, own && !(E != E) && E != INFINITY);
      const uint32_t wmin = wave_min_u32(key);
      // lanes holding the minimum; taken with the whole wave active (a
      // ballot sees only active lanes), non-zero whenever wmin is a key
      const uint64_t hit = __builtin_amdgcn_ballot_w64(key == wmin);
      if (lane == 0)  // the lowest such lane is the wave's lowest entry
        s.part[v][wave] = wmin == 0xffffffffu ? ~0ull
                                              : (((unsigned long long)wmin << 32) |
                                                 (uint32_t)(wave * 64 + __builtin_ctzll(hit)));
    }
    cnk = cn[(int64_t)mn * K + kc];
    lds_barrier();
    // B: row `wave`'s winner, residual update and new squared norm
    if (wave < R && lane < 16) {
      const int v = wave;
      unsigned long long b = s.part[v][0];
#pragma unroll
      for (int x = 1; x < 4; ++x) b = s.part[v][x] < b ? s.part[v][x] : b;
      // none finite: entry 0; an entry is always below K (only threads
      // k < K offer one), and the test keeps the row read in bounds
      const uint32_t e = (uint32_t)b;
      const int code = b == ~0ull || e >= (uint32_t)K ? 0 : (int)e;
      const float* cw = cb + ((int64_t)m * K + code) * D + lane * L;
      float4 w4[QC];
#pragma unroll
      for (int qq = 0; qq < QC; ++qq) w4[qq] = *reinterpret_cast<const float4*>(cw + 4 * qq);
      float a2 = 0.f;
#pragma unroll
      for (int qq = 0; qq < QC; ++qq) {
        float4 r4 = *reinterpret_cast<const float4*>(&s.r[v][lane * L + 4 * qq]);
        r4.x = r4.x - w4[qq].x;
        r4.y = r4.y - w4[qq].y;
        r4.z = r4.z - w4[qq].z;
        r4.w = r4.w - w4[qq].w;
        *reinterpret_cast<float4*>(&s.r[v][lane * L + 4 * qq]) = r4;
        a2 = __builtin_fmaf(r4.x, r4.x, a2);
        a2 = __builtin_fmaf(r4.y, r4.y, a2);
        a2 = __builtin_fmaf(r4.z, r4.z, a2);
        a2 = __builtin_fmaf(r4.w, r4.w, a2);
      }
      a2 = row_fold16(a2);
      if (lane == 0) {
        s.rn[v] = a2;
        if (m < kCodeStage) s.code[v][m] = (uint8_t)code;
        else if (row0 + v < N && rm.live(row0 + v)) rm.crow(row0 + v)[m] = (uint8_t)code;
      }
    }
    lds_barrier();
  }
  const int mc = M < kCodeStage ? M : kCodeStage;
  for (int i = tid; i < R * mc; i += 256) {
    const int r = i / mc, mm = i - r * mc;
    if (row0 + r < N && rm.live(row0 + r)) rm.crow(row0 + r)[mm] = s.code[r][mm];
  }
  if (tid < R && rnorm && row0 + tid < N && rm.live(row0 + tid))
    rnorm[row0 + tid] = sqrtf(s.rn[tid]);
}

// ------------------------------------------------ reconstruction
// recon[n] = sum over m ascending of C[m][code(n, m)], elementwise fp32 from
// 0 (laprune/llm/aq_kv.py:431-457).  A thread owns four consecutive
// elements of one row; the codebook rows it gathers are 16-byte vectors.
template <typename CT>
__global__ __launch_bounds__(256) void aq_reconstruct_kernel(
    const float* __restrict__ cb, int M, int K, int D, const CT* __restrict__ codes,
    int64_t cs, int N, float* __restrict__ out) {
  const int D4 = D / 4;
  const int64_t total = (int64_t)N * D4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int64_t n = i / D4;
    const int q = (int)(i - n * D4);
    const CT* cp = codes + n * cs;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int m = 0; m < M; ++m) {
      // the low 8 bits as an unsigned code, clamped to the last entry
      const int c = min((int)(uint8_t)(cp[m] & (CT)0xff), K - 1);
      const float4 v = *reinterpret_cast<const float4*>(cb + ((int64_t)m * K + c) * D + 4 * q);
      acc.x = acc.x + v.x;
      acc.y = acc.y + v.y;
      acc.z = acc.z + v.z;
      acc.w = acc.w + v.w;
    }
    *reinterpret_cast<float4*>(out + n * D + 4 * q) = acc;
  }
}

// ------------------------------------------------ large launches (prefill)
// The same stage as enc_stage for 64 rows per workgroup.  A 16-row workgroup
// holds its stage fragments (64 KiB at K = 256, D = 128) in registers, twice
// over for the prefetch, so register space caps a CU at 32 rows in flight;
// and the exact recheck makes every stage a chain of dependent latencies, so
// throughput follows the rows in flight.  Here 16 waves (4 row groups x 4
// tile quarters) share one LDS copy of the stage's fragments, the next
// stage's slice is fetched into registers (64 B per thread) while the
// current stage runs, and each of the 64 rows keeps its own 16-lane recheck
// group: 64 rows per CU, each stage costing what it costs a 16-row workgroup.
constexpr int kTileRows = 64;
constexpr int kTileThreads = 1024;

template <int D>
struct TileShared {
  static constexpr int KS = D / 16;
  uint2 frag[16 * KS * 64];    // stage fragments [tile][ks][lane], K <= 256
  float r[kTileRows][D];
  // bf16(r): the MFMA A operand.  The pitch (D + 8) puts the 16 rows of one
  // operand read in different banks (a pitch of D, a multiple of 64 banks,
  // would put them all in the same two)
  uint16_t rb[kTileRows][D + 8];
  float rn[kTileRows];
  float u[4][kTileRows];       // per tile quarter: min of G + eps per row
  uint32_t cnt[kTileRows];
  uint8_t list[kTileRows][256];
};

// This thread's slice of stage m's fragments: uint4 i of the stage lies at
// thread i % 1024, slot i / 1024 (clamped into the stage; at most 4 slots).
// Four named members, not an array, so that they stay in registers.
struct TileSlice {
  uint4 v0, v1, v2, v3;
};
template <int D>
__device__ __forceinline__ TileSlice tile_frag_load(const uint2* __restrict__ frag, int m, int NT,
                                                    int tid) {
  constexpr int KS = D / 16;
  const int n4 = NT * KS * 32;  // uint4 per stage
  const uint4* src = reinterpret_cast<const uint4*>(frag + (int64_t)m * NT * KS * 64);
  TileSlice p;
  p.v0 = src[min(tid, n4 - 1)];
  p.v1 = src[min(tid + kTileThreads, n4 - 1)];
  p.v2 = src[min(tid + 2 * kTileThreads, n4 - 1)];
  p.v3 = src[min(tid + 3 * kTileThreads, n4 - 1)];
  return p;
}
template <int D>
__device__ __forceinline__ void tile_frag_store(const TileSlice& p, uint2* s_frag, int NT,
                                                int tid) {
  constexpr int KS = D / 16;
  const int n4 = NT * KS * 32;
  uint4* dst = reinterpret_cast<uint4*>(s_frag);
  if (tid < n4) dst[tid] = p.v0;
  if (tid + kTileThreads < n4) dst[tid + kTileThreads] = p.v1;
  if (tid + 2 * kTileThreads < n4) dst[tid + 2 * kTileThreads] = p.v2;
  if (tid + 3 * kTileThreads < n4) dst[tid + 3 * kTileThreads] = p.v3;
}

template <int D>
__global__ __launch_bounds__(kTileThreads) void encode_tile_kernel(
    RowMap rm, int N, const float* __restrict__ cb, int M,
    int K, const uint2* __restrict__ frag, const float* __restrict__ cn,
    const float* __restrict__ scn, float* __restrict__ rnorm) {
  constexpr int KS = D / 16, L = D / 16, CAP = 2, TPW = 4;  // CAP 2: fits 128 VGPRs
  extern __shared__ __attribute__((aligned(16))) char tile_smem[];
  TileShared<D>& s = *reinterpret_cast<TileShared<D>*>(tile_smem);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rg = wave >> 2, q = wave & 3;  // row group, tile quarter
  const int row0 = blockIdx.x * kTileRows;
  const int NT = K / 16;
  if (rm.ranges) {  // a workgroup with no live row leaves at once (same test in every thread)
    bool any = false;
    for (int r = 0; r < kTileRows; ++r) any = any || (row0 + r < N && rm.live(row0 + r));
    if (!any) return;
  }
  TileSlice pf = tile_frag_load<D>(frag, 0, NT, tid);
  for (int i = tid; i < kTileRows * D; i += kTileThreads) {
    const int r = i / D, d = i - r * D;
    const float v = (row0 + r < N && rm.live(row0 + r)) ? rm.xval(row0 + r, d) : 0.f;
    s.r[r][d] = v;
    s.rb[r][d] = __builtin_bit_cast(uint16_t, (__bf16)v);
  }
  if (tid < kTileRows) s.cnt[tid] = 0;
  tile_frag_store<D>(pf, s.frag, NT, tid);
  __syncthreads();
  const int grp = wave * 4 + (lane >> 4), j = lane & 15;  // recheck group = row
  {
    const float* rr = s.r[grp] + j * L;
    float a2 = 0.f;
#pragma unroll
    for (int t = 0; t < L; ++t) a2 = __builtin_fmaf(rr[t], rr[t], a2);
    a2 = row_fold16(a2);
    if (j == 0) s.rn[grp] = a2;
  }
  __syncthreads();

  for (int m = 0; m < M; ++m) {
    // This stage's entry norms for the coarse pass's tiles (q, q+4, q+8,
    // q+12), requested before anything else of the stage: left to the
    // compiler, their loads sink below the MFMAs (to save the registers) and
    // each wave then waits an L2 round trip for them after its MFMAs (1,048,576
    // rows: 18.46 ms against 18.72 ms).
    float cnv[TPW], scv[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int tile = min(q + 4 * i, NT - 1);
      const int64_t ci = (int64_t)m * K + tile * 16 + (lane & 15);
      cnv[i] = cn[ci];
      scv[i] = scn[ci];
    }
    __builtin_amdgcn_sched_barrier(0);
    // next stage's fragments: in flight for the whole stage (re-requests the
    // last stage on the last pass, so the loads are unconditional)
    pf = tile_frag_load<D>(frag, min(m + 1, M - 1), NT, tid);
    // ---- coarse pass: rows rg*16.., tiles q, q+4, q+8, q+12
    bf16x4_t a[KS];
    {
      const uint16_t* rr = s.rb[rg * 16 + (lane & 15)] + 4 * (lane >> 4);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        a[ks] = __builtin_bit_cast(bf16x4_t, *reinterpret_cast<const uint2*>(rr + ks * 16));
    }
    float g_lo[TPW][4];
    float umin[4] = {INFINITY, INFINITY, INFINITY, INFINITY};
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int tile = min(q + 4 * i, NT - 1);
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
            a[ks], __builtin_bit_cast(bf16x4_t, s.frag[(tile * KS + ks) * 64 + lane]), acc, 0,
            0, 0);
      const bool live = q + 4 * i < NT;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float rn = s.rn[rg * 16 + 4 * (lane >> 4) + e];
        const float srn = __builtin_amdgcn_sqrtf(rn);
        const float A = rn + cnv[i];
        const float dm = acc[e];
        const float g = A - 2.0f * dm;
        const float eps = 0x1.02p-6f * (srn * scv[i]) + 0x1p-21f * (fabsf(A) + 2.0f * fabsf(dm)) +
                          0x1p-116f * (1.0f + srn + scv[i]);
        g_lo[i][e] = live ? g - eps : INFINITY;
        umin[e] = fminf(umin[e], live ? g + eps : INFINITY);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) umin[e] = row_min16(umin[e]);
    if ((lane & 15) == 0)
#pragma unroll
      for (int e = 0; e < 4; ++e) s.u[q][rg * 16 + 4 * (lane >> 4) + e] = umin[e];
    lds_barrier();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = rg * 16 + 4 * (lane >> 4) + e;
      const float U = fminf(fminf(s.u[0][row], s.u[1][row]), fminf(s.u[2][row], s.u[3][row]));
      uint32_t keep = 0;
#pragma unroll
      for (int i = 0; i < TPW; ++i) keep |= (uint32_t)(q + 4 * i < NT && !(g_lo[i][e] > U)) << i;
      if (keep) {
        uint32_t slot = atomicAdd(&s.cnt[row], (uint32_t)__builtin_popcount(keep));
#pragma unroll
        for (int i = 0; i < TPW; ++i)
          if (keep & (1u << i)) s.list[row][slot++] = (uint8_t)((q + 4 * i) * 16 + (lane & 15));
      }
    }
    lds_barrier();
    // ---- exact recheck: group grp owns row grp (same rules as enc_stage)
    {
      const int row = grp;
      float rc[L];
#pragma unroll
      for (int t = 0; t < L; t += 4) {
        const float4 v = *reinterpret_cast<const float4*>(&s.r[row][j * L + t]);
        rc[t] = v.x;
        rc[t + 1] = v.y;
        rc[t + 2] = v.z;
        rc[t + 3] = v.w;
      }
      const float rn = s.rn[row];
      const uint32_t n = s.cnt[row];
      if (j == 0) s.cnt[row] = 0;
      float bc[L];
#pragma unroll
      for (int t = 0; t < L; ++t) bc[t] = 0.f;
      float best = 0.f;
      int bk = -1;
      for (uint32_t base = 0; base < n; base += CAP) {
        const uint32_t word = *reinterpret_cast<const uint16_t*>(&s.list[row][base]);
        int kq[CAP];
        float c[CAP][L], cnk[CAP];
#pragma unroll
        for (int qq = 0; qq < CAP; ++qq) {
          kq[qq] = base + qq < n ? (int)((word >> (8 * qq)) & 0xffu) : (int)(word & 0xffu);
          const float* cr = cb + ((int64_t)m * K + kq[qq]) * D + j * L;
#pragma unroll
          for (int t = 0; t < L; t += 4) {
            const float4 v = *reinterpret_cast<const float4*>(cr + t);
            c[qq][t] = v.x;
            c[qq][t + 1] = v.y;
            c[qq][t + 2] = v.z;
            c[qq][t + 3] = v.w;
          }
          cnk[qq] = cn[(int64_t)m * K + kq[qq]];
        }
#pragma unroll
        for (int qq = 0; qq < CAP; ++qq) {
          float dot = 0.f;
#pragma unroll
          for (int t = 0; t < L; ++t) dot = __builtin_fmaf(rc[t], c[qq][t], dot);
          dot = row_fold16(dot);
          const float E = (rn + cnk[qq]) - 2.0f * dot;
          const int k = kq[qq];
          if (base + qq < n && !(E != E) && E != INFINITY &&
              (bk < 0 || E < best || (E == best && k < bk))) {
            best = E;
            bk = k;
#pragma unroll
            for (int t = 0; t < L; ++t) bc[t] = c[qq][t];
          }
        }
      }
      const int code = bk < 0 ? 0 : bk;
      if (bk < 0) {
        const float* cr = cb + (int64_t)m * K * D + j * L;
#pragma unroll
        for (int t = 0; t < L; ++t) bc[t] = cr[t];
      }
      float a2 = 0.f;
#pragma unroll
      for (int t = 0; t < L; t += 4) {
        float4 r4;
        r4.x = rc[t] - bc[t];
        r4.y = rc[t + 1] - bc[t + 1];
        r4.z = rc[t + 2] - bc[t + 2];
        r4.w = rc[t + 3] - bc[t + 3];
        *reinterpret_cast<float4*>(&s.r[row][j * L + t]) = r4;
        *reinterpret_cast<uint2*>(&s.rb[row][j * L + t]) = bf16x4_bits(r4);
        a2 = __builtin_fmaf(r4.x, r4.x, a2);
        a2 = __builtin_fmaf(r4.y, r4.y, a2);
        a2 = __builtin_fmaf(r4.z, r4.z, a2);
        a2 = __builtin_fmaf(r4.w, r4.w, a2);
      }
      a2 = row_fold16(a2);
      if (j == 0) {
        s.rn[row] = a2;
        if (row0 + row < N && rm.live(row0 + row)) rm.crow(row0 + row)[m] = (uint8_t)code;
      }
    }
    // every wave has read this stage's fragments (before the first barrier):
    // the next stage's may replace them
    tile_frag_store<D>(pf, s.frag, NT, tid);
    lds_barrier();
  }
  if (tid < kTileRows && rnorm && row0 + tid < N && rm.live(row0 + tid))
    rnorm[row0 + tid] = sqrtf(s.rn[tid]);
}

}  // namespace
}  // namespace lap

using namespace lap;

// LAPRUNE_ENCODE_IMPL=valu selects the all-VALU search (measurements and
// cross-checks); the MFMA search is the default wherever K % 16 == 0.
static bool encode_impl_mfma() {
  static const bool v = [] {
    const char* e = getenv("LAPRUNE_ENCODE_IMPL");
    return !(e && strcmp(e, "valu") == 0);
  }();
  return v;
}

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
                     M, K, D, p.cn, p.scn);
  LAP_LAUNCH_CHECK("encode_prep_norms");
  {
    const int64_t n = (int64_t)M * (D / 4) * K;
    hipLaunchKernelGGL(encode_prep_c4, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 4096)),
                       dim3(256), 0, st, codebooks, M, K, D, p.c4);
    LAP_LAUNCH_CHECK("encode_prep_c4");
  }
  if (K % 16 == 0) {
    const int64_t n = (int64_t)M * (K / 16) * (D / 16) * 64;
    hipLaunchKernelGGL(encode_prep_frag, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       codebooks, M, K, D, p.frag);
    LAP_LAUNCH_CHECK("encode_prep_frag");
    const int64_t n4 = (int64_t)M * ((K + 63) / 64) * (D / 8) * 64;
    hipLaunchKernelGGL(encode_prep_frag4, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st,
                       codebooks, M, K, D, p.frag4);
    LAP_LAUNCH_CHECK("encode_prep_frag4");
  }
  return LAP_OK;
}

// The 64-row workgroups pay off once every CU gets several of them; smaller
// launches (a decode flush) keep 16-row workgroups for their parallelism.
// D = 256 and K > 256 stay on the 16-row kernel.  LAPRUNE_ENCODE_TILE=0|1
// forces the choice.
static bool encode_use_tile(int N, int D, int K) {
  if (!(D == 64 || D == 128) || K > 256) return false;
  static const int forced = [] {
    const char* e = getenv("LAPRUNE_ENCODE_TILE");
    return e ? atoi(e) : -1;
  }();
  if (forced == 0 || forced == 1) return forced == 1;
  DevInfo di;
  const int cus = device_info(&di) == LAP_OK ? di.cu_count : 256;
  return (int64_t)N >= (int64_t)kTileRows * 2 * cus;
}

// Small encodes (decode flushes) take the 4-row kernel while its workgroups
// fit twice over on the chip; larger ones the 16-row kernel.
// LAPRUNE_ENCODE_ROWS=4|16 forces the choice (D = 64 or 128); read at every
// call, so that one process can run both.
static bool encode_use_rows4(int N, int D) {
  if (!(D == 64 || D == 128)) return false;
  const char* e = getenv("LAPRUNE_ENCODE_ROWS");
  const int forced = e ? atoi(e) : 0;
  if (forced == 4 || forced == 16) return forced == 4;
  DevInfo di;
  const int cus = device_info(&di) == LAP_OK ? di.cu_count : 256;
  return (int64_t)(N + kR4 - 1) / kR4 <= 2 * (int64_t)cus;
}

// Flushes take the exact kernel while its workgroups fit once on the chip:
// one row per workgroup up to one workgroup per CU, two rows up to twice
// that (a 512-row C3 flush: 256 workgroups).  A workgroup streams the whole
// codebook whatever its row count, so two workgroups on one CU take about
// twice as long, and larger flushes go to the 4-row MFMA kernel.
// LAPRUNE_ENCODE_EXACT=0|1 forces the choice and LAPRUNE_ENCODE_EXACT_ROWS=1|2
// the rows per workgroup; LAPRUNE_ENCODE_ROWS=4|16 (a forced MFMA kernel)
// turns it off.  All are read at every call, so that one process can compare
// them.
static int encode_cus() {
  DevInfo di;
  return device_info(&di) == LAP_OK ? di.cu_count : 256;
}
static int encode_exact_rows(int N) {
  const char* e = getenv("LAPRUNE_ENCODE_EXACT_ROWS");
  const int r = e ? atoi(e) : 0;
  if (r == 1 || r == 2) return r;
  return N <= encode_cus() ? 1 : 2;
}
static bool encode_use_exact(int N, int D, int K) {
  if (!(D == 64 || D == 128) || K > 256) return false;
  const char* e = getenv("LAPRUNE_ENCODE_EXACT");
  if (e && (e[0] == '0' || e[0] == '1') && e[1] == 0) return e[0] == '1';
  const char* rows = getenv("LAPRUNE_ENCODE_ROWS");
  if (rows && (atoi(rows) == 4 || atoi(rows) == 16)) return false;
  if (!encode_impl_mfma()) return false;
  return (int64_t)(N + 1) / 2 <= encode_cus();
}

// Shared checks and launch of both encode entry points.
static int run_encode(const RowMap& rm, int N, int D, const float* codebooks, int M, int K,
                      const void* prep, size_t prep_bytes, float* resid_norm,
                      lap_stream_t stream, const char* who) {
  LAP_CHECK(codebooks && prep, "%s: null pointer", who);
  LAP_CHECK(N >= 0 && M > 0 && K > 0 && D > 0, "%s: bad sizes", who);
  LAP_CHECK(K <= 256, "%s: K=%d exceeds 256 (uint8 codes)", who, K);
  LAP_CHECK_CODE(K % 4 == 0, LAP_ERR_UNSUPPORTED, "%s: K must be a multiple of 4", who);
  LAP_CHECK_CODE(D == 64 || D == 128 || D == 256, LAP_ERR_UNSUPPORTED,
                 "%s: D=%d unsupported (64/128/256)", who, D);
  Prep p = carve_prep(const_cast<void*>(prep), M, K, D);
  LAP_CHECK_CODE(prep_bytes >= p.bytes, LAP_ERR_WORKSPACE, "%s: prep buffer of %zu bytes needed",
                 who, p.bytes);
  LAP_CHECK((reinterpret_cast<uintptr_t>(p.ct) & 15) == 0, "%s: prep misaligned", who);
  // exact rechecks read codebook rows as 16-byte vectors
  LAP_CHECK((reinterpret_cast<uintptr_t>(codebooks) & 15) == 0,
            "%s: codebooks must be 16-byte aligned", who);
  if (N == 0) return LAP_OK;
  hipStream_t st = as_stream(stream);
  if (encode_use_exact(N, D, K)) {
    const int R = encode_exact_rows(N);
    dim3 g((N + R - 1) / R);
#define LAP_ENCX(D_, R_)                                                                 \
  hipLaunchKernelGGL((encode_exact_kernel<D_, R_>), g, dim3(256), 0, st, rm, N, codebooks, \
                     p.c4, p.cn, M, K, resid_norm)
    if (D == 64) {
      if (R == 1) LAP_ENCX(64, 1); else LAP_ENCX(64, 2);
    } else {
      if (R == 1) LAP_ENCX(128, 1); else LAP_ENCX(128, 2);
    }
#undef LAP_ENCX
    LAP_LAUNCH_CHECK("encode_exact_kernel");
    return LAP_OK;
  }
  if (K % 16 == 0 && encode_impl_mfma() && encode_use_tile(N, D, K)) {
    dim3 grid((N + kTileRows - 1) / kTileRows);
    const uint2* fr = reinterpret_cast<const uint2*>(p.frag);
    if (D == 64)
      hipLaunchKernelGGL(encode_tile_kernel<64>, grid, dim3(kTileThreads),
                         sizeof(TileShared<64>), st, rm, N, codebooks, M, K, fr, p.cn, p.scn,
                         resid_norm);
    else
      hipLaunchKernelGGL(encode_tile_kernel<128>, grid, dim3(kTileThreads),
                         sizeof(TileShared<128>), st, rm, N, codebooks, M, K, fr, p.cn, p.scn,
                         resid_norm);
    LAP_LAUNCH_CHECK("encode_tile_kernel");
    return LAP_OK;
  }
  if (K % 16 == 0 && encode_impl_mfma() && encode_use_rows4(N, D)) {
    dim3 g4((N + kR4 - 1) / kR4);
    const uint4* fr = reinterpret_cast<const uint4*>(p.frag4);
    if (D == 64)
      hipLaunchKernelGGL(encode_mfma4_kernel<64>, g4, dim3(256), 0, st, rm, N, codebooks, M, K,
                         fr, p.cn, p.scn, resid_norm);
    else
      hipLaunchKernelGGL(encode_mfma4_kernel<128>, g4, dim3(256), 0, st, rm, N, codebooks, M, K,
                         fr, p.cn, p.scn, resid_norm);
    LAP_LAUNCH_CHECK("encode_mfma4_kernel");
    return LAP_OK;
  }
  if (K % 16 == 0 && encode_impl_mfma()) {
    dim3 g16((N + 15) / 16);
    const uint2* fr = reinterpret_cast<const uint2*>(p.frag);
#define LAP_ENCM(D_)                                                                         \
  hipLaunchKernelGGL(encode_mfma_kernel<D_>, g16, dim3(EncCfg<D_>::THREADS), 0, st, rm, N,   \
                     codebooks, M, K, fr, p.cn, p.scn, resid_norm)
    if (D == 64) LAP_ENCM(64);
    else if (D == 128) LAP_ENCM(128);
    else LAP_ENCM(256);
#undef LAP_ENCM
    LAP_LAUNCH_CHECK("encode_mfma_kernel");
    return LAP_OK;
  }
  dim3 grid((N + 3) / 4);
#define LAP_ENC(D_)                                                                          \
  hipLaunchKernelGGL(encode_greedy_kernel<D_>, grid, dim3(256), 0, st, rm, N, codebooks, M,  \
                     K, p.ct, p.cn, resid_norm)
  if (D == 64) LAP_ENC(64);
  else if (D == 128) LAP_ENC(128);
  else LAP_ENC(256);
#undef LAP_ENC
  LAP_LAUNCH_CHECK("encode_greedy_kernel");
  return LAP_OK;
}

extern "C" int lap_encode_greedy(const float* x, int64_t x_row_stride, int N, int D,
                                 const float* codebooks, int M, int K, const void* prep,
                                 size_t prep_bytes, uint8_t* codes_out, int64_t codes_row_stride,
                                 float* resid_norm, lap_stream_t stream) {
  clear_error();
  LAP_CHECK(x && codes_out, "lap_encode_greedy: null pointer");
  LAP_CHECK(N >= 0 && D > 0 && M > 0, "lap_encode_greedy: bad sizes");
  LAP_CHECK(x_row_stride >= D && codes_row_stride >= M, "lap_encode_greedy: bad row strides");
  const RowMap rm{x, LAP_DTYPE_F32, 0, 0, x_row_stride, codes_out, 0, 0, codes_row_stride,
                  N > 0 ? N : 1, 1, 0, nullptr, 0};
  return run_encode(rm, N, D, codebooks, M, K, prep, prep_bytes, resid_norm, stream,
                    "lap_encode_greedy");
}

extern "C" int lap_encode_keys(const void* keys, int key_dtype, int64_t k_sb, int64_t k_sh,
                               int64_t k_st, int B, int Hkv, int t0, int t1, int D,
                               const float* codebooks, int M, int K, const void* prep,
                               size_t prep_bytes, uint8_t* codes, int64_t c_sb, int64_t c_sh,
                               int64_t c_st, float* resid_norm, lap_stream_t stream) {
  clear_error();
  LAP_CHECK(keys && codes, "lap_encode_keys: null pointer");
  LAP_CHECK(key_dtype == LAP_DTYPE_F32 || key_dtype == LAP_DTYPE_F16 ||
                key_dtype == LAP_DTYPE_BF16,
            "lap_encode_keys: keys must be f32, f16 or bf16");
  LAP_CHECK(B > 0 && Hkv > 0 && D > 0 && M > 0, "lap_encode_keys: bad sizes");
  LAP_CHECK(0 <= t0 && t0 <= t1, "lap_encode_keys: bad token range [%d, %d)", t0, t1);
  LAP_CHECK(k_st >= D && c_st >= M, "lap_encode_keys: token strides smaller than D / M");
  const int64_t n = (int64_t)B * Hkv * (t1 - t0);
  LAP_CHECK(n <= (int64_t)1 << 30, "lap_encode_keys: too many rows");
  const RowMap rm{keys, key_dtype, k_sb, k_sh, k_st, codes, c_sb, c_sh, c_st,
                  t1 > t0 ? t1 - t0 : 1, Hkv, t0, nullptr, 0};
  return run_encode(rm, (int)n, D, codebooks, M, K, prep, prep_bytes, resid_norm, stream,
                    "lap_encode_keys");
}

extern "C" int lap_encode_keys_ranges(const void* keys, int key_dtype, int64_t k_sb,
                                      int64_t k_sh, int64_t k_st, int B, int Hkv,
                                      const int32_t* ranges, int max_len, int t_cap, int D,
                                      const float* codebooks, int M, int K, const void* prep,
                                      size_t prep_bytes, uint8_t* codes, int64_t c_sb,
                                      int64_t c_sh, int64_t c_st, lap_stream_t stream) {
  clear_error();
  LAP_CHECK(keys && codes && ranges, "lap_encode_keys_ranges: null pointer");
  LAP_CHECK(key_dtype == LAP_DTYPE_F32 || key_dtype == LAP_DTYPE_F16 ||
                key_dtype == LAP_DTYPE_BF16,
            "lap_encode_keys_ranges: keys must be f32, f16 or bf16");
  LAP_CHECK(B > 0 && Hkv > 0 && D > 0 && M > 0 && max_len > 0 && t_cap > 0,
            "lap_encode_keys_ranges: bad sizes");
  LAP_CHECK(k_st >= D && c_st >= M, "lap_encode_keys_ranges: token strides smaller than D / M");
  const int64_t n = (int64_t)B * Hkv * max_len;
  LAP_CHECK(n <= (int64_t)1 << 30, "lap_encode_keys_ranges: too many rows");
  const RowMap rm{keys, key_dtype, k_sb, k_sh, k_st, codes, c_sb, c_sh, c_st,
                  max_len, Hkv, 0, ranges, t_cap};
  return run_encode(rm, (int)n, D, codebooks, M, K, prep, prep_bytes, nullptr, stream,
                    "lap_encode_keys_ranges");
}

extern "C" int lap_aq_reconstruct(const float* codebooks, int M, int K, int D, const void* codes,
                                  int codes_dtype, int64_t codes_row_stride, int N, float* out,
                                  lap_stream_t stream) {
  clear_error();
  LAP_CHECK(codebooks && codes && out, "lap_aq_reconstruct: null pointer");
  LAP_CHECK(M > 0 && K > 0 && D > 0 && N >= 0, "lap_aq_reconstruct: bad sizes");
  LAP_CHECK(D % 4 == 0, "lap_aq_reconstruct: D=%d must be a multiple of 4", D);
  LAP_CHECK(codes_row_stride >= M, "lap_aq_reconstruct: codes row stride %lld < M=%d",
            (long long)codes_row_stride, M);
  LAP_CHECK(codes_dtype == LAP_DTYPE_U8 || codes_dtype == LAP_DTYPE_I8 ||
                codes_dtype == LAP_DTYPE_I64,
            "codes must be int64 (Long) or uint8 (Byte) or int8 (Char)");
  LAP_CHECK((reinterpret_cast<uintptr_t>(codebooks) & 15) == 0 &&
                (reinterpret_cast<uintptr_t>(out) & 15) == 0,
            "lap_aq_reconstruct: codebooks and out must be 16-byte aligned");
  if (N == 0) return LAP_OK;
  DevInfo di;
  int s = device_info(&di);
  if (s != LAP_OK) return s;
  const int64_t total = (int64_t)N * (D / 4);
  const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 16LL * di.cu_count);
  hipStream_t st = as_stream(stream);
  if (codes_dtype == LAP_DTYPE_U8)
    hipLaunchKernelGGL(aq_reconstruct_kernel<uint8_t>, dim3(grid), dim3(256), 0, st, codebooks, M,
                       K, D, static_cast<const uint8_t*>(codes), codes_row_stride, N, out);
  else if (codes_dtype == LAP_DTYPE_I8)
    hipLaunchKernelGGL(aq_reconstruct_kernel<int8_t>, dim3(grid), dim3(256), 0, st, codebooks, M,
                       K, D, static_cast<const int8_t*>(codes), codes_row_stride, N, out);
  else
    hipLaunchKernelGGL(aq_reconstruct_kernel<int64_t>, dim3(grid), dim3(256), 0, st, codebooks,
                       M, K, D, static_cast<const int64_t*>(codes), codes_row_stride, N, out);
  LAP_LAUNCH_CHECK("aq_reconstruct_kernel");
  return LAP_OK;
}

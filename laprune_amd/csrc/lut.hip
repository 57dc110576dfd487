// lut.hip — A1: per-query-head AQ lookup table.
//
//   lut[h, m, k] = fp16_rne( sum_d q[h, d] * C[m, k, d] )
//
// with the sum taken as one fp32 fmaf chain over d = 0..D-1 starting from 0
// (the order the CPU oracle restates).  The reference forms this LUT with a
// vendor GEMM (laprune/llm/aq_kv.py:681-682) or an fp32 einsum (:620).
//
// Work shape: a workgroup owns a tile of 32 codebook rows (row = m*K + k) x
// 8*HPT query heads; thread t runs HPT independent fmaf chains, row t % 32
// against heads (t / 32) * HPT + j.  The 32 rows are one contiguous block of
// the [M*K][D] codebook, staged in LDS as fp32 with coalesced loads.  The
// chains need one codebook value and HPT query values per step; where the
// query values come from decides the cost:
//   * lut_dpp_kernel (D = 64 or 128): lane l keeps q[h][64 b + 4 (l % 16) + e]
//     in four VGPRs per 64-wide block b (one 8-byte load), and every FMA
//     takes its query operand through DPP row_newbcast:n (lane n of the
//     lane's 16-lane row), so LDS serves only the codebook: one ds_read_b128
//     per 4*HPT FMAs.
//   * lut_tile_kernel (any D): the query tile sits in LDS too and is read as
//     16-byte broadcasts, which makes the chains LDS-bound.
// The interleaved layout [Hq/G][M][K][G] is written directly (8 contiguous
// bytes per row and KV group) so the scorer can fill its LDS table with a
// linear copy.
#include "common.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>

namespace lap {
namespace {

constexpr int kTileRows = 32;    // codebook rows per workgroup
constexpr int kThreads = 256;
constexpr int kHeadGroups = kThreads / kTileRows;  // 8

// Load 4 consecutive elements of dtype DT at element offset i as fp32.
template <int DT>
__device__ __forceinline__ float4 load4(const void* p, int64_t i) {
  if (DT == LAP_DTYPE_F32) return *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
  const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
  if (DT == LAP_DTYPE_F16)
    return make_float4(h2f(w.x & 0xffffu), h2f(w.x >> 16), h2f(w.y & 0xffffu), h2f(w.y >> 16));
  return make_float4(bf2f(w.x & 0xffffu), bf2f(w.x >> 16), bf2f(w.y & 0xffffu), bf2f(w.y >> 16));
}

// Codebook rows sit in LDS with a row pitch of D + 4 floats: a 16-lane pass
// of ds_read_b128 over 16 consecutive rows then covers 64 distinct banks.
__host__ __device__ constexpr int c_pitch(int D) { return D + 4; }

// Stage the tile's 32 codebook rows in LDS.  Every load is issued before the
// first LDS write (at most 8 float4 per thread for D <= 256), unconditionally
// with clamped indices so that the compiler keeps them all in flight.
template <int CDT>
__device__ __forceinline__ void stage_rows(const void* __restrict__ cb, int D, int MK, int row0,
                                           float* s_c) {
  constexpr int kC = kTileRows * 64 / kThreads;
  const int D4 = D / 4, P = c_pitch(D), nC = kTileRows * D4;
  const int tid = threadIdx.x;
  float4 vc[kC];
#pragma unroll
  for (int j = 0; j < kC; ++j) {
    const int i = min(tid + j * kThreads, nC - 1);
    const int r = i / D4, d = (i - r * D4) * 4;
    vc[j] = load4<CDT>(cb, (int64_t)min(row0 + r, MK - 1) * D + d);
  }
#pragma unroll
  for (int j = 0; j < kC; ++j) {
    const int i = tid + j * kThreads;
    const int r = i / D4, d = (i - r * D4) * 4;
    if (i < nC) *reinterpret_cast<float4*>(s_c + r * P + d) = vc[j];
  }
}

// Write the thread's HPT results for one row (heads h0 .. h0 + HPT - 1).
template <int HPT>
__device__ __forceinline__ void write_row(const float (&acc)[HPT], int h0, int row, int Hq,
                                          int MK, int G, int layout, uint16_t* __restrict__ out) {
#pragma unroll
  for (int j0 = 0; j0 < HPT; j0 += 4) {
    const int h = h0 + j0;
    if (layout == LAP_LUT_GMKG && G == 4 && h + 3 < Hq) {
      // the four heads of one KV group: 8 contiguous bytes; 32 lanes write
      // 256 contiguous bytes
      const uint32_t w0 = (uint32_t)f2h(acc[j0]) | ((uint32_t)f2h(acc[j0 + 1]) << 16);
      const uint32_t w1 = (uint32_t)f2h(acc[j0 + 2]) | ((uint32_t)f2h(acc[j0 + 3]) << 16);
      *reinterpret_cast<uint2*>(out + ((int64_t)(h >> 2) * MK + row) * 4) = make_uint2(w0, w1);
      continue;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int head = h + j;
      if (head >= Hq) continue;
      int64_t idx;
      if (layout == LAP_LUT_HMK) idx = (int64_t)head * MK + row;
      else idx = ((int64_t)(head / G) * MK + row) * G + (head % G);
      out[idx] = f2h(acc[j0 + j]);
    }
  }
}

// Sixteen steps of one chain, d = 64 B + 4 n + e for n = N0..N0+3, e = 0..3
// (ascending d):  acc = fmaf(q[h][d], c[d], acc).  Lane l holds
// q[h][64 B + 4 (l % 16) + e] in qv[e], so q[h][d] is lane n of the lane's
// 16-lane row of qv[e] (DPP row_newbcast:n).  A DPP source VGPR written by a
// VALU instruction needs two wait states before it is read; the leading s_nop
// covers that for qv, and nothing inside the block writes qv.
#define LAP_FMA_DPP(N, E, C) \
  "v_fmac_f32_dpp %0, %" #E ", %" #C " row_newbcast:" #N " row_mask:0xf bank_mask:0xf\n\t"
#define LAP_FMA16(N0, N1, N2, N3)                                                           \
  template <>                                                                              \
  __device__ __forceinline__ void fma16_bcast<N0>(float& acc, const float(&qv)[4],         \
                                                  const float4& c0, const float4& c1,      \
                                                  const float4& c2, const float4& c3) {    \
    asm("s_nop 1\n\t"                                                                      \
        LAP_FMA_DPP(N0, 1, 5) LAP_FMA_DPP(N0, 2, 6) LAP_FMA_DPP(N0, 3, 7) LAP_FMA_DPP(N0, 4, 8) \
        LAP_FMA_DPP(N1, 1, 9) LAP_FMA_DPP(N1, 2, 10) LAP_FMA_DPP(N1, 3, 11)                  \
        LAP_FMA_DPP(N1, 4, 12) LAP_FMA_DPP(N2, 1, 13) LAP_FMA_DPP(N2, 2, 14)                 \
        LAP_FMA_DPP(N2, 3, 15) LAP_FMA_DPP(N2, 4, 16) LAP_FMA_DPP(N3, 1, 17)                 \
        LAP_FMA_DPP(N3, 2, 18) LAP_FMA_DPP(N3, 3, 19) LAP_FMA_DPP(N3, 4, 20)                 \
        : "+v"(acc)                                                                        \
        : "v"(qv[0]), "v"(qv[1]), "v"(qv[2]), "v"(qv[3]), "v"(c0.x), "v"(c0.y), "v"(c0.z),  \
          "v"(c0.w), "v"(c1.x), "v"(c1.y), "v"(c1.z), "v"(c1.w), "v"(c2.x), "v"(c2.y),      \
          "v"(c2.z), "v"(c2.w), "v"(c3.x), "v"(c3.y), "v"(c3.z), "v"(c3.w));                 \
  }
template <int N0>
__device__ __forceinline__ void fma16_bcast(float& acc, const float (&qv)[4], const float4& c0,
                                            const float4& c1, const float4& c2,
                                            const float4& c3);
LAP_FMA16(0, 1, 2, 3)
LAP_FMA16(4, 5, 6, 7)
LAP_FMA16(8, 9, 10, 11)
LAP_FMA16(12, 13, 14, 15)
#undef LAP_FMA16
#undef LAP_FMA_DPP

// Workgroup -> (head tile, first row tile).  A workgroup computes `tpw`
// consecutive row tiles with the same heads: its query values are loaded once
// and the next tile's codebook rows are fetched while the current one is
// computed.  Workgroups are dispatched to the eight XCDs round-robin
// (workgroup i to XCD i % 8) and each XCD has its own L2, so XCD x takes a
// contiguous range of work units with all head tiles of a row group back to
// back: every codebook row is then fetched into one L2 only.
struct TileId {
  int row_tile, head_tile;
};
__device__ __forceinline__ TileId tile_of(int wg, int n_wg, int head_tiles, int tpw) {
  constexpr int kXcds = 8;
  const int u = n_wg % kXcds == 0 ? (wg % kXcds) * (n_wg / kXcds) + wg / kXcds : wg;
  return TileId{(u / head_tiles) * tpw, u % head_tiles};
}

// Issue the loads of one tile's 32 codebook rows (at most 8 float4 per
// thread for D <= 256), unconditionally with clamped indices so that the
// compiler keeps them all in flight; rows_to_lds writes them.
template <int CDT, int D>
__device__ __forceinline__ void rows_load(const void* __restrict__ cb, int MK, int row0,
                                          float4 (&vc)[kTileRows * D / 4 / kThreads]) {
  constexpr int D4 = D / 4, kC = kTileRows * D4 / kThreads;
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < kC; ++j) {
    const int i = tid + j * kThreads;
    const int r = i / D4, d = (i - r * D4) * 4;
    vc[j] = load4<CDT>(cb, (int64_t)min(row0 + r, MK - 1) * D + d);
  }
}
template <int D>
__device__ __forceinline__ void rows_to_lds(const float4 (&vc)[kTileRows * D / 4 / kThreads],
                                            float* s_c) {
  constexpr int D4 = D / 4, kC = kTileRows * D4 / kThreads;
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < kC; ++j) {
    const int i = tid + j * kThreads;
    const int r = i / D4, d = (i - r * D4) * 4;
    *reinterpret_cast<float4*>(s_c + r * c_pitch(D) + d) = vc[j];
  }
}

template <int QDT, int CDT, int HPT, int D>
__global__ __launch_bounds__(kThreads) void lut_dpp_kernel(
    const void* __restrict__ q, int64_t q_row_stride,
    const void* __restrict__ cb, int Hq, int MK, int G, int layout,
    uint16_t* __restrict__ out, int head_tiles, int tpw) {
  static_assert(HPT % 4 == 0 && D % 64 == 0 && D <= 256, "bad shape");
  constexpr int NB = D / 64;
  constexpr int P = c_pitch(D);
  __shared__ __attribute__((aligned(16))) float s_c[kTileRows * P];
  const int tid = threadIdx.x;
  const TileId ti = tile_of(blockIdx.x, gridDim.x, head_tiles, tpw);
  const int h0 = ti.head_tile * (kHeadGroups * HPT) + (tid / kTileRows) * HPT;
  const int row_tiles = (MK + kTileRows - 1) / kTileRows;
  const int n_tiles = min(tpw, row_tiles - ti.row_tile);

  float4 vc[kTileRows * D / 4 / kThreads];
  rows_load<CDT, D>(cb, MK, ti.row_tile * kTileRows, vc);
  // This lane's query values: qv[j][B][e] = q[h0 + j][64 B + 4 (lane % 16) + e]
  // (heads past Hq read the last head; their results are not written).
  float qv[HPT][NB][4];
  const int n = tid & 15;
#pragma unroll
  for (int j = 0; j < HPT; ++j) {
    const int64_t base = (int64_t)min(h0 + j, Hq - 1) * q_row_stride + 4 * n;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float4 v = load4<QDT>(q, base + 64 * b);
      qv[j][b][0] = v.x;
      qv[j][b][1] = v.y;
      qv[j][b][2] = v.z;
      qv[j][b][3] = v.w;
    }
  }
  rows_to_lds<D>(vc, s_c);

  const float* cr = s_c + (tid % kTileRows) * P;
  for (int t = 0; t < n_tiles; ++t) {
    __syncthreads();  // tile t is in LDS
    const int row0 = (ti.row_tile + t) * kTileRows;
    if (t + 1 < n_tiles) rows_load<CDT, D>(cb, MK, row0 + kTileRows, vc);
    float acc[HPT];
#pragma unroll
    for (int j = 0; j < HPT; ++j) acc[j] = 0.f;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {  // d = 64 b + 16 g .. + 15
        const float* cp = cr + 64 * b + 16 * g;
        const float4 c0 = *reinterpret_cast<const float4*>(cp);
        const float4 c1 = *reinterpret_cast<const float4*>(cp + 4);
        const float4 c2 = *reinterpret_cast<const float4*>(cp + 8);
        const float4 c3 = *reinterpret_cast<const float4*>(cp + 12);
#pragma unroll
        for (int j = 0; j < HPT; ++j) {
          if (g == 0) fma16_bcast<0>(acc[j], qv[j][b], c0, c1, c2, c3);
          else if (g == 1) fma16_bcast<4>(acc[j], qv[j][b], c0, c1, c2, c3);
          else if (g == 2) fma16_bcast<8>(acc[j], qv[j][b], c0, c1, c2, c3);
          else fma16_bcast<12>(acc[j], qv[j][b], c0, c1, c2, c3);
        }
      }
    }
    const int row = row0 + tid % kTileRows;
    if (row < MK) write_row<HPT>(acc, h0, row, Hq, MK, G, layout, out);
    if (t + 1 < n_tiles) {
      __syncthreads();  // every read of tile t is done
      rows_to_lds<D>(vc, s_c);
    }
  }
}

// ---- fp32 MFMA form.  v_mfma_f32_16x16x4f32 accumulates its four k terms
// into each output as four fused multiply-adds in ascending k: measured on
// gfx950 bit for bit against a per-element fmaf chain (random, mixed-exponent,
// cancelling, subnormal and signed-zero operands, K up to 512), and checked
// here by every LUT test against the CPU oracle.  So a chain of these MFMAs
// over k-blocks 0, 4, 8, ... from a zero accumulator is the contract's fmaf
// chain over d, on the matrix cores.
//   A = q (16 heads: lane l supplies head l % 16, d = 4 j + l / 16)
//   B = C^T (16 codebook rows: lane l supplies row l % 16, d = 4 j + l / 16)
//   D: lane l holds heads 4 (l / 16) + e, row l % 16: the four heads of one
//      KV group for one row, 8 contiguous bytes of the interleaved layout.
// In LDS each head or row keeps its d in the order (d % 4, d / 4): lane group
// l / 16 then finds the operands of four consecutive k-blocks in 16
// contiguous bytes, one ds_read_b128 per four MFMAs.  Pitch D + 4 floats:
// the 16 lanes of one pass land on 64 distinct banks.
// A workgroup (4 waves) owns 16 HT heads x 16 RTW (4 / HT) rows; wave w takes
// head tile w % HT and RTW row tiles, reusing each q value RTW times.
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__host__ __device__ constexpr int mfma_rows(int HT, int RTW) { return 16 * RTW * (4 / HT); }

// Staging of n rows of D values (row i from src at min(base + i, last) *
// stride) in the (d % 4, d / 4) order: a thread moves 16 consecutive d per
// unit.  The loads and the LDS writes are separate steps so that a caller can
// issue every global load before its first LDS access.
template <int D, int N, int TH = kThreads>
struct MfmaStage {
  static constexpr int UPR = D / 16, NU = N * UPR, PER = (NU + TH - 1) / TH;
  float4 v[PER][4];

  template <int DT>
  __device__ __forceinline__ void load(const void* __restrict__ src, int64_t stride, int base,
                                       int last, int tid) {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int u = min(tid + k * TH, NU - 1);
      const int r = u / UPR, d0 = (u % UPR) * 16;
      const int64_t off = (int64_t)min(base + r, last) * stride + d0;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[k][i] = load4<DT>(src, off + 4 * i);
    }
  }

  __device__ __forceinline__ void store(float* __restrict__ dst, int tid) const {
    constexpr int P = c_pitch(D);
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int u = min(tid + k * TH, NU - 1);
      const int r = u / UPR, j0 = (u % UPR) * 4;
      float* row = dst + r * P + j0;
      *reinterpret_cast<float4*>(row) = make_float4(v[k][0].x, v[k][1].x, v[k][2].x, v[k][3].x);
      *reinterpret_cast<float4*>(row + D / 4) =
          make_float4(v[k][0].y, v[k][1].y, v[k][2].y, v[k][3].y);
      *reinterpret_cast<float4*>(row + D / 2) =
          make_float4(v[k][0].z, v[k][1].z, v[k][2].z, v[k][3].z);
      *reinterpret_cast<float4*>(row + 3 * D / 4) =
          make_float4(v[k][0].w, v[k][1].w, v[k][2].w, v[k][3].w);
    }
  }
};

// acc[t] += q-tile x rows 16 t .. 16 t + 15 of the staged tile, over all D:
// for each block of 16 d, four ds_read_b128 (one per row tile) then sixteen
// MFMAs.  The operands of block jb + 1 are read before the MFMAs of block jb
// issue, so the LDS latency hides behind the matrix pipe even with one wave
// per SIMD; the scheduling barriers keep the compiler from regrouping them.
template <int D, int NT>
__device__ __forceinline__ void mfma_tile_chain(const float4 (&a)[D / 16], const float* cp,
                                                f32x4_t (&acc)[NT]) {
  constexpr int P = c_pitch(D);
  float4 bc[NT], bn[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) bc[t] = *reinterpret_cast<const float4*>(cp + t * 16 * P);
#pragma unroll
  for (int jb = 0; jb < D / 16; ++jb) {
    if (jb + 1 < D / 16) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        bn[t] = *reinterpret_cast<const float4*>(cp + t * 16 * P + 4 * (jb + 1));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[jb].x, bc[t].x, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[jb].y, bc[t].y, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[jb].z, bc[t].z, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[jb].w, bc[t].w, acc[t], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < NT; ++t) bc[t] = bn[t];
  }
}

template <int QDT, int CDT, int HT, int RTW, int D>
__global__ __launch_bounds__(kThreads) void lut_mfma_kernel(
    const void* __restrict__ q, int64_t q_row_stride,
    const void* __restrict__ cb, int Hq, int MK, int G, int layout,
    uint16_t* __restrict__ out, int head_tiles) {
  constexpr int ROWS = mfma_rows(HT, RTW), HEADS = 16 * HT, P = c_pitch(D);
  // Each wave keeps its 16 heads' q (D / 4 floats per lane) in registers.
  // With 64 x 64 tiles one LDS region holds the q tile, then the codebook tile
  // (half the LDS, so four workgroups fit per CU); smaller tiles stage both at
  // once in two regions.
  constexpr bool kShare = HT == 4;
  extern __shared__ __attribute__((aligned(16))) float mfma_smem[];
  float* const s_q = kShare ? mfma_smem : mfma_smem + ROWS * P;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const TileId ti = tile_of(blockIdx.x, gridDim.x, head_tiles, 1);
  const int row0 = ti.row_tile * ROWS, head0 = ti.head_tile * HEADS;
  MfmaStage<D, ROWS> sc;
  MfmaStage<D, HEADS> sq;
  sc.template load<CDT>(cb, D, row0, MK - 1, tid);
  sq.template load<QDT>(q, q_row_stride, head0, Hq - 1, tid);
  sq.store(s_q, tid);
  if (!kShare) sc.store(mfma_smem, tid);
  __syncthreads();

  const int ht = wave % HT, rt0 = (wave / HT) * RTW;
  const int hl = lane & 15, kj = lane >> 4;
  float4 a[D / 16];
  {
    const float* qp = s_q + (ht * 16 + hl) * P + kj * (D / 4);
#pragma unroll
    for (int jb = 0; jb < D / 16; ++jb) a[jb] = *reinterpret_cast<const float4*>(qp + 4 * jb);
  }
  if (kShare) {
    __syncthreads();
    sc.store(mfma_smem, tid);
    __syncthreads();
  }

  const float* cp = mfma_smem + (rt0 * 16 + hl) * P + kj * (D / 4);
  f32x4_t acc[RTW];
#pragma unroll
  for (int i = 0; i < RTW; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  mfma_tile_chain<D, RTW>(a, cp, acc);
  const int hA = head0 + ht * 16 + 4 * kj;
#pragma unroll
  for (int i = 0; i < RTW; ++i) {
    const int row = row0 + (rt0 + i) * 16 + hl;
    if (row >= MK) continue;
    const float r4[4] = {acc[i][0], acc[i][1], acc[i][2], acc[i][3]};
    write_row<4>(r4, hA, row, Hq, MK, G, layout, out);
  }
}

// The 64 x 64 form over `tpw` consecutive row tiles of one head tile: the
// workgroup's q fragments stay in registers, the codebook tile is staged in
// one of two LDS buffers, and the next tile's rows are requested from global
// memory before the current tile's MFMA chain, so their latency runs under
// it.  One barrier per tile: after it, the buffer just read may be written.
// (With every tile its own workgroup, the four workgroups a CU holds load,
// compute and write in step, and nothing overlaps the loads.)
template <int QDT, int CDT, int D>
__global__ __launch_bounds__(kThreads) void lut_mfma_pipe_kernel(
    const void* __restrict__ q, int64_t q_row_stride,
    const void* __restrict__ cb, int Hq, int MK, int G, int layout,
    uint16_t* __restrict__ out, int head_tiles, int tpw) {
  constexpr int HT = 4, RTW = 4, ROWS = mfma_rows(HT, RTW), HEADS = 16 * HT, P = c_pitch(D);
  static_assert(ROWS == 64 && HEADS == 64, "64 x 64 tiles");
  extern __shared__ __attribute__((aligned(16))) float mfma_smem[];
  float* const buf0 = mfma_smem;
  float* const buf1 = mfma_smem + ROWS * P;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const TileId ti = tile_of(blockIdx.x, gridDim.x, head_tiles, tpw);
  const int n_rt = (MK + ROWS - 1) / ROWS;
  const int n_t = min(tpw, n_rt - ti.row_tile);
  if (n_t <= 0) return;
  const int head0 = ti.head_tile * HEADS;
  MfmaStage<D, ROWS> sc;
  MfmaStage<D, HEADS> sq;
  sc.template load<CDT>(cb, D, ti.row_tile * ROWS, MK - 1, tid);
  sq.template load<QDT>(q, q_row_stride, head0, Hq - 1, tid);
  sq.store(buf1, tid);
  sc.store(buf0, tid);
  __syncthreads();
  // wave w takes head tile w; every wave covers the tile's four row tiles
  const int hl = lane & 15, kj = lane >> 4;
  float4 a[D / 16];
  {
    const float* qp = buf1 + (wave * 16 + hl) * P + kj * (D / 4);
#pragma unroll
    for (int jb = 0; jb < D / 16; ++jb) a[jb] = *reinterpret_cast<const float4*>(qp + 4 * jb);
  }
  __syncthreads();  // buf1 (the q tile) is read: it may take tile 1
  const int hA = head0 + wave * 16 + 4 * kj;
  for (int t = 0; t < n_t; ++t) {
    const float* cur = (t & 1) ? buf1 : buf0;
    float* nxt = (t & 1) ? buf0 : buf1;
    const int row0 = (ti.row_tile + t) * ROWS;
    const bool more = t + 1 < n_t;
    if (more) sc.template load<CDT>(cb, D, row0 + ROWS, MK - 1, tid);
    f32x4_t acc[RTW];
#pragma unroll
    for (int i = 0; i < RTW; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    mfma_tile_chain<D, RTW>(a, cur + hl * P + kj * (D / 4), acc);
#pragma unroll
    for (int i = 0; i < RTW; ++i) {
      const int row = row0 + i * 16 + hl;
      if (row >= MK) continue;
      const float r4[4] = {acc[i][0], acc[i][1], acc[i][2], acc[i][3]};
      write_row<4>(r4, hA, row, Hq, MK, G, layout, out);
    }
    // nxt was last read at tile t - 1 (or held q), before the previous barrier
    if (more) sc.store(nxt, tid);
    __syncthreads();
  }
}

template <int QDT, int CDT, int HPT>
__global__ __launch_bounds__(kThreads) void lut_tile_kernel(
    const void* __restrict__ q, int64_t q_row_stride,
    const void* __restrict__ cb, int Hq, int D, int MK, int G, int layout,
    uint16_t* __restrict__ out) {
  static_assert(HPT % 4 == 0, "heads per thread must be a multiple of 4");
  constexpr int TH = kHeadGroups * HPT;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int P = c_pitch(D);
  float* s_c = smem;                   // [32][P]
  float* s_q = smem + kTileRows * P;   // [TH][D]
  const int tid = threadIdx.x;
  const int row0 = blockIdx.x * kTileRows;
  const int head0 = blockIdx.y * TH;
  const int D4 = D / 4;

  for (int i = tid; i < TH * D4; i += kThreads) {
    const int h = i / D4, d = (i - h * D4) * 4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (head0 + h < Hq) v = load4<QDT>(q, (int64_t)(head0 + h) * q_row_stride + d);
    *reinterpret_cast<float4*>(s_q + h * D + d) = v;
  }
  stage_rows<CDT>(cb, D, MK, row0, s_c);
  __syncthreads();

  const int hg = tid / kTileRows;
  const float* cr = s_c + (tid % kTileRows) * P;
  const float* qh = s_q + hg * HPT * D;
  float acc[HPT];
#pragma unroll
  for (int j = 0; j < HPT; ++j) acc[j] = 0.f;
#pragma unroll 4
  for (int d = 0; d < D; d += 4) {
    const float4 c = *reinterpret_cast<const float4*>(cr + d);
#pragma unroll
    for (int j = 0; j < HPT; ++j) {
      const float4 qq = *reinterpret_cast<const float4*>(qh + j * D + d);
      acc[j] = __builtin_fmaf(qq.x, c.x, acc[j]);
      acc[j] = __builtin_fmaf(qq.y, c.y, acc[j]);
      acc[j] = __builtin_fmaf(qq.z, c.z, acc[j]);
      acc[j] = __builtin_fmaf(qq.w, c.w, acc[j]);
    }
  }
  const int row = row0 + tid % kTileRows;
  if (row < MK) write_row<HPT>(acc, head0 + hg * HPT, row, Hq, MK, G, layout, out);
}

size_t lut_tile_smem_bytes(int D) {
  return ((size_t)kTileRows * c_pitch(D) + (size_t)kHeadGroups * 4 * D) * sizeof(float);
}

// Heads per thread: 8 when there are enough heads to give every CU several
// tiles (batched decode), else 4 (batch 1 at Hq = 32: 256 tiles).
int lut_heads_per_thread(int Hq, int MK, const DevInfo& di) {
  const int64_t tiles = (int64_t)(MK + kTileRows - 1) / kTileRows;
  return tiles * ((Hq + 8 * kHeadGroups - 1) / (8 * kHeadGroups)) >= 4 * di.cu_count ? 8 : 4;
}

// Row tiles per workgroup: enough workgroups for four per CU, the rest as
// consecutive tiles of one workgroup.  LAPRUNE_LUT_TPW overrides it.
int lut_tiles_per_wg(int Hq, int MK, int hpt, const DevInfo& di) {
  static const int forced = [] {
    const char* e = getenv("LAPRUNE_LUT_TPW");
    return e ? atoi(e) : 0;
  }();
  if (forced > 0) return forced;
  const int64_t tiles = (int64_t)((MK + kTileRows - 1) / kTileRows) *
                        ((Hq + hpt * kHeadGroups - 1) / (hpt * kHeadGroups));
  const int64_t t = tiles / (4 * (int64_t)di.cu_count);
  return t < 1 ? 1 : (int)t;
}

// LAPRUNE_LUT_IMPL=dpp selects the VALU kernels (measurements, cross-checks);
// the fp32-MFMA kernel is the default.  Read at every call, so that one
// process can run both.
bool lut_impl_mfma() {
  const char* e = getenv("LAPRUNE_LUT_IMPL");
  return !(e && strcmp(e, "dpp") == 0);
}

// fp32-MFMA LUT (D = 64 or 128): 64 x 64 tiles (four row tiles per wave)
// once there are two of them per CU, else 32 x 32 tiles (one per wave).
bool lut_mfma_ok(int D) { return lut_impl_mfma() && (D == 64 || D == 128); }

constexpr size_t lut_mfma_smem_bytes(int D, int HT, int RTW) {
  const int rows = HT == 4 ? std::max(mfma_rows(HT, RTW), 16 * HT) : mfma_rows(HT, RTW) + 16 * HT;
  return (size_t)rows * c_pitch(D) * sizeof(float);
}

// Row tiles per workgroup of the pipelined 64 x 64 form: enough workgroups
// for two per CU (each holds two 33 KiB tile buffers); 1 keeps one tile per
// workgroup (lut_mfma_kernel).  LAPRUNE_LUT_MFMA_TPW overrides it (read at
// every call, for measurements).
static int lut_mfma_tpw(int64_t tiles, int cus) {
  const char* e = getenv("LAPRUNE_LUT_MFMA_TPW");
  if (e && atoi(e) > 0) return atoi(e);
  const int64_t t = tiles / (2 * (int64_t)cus);
  return t < 1 ? 1 : (int)std::min<int64_t>(t, 8);
}

template <int QDT, int CDT, int D>
void launch_lut_mfma_d(const void* q, int64_t qs, const void* cb, int Hq, int MK, int G,
                       int layout, uint16_t* out, int cus, hipStream_t st) {
  const int64_t big_tiles = (int64_t)((MK + 63) / 64) * ((Hq + 63) / 64);
  const int tpw = lut_mfma_tpw(big_tiles, cus);
  if (Hq >= 64 && big_tiles >= 2 * cus && tpw > 1) {
    const int htl = (Hq + 63) / 64;
    const int units = (int)(((MK + 63) / 64 + tpw - 1) / tpw) * htl;
    hipLaunchKernelGGL((lut_mfma_pipe_kernel<QDT, CDT, D>), dim3((unsigned)units),
                       dim3(kThreads), 2 * lut_mfma_smem_bytes(D, 4, 4), st, q, qs, cb, Hq, MK,
                       G, layout, out, htl, tpw);
  } else if (Hq >= 64 && big_tiles >= 2 * cus) {
    const int htl = (Hq + 63) / 64;
    const dim3 g((unsigned)(((MK + 63) / 64) * htl));
    hipLaunchKernelGGL((lut_mfma_kernel<QDT, CDT, 4, 4, D>), g, dim3(kThreads),
                       lut_mfma_smem_bytes(D, 4, 4), st, q, qs, cb, Hq, MK, G, layout, out, htl);
  } else {
    const int htl = (Hq + 31) / 32;
    const dim3 g((unsigned)(((MK + 31) / 32) * htl));
    hipLaunchKernelGGL((lut_mfma_kernel<QDT, CDT, 2, 1, D>), g, dim3(kThreads),
                       lut_mfma_smem_bytes(D, 2, 1), st, q, qs, cb,
                       Hq, MK, G, layout, out, htl);
  }
}

template <int QDT, int CDT>
void launch_lut_mfma(const void* q, int64_t qs, const void* cb, int Hq, int D, int MK, int G,
                     int layout, uint16_t* out, int cus, hipStream_t st) {
  if (D == 64) launch_lut_mfma_d<QDT, CDT, 64>(q, qs, cb, Hq, MK, G, layout, out, cus, st);
  else launch_lut_mfma_d<QDT, CDT, 128>(q, qs, cb, Hq, MK, G, layout, out, cus, st);
}

template <int QDT, int CDT, int HPT>
void launch_hpt(const void* q, int64_t qs, const void* cb, int Hq, int D, int MK, int G,
                int layout, uint16_t* out, int tpw, hipStream_t st) {
  const int row_tiles = (MK + kTileRows - 1) / kTileRows;
  const int head_tiles = (Hq + kHeadGroups * HPT - 1) / (kHeadGroups * HPT);
  const int groups = (row_tiles + tpw - 1) / tpw;
  const dim3 grid((unsigned)(groups * head_tiles));
  if (D == 128)
    hipLaunchKernelGGL((lut_dpp_kernel<QDT, CDT, HPT, 128>), grid, dim3(kThreads), 0, st, q, qs,
                       cb, Hq, MK, G, layout, out, head_tiles, tpw);
  else if (D == 64)
    hipLaunchKernelGGL((lut_dpp_kernel<QDT, CDT, HPT, 64>), grid, dim3(kThreads), 0, st, q, qs,
                       cb, Hq, MK, G, layout, out, head_tiles, tpw);
  else
    hipLaunchKernelGGL((lut_tile_kernel<QDT, CDT, 4>), dim3(row_tiles, (Hq + 31) / 32),
                       dim3(kThreads), lut_tile_smem_bytes(D), st, q, qs, cb, Hq, D, MK, G,
                       layout, out);
}

template <int QDT>
hipError_t launch_lut(const void* q, int64_t qs, const void* cb, int cb_dtype, int Hq, int D,
                      int MK, int G, int layout, uint16_t* out, int hpt, int tpw, int cus,
                      hipStream_t st) {
  if (lut_mfma_ok(D)) {
    if (cb_dtype == LAP_DTYPE_F32)
      launch_lut_mfma<QDT, LAP_DTYPE_F32>(q, qs, cb, Hq, D, MK, G, layout, out, cus, st);
    else
      launch_lut_mfma<QDT, LAP_DTYPE_F16>(q, qs, cb, Hq, D, MK, G, layout, out, cus, st);
    return hipGetLastError();
  }
  if (cb_dtype == LAP_DTYPE_F32) {
    if (hpt == 8) launch_hpt<QDT, LAP_DTYPE_F32, 8>(q, qs, cb, Hq, D, MK, G, layout, out, tpw, st);
    else launch_hpt<QDT, LAP_DTYPE_F32, 4>(q, qs, cb, Hq, D, MK, G, layout, out, tpw, st);
  } else {
    if (hpt == 8) launch_hpt<QDT, LAP_DTYPE_F16, 8>(q, qs, cb, Hq, D, MK, G, layout, out, tpw, st);
    else launch_hpt<QDT, LAP_DTYPE_F16, 4>(q, qs, cb, Hq, D, MK, G, layout, out, tpw, st);
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
  // q and codebook rows are read four elements at a time (8 or 16 bytes)
  const uintptr_t q_align = q_dtype == LAP_DTYPE_F32 ? 16 : 8;
  const uintptr_t cb_align = cb_dtype == LAP_DTYPE_F32 ? 16 : 8;
  LAP_CHECK(reinterpret_cast<uintptr_t>(q) % q_align == 0 && q_row_stride % 4 == 0,
            "lap_lut_build: q must be %d-byte aligned with a row stride that is a multiple of 4",
            (int)q_align);
  LAP_CHECK(reinterpret_cast<uintptr_t>(codebooks) % cb_align == 0,
            "lap_lut_build: codebooks must be %d-byte aligned", (int)cb_align);
  LAP_CHECK(layout == LAP_LUT_HMK || layout == LAP_LUT_GMKG, "lap_lut_build: bad layout");
  if (layout == LAP_LUT_GMKG)
    LAP_CHECK(G > 0 && Hq % G == 0, "lap_lut_build: Hq=%d not divisible by G=%d", Hq, G);
  LAP_CHECK((int64_t)M * K <= (1 << 30), "lap_lut_build: M*K too large");
  DevInfo di;
  int ds = device_info(&di);
  if (ds != LAP_OK) return ds;
  const size_t smem = lut_tile_smem_bytes(D);
  LAP_CHECK_CODE(smem <= (size_t)di.lds_per_block, LAP_ERR_UNSUPPORTED,
                 "lap_lut_build: D=%d needs %zu bytes of LDS", D, smem);
  const int MK = M * K;
  const int hpt = lut_heads_per_thread(Hq, MK, di);
  const int tpw = lut_tiles_per_wg(Hq, MK, hpt, di);
  hipError_t e;
  uint16_t* out = static_cast<uint16_t*>(lut_out);
  hipStream_t st = as_stream(stream);
  switch (q_dtype) {
    case LAP_DTYPE_F32:
      e = launch_lut<LAP_DTYPE_F32>(q, q_row_stride, codebooks, cb_dtype, Hq, D, MK, G, layout,
                                    out, hpt, tpw, di.cu_count, st);
      break;
    case LAP_DTYPE_F16:
      e = launch_lut<LAP_DTYPE_F16>(q, q_row_stride, codebooks, cb_dtype, Hq, D, MK, G, layout,
                                    out, hpt, tpw, di.cu_count, st);
      break;
    default:
      e = launch_lut<LAP_DTYPE_BF16>(q, q_row_stride, codebooks, cb_dtype, Hq, D, MK, G, layout,
                                     out, hpt, tpw, di.cu_count, st);
      break;
  }
  LAP_HIP(e, "lap_lut_build launch");
  return LAP_OK;
}

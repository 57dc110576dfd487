// attn_core.h — the decode attention's MFMA wave step and online softmax,
// shared by the split-K decode kernels (attn.hip) and the fused decode
// step (step.hip).
#pragma once

#include "common.h"

namespace lap {
namespace {

constexpr int kTile = 64;     // keys per workgroup step (4 waves x 16)
constexpr int kKeys = 16;     // keys per wave step
constexpr float kLog2e = 1.4426950408889634f;

template <int DT>
__device__ __forceinline__ float ld16(const uint16_t v) {
  return DT == LAP_DTYPE_F16 ? h2f(v) : bf2f(v);
}
template <int DT>
__device__ __forceinline__ uint16_t st16(float f) {
  return DT == LAP_DTYPE_F16 ? f2h(f) : f2bf(f);
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16x16x16 MFMA in the data type (fp32 accumulate).
template <int DT>
__device__ __forceinline__ f32x4 mfma16(i16x4 a, i16x4 b, f32x4 c) {
  if constexpr (DT == LAP_DTYPE_F16)
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// One wave step = 16 keys, computed with 16x16x16 MFMAs.  Operand layouts
// (lane l, r = l / 16, c = l % 16):
//   q.k:  A = K (row = key c), B = Q^T (column = head c); the reduction index
//         4r + e of k-step ks stands for dim r * D/4 + 4 ks + e, so a lane
//         needs one contiguous quarter row of K.  Output: lane l holds the
//         scores of keys 4r + e for head c.
//   p.V:  A = P (row = head c, reduction index = key 4r + e): exactly the
//         score layout, no data movement.  B = V with column c of chunk ch
//         standing for dim c * D/16 + ch, so a lane needs D/16 contiguous
//         values of each of its four keys.  Output: lane l holds o for heads
//         4r + e and dims c * D/16 + ch.
template <int D>
struct KvStep {
  static constexpr int NK = D / 32;  // uint4 of K per lane (a quarter row)
  static constexpr int NV = D / 32;  // dwords of V per key per lane (D/16 values)
  uint4 k[NK];
  uint32_t v[4][NV];
  int tv[4];  // cache rows of keys 4r + e (-1: invalid)
  int mk[4];  // heads that keep keys 4r + e (bit c: head c), read by masked steps
};

// The K quarter rows of key lane % 16 (lane row r = lane / 16 reads quarter r).
template <int D>
__device__ __forceinline__ void k_issue(KvStep<D>& st, const uint16_t* __restrict__ kb,
                                        int64_t k_st, int tok, int r) {
  const uint4* kp = reinterpret_cast<const uint4*>(kb + (int64_t)(tok < 0 ? 0 : tok) * k_st +
                                                   r * (D / 4));
#pragma unroll
  for (int i = 0; i < KvStep<D>::NK; ++i) st.k[i] = kp[i];
}

// The D/16 values (from c * D/16) of key 4r + e's V row tv.
template <int D>
__device__ __forceinline__ void v_issue(KvStep<D>& st, const uint16_t* __restrict__ vb,
                                        int64_t v_st, int e, int tv, int c) {
  st.tv[e] = tv;
  const uint16_t* vp = vb + (int64_t)(tv < 0 ? 0 : tv) * v_st + c * (D / 16);
  if (KvStep<D>::NV == 2) {
    const uint2 w = *reinterpret_cast<const uint2*>(vp);
    st.v[e][0] = w.x;
    st.v[e][1] = w.y;
  } else {
#pragma unroll
    for (int i = 0; i < KvStep<D>::NV; i += 4) {
      const uint4 w = reinterpret_cast<const uint4*>(vp)[i / 4];
      st.v[e][i] = w.x;
      st.v[e][i + 1] = w.y;
      st.v[e][i + 2] = w.z;
      st.v[e][i + 3] = w.w;
    }
  }
}

// tok: lane j < 16 holds key j's cache row (-1: none); mask: its head bits
// (masked steps only).  Lanes of row r take keys 4r + e's rows and bits
// from lanes 4r + e.
template <int D>
__device__ __forceinline__ void kv_issue(KvStep<D>& st, const uint16_t* __restrict__ kb,
                                         const uint16_t* __restrict__ vb, int64_t k_st,
                                         int64_t v_st, int tok, int lane, int mask = 0) {
  const int r = lane >> 4, c = lane & 15;
#pragma unroll
  for (int e = 0; e < 4; ++e) st.mk[e] = __shfl(mask, 4 * r + e, 64);
  k_issue<D>(st, kb, k_st, tok, r);
#pragma unroll
  for (int e = 0; e < 4; ++e) v_issue<D>(st, vb, v_st, e, __shfl(tok, 4 * r + e, 64), c);
}

// The same with keys 4r + e's cache rows tv[e] and head bits mk[e] given by
// the caller (read where the lane's own key is read, instead of broadcast
// from lanes < 16 after that read returns).
template <int D>
__device__ __forceinline__ void kv_issue_rows(KvStep<D>& st, const uint16_t* __restrict__ kb,
                                              const uint16_t* __restrict__ vb, int64_t k_st,
                                              int64_t v_st, int tok, const int (&tv)[4],
                                              const int (&mk)[4], int lane) {
  const int r = lane >> 4, c = lane & 15;
#pragma unroll
  for (int e = 0; e < 4; ++e) st.mk[e] = mk[e];
  k_issue<D>(st, kb, k_st, tok, r);
#pragma unroll
  for (int e = 0; e < 4; ++e) v_issue<D>(st, vb, v_st, e, tv[e], c);
}

template <int DT, int HPR, int D>
struct WaveState {
  i16x4 qf[D / 16];     // Q^T fragments (head = lane % 16; zero past HPR)
  f32x4 acc[D / 16];    // o, heads 4r + e, dims c * D/16 + ch
  float m, l;           // running max / sum of head lane % 16 (equal in its 4 lanes)
};

// One step: scores by MFMA, online-softmax update, p.V by MFMA.  MASK: key
// 4r + e counts for head c only where bit c of its mask is set (each head
// attends over its own subset of the step's keys).
template <int DT, int HPR, int D, bool MASK = false>
__device__ __forceinline__ void attn_step(WaveState<DT, HPR, D>& ws, const KvStep<D>& st,
                                          float scale_log2, int lane) {
  const int r = lane >> 4, c = lane & 15;
  f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    const uint4 w = st.k[ks / 2];
    const uint2 kk = (ks & 1) ? make_uint2(w.z, w.w) : make_uint2(w.x, w.y);
    sacc = mfma16<DT>(__builtin_bit_cast(i16x4, kk), ws.qf[ks], sacc);
  }
  float sc[4];
  float mx = -INFINITY;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const bool kept = c < HPR && st.tv[e] >= 0 && (!MASK || ((st.mk[e] >> c) & 1));
    sc[e] = kept ? sacc[e] * scale_log2 : -INFINITY;
    mx = fmaxf(mx, sc[e]);
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float m_new = fmaxf(ws.m, mx);
  float pe[4], alpha = 1.f, ps = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    pe[e] = m_new == -INFINITY ? 0.f : exp2f(sc[e] - m_new);  // 0 for sc = -inf
    ps += pe[e];
  }
  if (m_new != -INFINITY) alpha = exp2f(ws.m - m_new);  // 0 for the first finite max
  ps += __shfl_xor(ps, 16, 64);
  ps += __shfl_xor(ps, 32, 64);
  ws.l = ws.l * alpha + ps;
  ws.m = m_new;
  // Rescale o: lane l holds heads 4r + e; head h's alpha lives in lanes h, h+16, ...
  float al[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int a0 = __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), e);
    float a = __builtin_bit_cast(float, a0);
    if (HPR > 4) {
      const float a1 =
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), 4 + e));
      a = r == 1 ? a1 : a;
    }
    al[e] = a;
  }
#pragma unroll
  for (int ch = 0; ch < D / 16; ++ch)
#pragma unroll
    for (int e = 0; e < 4; ++e) ws.acc[ch][e] *= al[e];
  // P operand (row = head c, keys 4r + e), in the data type.
  i16x4 pa;
#pragma unroll
  for (int e = 0; e < 4; ++e) pa[e] = (short)st16<DT>(pe[e]);
#pragma unroll
  for (int ch = 0; ch < D / 16; ++ch) {
    uint32_t vx[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t wv = st.v[e][ch / 2];
      vx[e] = st.tv[e] >= 0 ? ((ch & 1) ? (wv >> 16) : (wv & 0xffffu)) : 0u;
    }
    const uint2 vb2 = make_uint2(vx[0] | (vx[1] << 16), vx[2] | (vx[3] << 16));
    ws.acc[ch] = mfma16<DT>(pa, __builtin_bit_cast(i16x4, vb2), ws.acc[ch]);
  }
}

}  // namespace
}  // namespace lap

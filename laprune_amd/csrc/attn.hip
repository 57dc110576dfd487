// attn.hip — A5: single-query decode attention over a keep list, with the
// K/V gather fused in, and the dense flash-decode comparator.
//
// For batch b and query head h the keep list is
//   L = indices[b, row(h), 0..n_idx) ++ [0, sink) ++ [tail_start, +tail_count)
// (the keep set of laprune/llm/modifiers/aq_evaluation.py:210-237: top-k,
// sink, local window, concatenated), and
//   o[b,h] = sum_j softmax_j(scale * q.K[t_j]) V[t_j]
// as F.scaled_dot_product_attention computes at aq_evaluation.py:251, but
// reading K/V rows straight from the strided cache instead of materialising
// the gathered [B,Hq,N,D] tensors.  Dense decode is the same kernel with
// L = [0, T).
//
// Work shape: workgroup = (b, selection row, split) with 256 threads; a row
// carries HPR query heads (HPR = G when one list serves a KV group, 1 for
// per-head lists) so K/V rows are read once per group.  Keys are processed in
// tiles of 64: phase 1 puts four lanes on each key (a quarter of D each) and
// reduces q.k across them; the online-softmax update runs one wave per head;
// phase 2 gives each wave 16 keys and each lane D/64 output dims.  V loads
// of a tile are issued before phase 1 so they overlap the q.k work.  Splits
// write (m, l, o) partials that a combine kernel merges.
#include "common.h"

namespace lap {
namespace {

constexpr int kTile = 64;
constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;

template <int DT>
__device__ __forceinline__ float ld16(const uint16_t v) {
  return DT == LAP_DTYPE_F16 ? h2f(v) : bf2f(v);
}
template <int DT>
__device__ __forceinline__ uint16_t st16(float f) {
  return DT == LAP_DTYPE_F16 ? f2h(f) : f2bf(f);
}

struct AttnArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
  int B, Hq, Hkv, T;
  const void* idx;
  int H_idx, n_idx, sink, tail_start, tail_count;
  float scale_log2;  // softmax scale * log2(e)
  int per_split, nsplit;
  uint16_t* out;     // [B][Hq][D]
  float* part;       // [B][Hq][nsplit][D + 2] (m, l, o...)
};

template <typename IT>
__device__ __forceinline__ int64_t keep_token(const AttnArgs& a, const IT* idx_row, int j) {
  if (j < a.n_idx) return (int64_t)idx_row[j];
  j -= a.n_idx;
  if (j < a.sink) return j;
  return (int64_t)a.tail_start + (j - a.sink);
}

template <int DT, typename IT, int HPR, int D>
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(AttnArgs a) {
  constexpr int DQ = D / 4;     // dims per phase-1 lane
  constexpr int DPL = D / 64;   // dims per phase-2 lane
  static_assert(D % 64 == 0 && DQ % 8 == 0, "D must be a multiple of 64");
  __shared__ __attribute__((aligned(16))) float s_q[HPR][D];
  __shared__ int64_t s_tok[kTile];
  __shared__ __attribute__((aligned(16))) float s_p[kTile][HPR];
  __shared__ float s_alpha[HPR], s_m[HPR], s_l[HPR];
  __shared__ __attribute__((aligned(16))) float s_o[4][HPR][D];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int s = blockIdx.x % a.nsplit;
  const int br = blockIdx.x / a.nsplit;
  const int b = br / a.H_idx, ri = br - b * a.H_idx;
  const int G = a.Hq / a.Hkv;
  const int h0 = (a.H_idx == a.Hq) ? ri : ri * G;  // first query head of the row
  const int hkv = h0 / G;
  const int L = a.n_idx + a.sink + a.tail_count;
  const int lo = s * a.per_split;
  const int hi = min(L, lo + a.per_split);
  const IT* idx_row =
      a.idx ? static_cast<const IT*>(a.idx) + ((int64_t)b * a.H_idx + ri) * a.n_idx : nullptr;
  const uint16_t* kb = a.k + (int64_t)b * a.k_sb + (int64_t)hkv * a.k_sh;
  const uint16_t* vb = a.v + (int64_t)b * a.v_sb + (int64_t)hkv * a.v_sh;

  for (int i = tid; i < HPR * D; i += kThreads) {
    const int g = i / D, d = i - g * D;
    const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)(h0 + g) * a.q_sh;
    s_q[g][d] = ld16<DT>(qp[d]) * a.scale_log2;
  }
  if (tid < HPR) {
    s_m[tid] = -INFINITY;
    s_l[tid] = 0.f;
  }
  float o[HPR][DPL];
#pragma unroll
  for (int g = 0; g < HPR; ++g)
#pragma unroll
    for (int e = 0; e < DPL; ++e) o[g][e] = 0.f;

  for (int t0 = lo; t0 < hi; t0 += kTile) {
    if (tid < kTile) {
      const int j = t0 + tid;
      int64_t tok = -1;
      if (j < hi) {
        tok = keep_token<IT>(a, idx_row, j);
        if (tok < 0 || tok >= a.T) tok = -1;
      }
      s_tok[tid] = tok;
    }
    __syncthreads();

    // Issue this wave's phase-2 V loads early.
    uint32_t vraw[16][(DPL + 1) / 2];
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      const int64_t tok = s_tok[wave * 16 + jj];
      const uint16_t* vp = vb + (tok < 0 ? 0 : tok) * a.v_st + lane * DPL;
      if (DPL == 1) {
        vraw[jj][0] = tok < 0 ? 0u : (uint32_t)vp[0];
      } else {
#pragma unroll
        for (int e = 0; e < DPL / 2; ++e)
          vraw[jj][e] = tok < 0 ? 0u : reinterpret_cast<const uint32_t*>(vp)[e];
      }
    }

    // Phase 1: four lanes per key, each over D/4 dims.
    {
      const int j = tid >> 2, qd = tid & 3;
      const int64_t tok = s_tok[j];
      float part[HPR];
#pragma unroll
      for (int g = 0; g < HPR; ++g) part[g] = 0.f;
      if (tok >= 0) {
        const uint4* kp = reinterpret_cast<const uint4*>(kb + tok * a.k_st + qd * DQ);
#pragma unroll
        for (int c = 0; c < DQ / 8; ++c) {
          const uint4 w = kp[c];
          const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float k0 = ld16<DT>((uint16_t)(ww[e] & 0xffffu));
            const float k1 = ld16<DT>((uint16_t)(ww[e] >> 16));
            const int d = qd * DQ + c * 8 + 2 * e;
#pragma unroll
            for (int g = 0; g < HPR; ++g) {
              part[g] = __builtin_fmaf(s_q[g][d], k0, part[g]);
              part[g] = __builtin_fmaf(s_q[g][d + 1], k1, part[g]);
            }
          }
        }
      }
#pragma unroll
      for (int g = 0; g < HPR; ++g) {
        part[g] += __shfl_xor(part[g], 1, 64);
        part[g] += __shfl_xor(part[g], 2, 64);
      }
      if (qd == 0) {
#pragma unroll
        for (int g = 0; g < HPR; ++g) s_p[j][g] = tok >= 0 ? part[g] : -INFINITY;
      }
    }
    __syncthreads();

    // Online softmax update: one wave per head (lane = key).
    for (int g = wave; g < HPR; g += 4) {
      const float x = s_p[lane][g];
      float tm = x;
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) tm = fmaxf(tm, __shfl_xor(tm, d, 64));
      const float m_old = s_m[g];
      const float m_new = fmaxf(m_old, tm);
      float p = 0.f, alpha = 1.f;
      if (m_new != -INFINITY) {
        p = (x == -INFINITY) ? 0.f : exp2f(x - m_new);
        alpha = (m_old == -INFINITY) ? 0.f : exp2f(m_old - m_new);
      }
      float ps = p;
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) ps += __shfl_xor(ps, d, 64);
      s_p[lane][g] = p;
      if (lane == 0) {
        s_alpha[g] = alpha;
        s_m[g] = m_new;
        s_l[g] = s_l[g] * alpha + ps;
      }
    }
    __syncthreads();

    // Phase 2: o = o * alpha + sum_j p_j V_j over this wave's 16 keys.
#pragma unroll
    for (int g = 0; g < HPR; ++g) {
      const float al = s_alpha[g];
#pragma unroll
      for (int e = 0; e < DPL; ++e) o[g][e] *= al;
    }
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      const int j = wave * 16 + jj;
      float vv[DPL];
      if (DPL == 1) {
        vv[0] = ld16<DT>((uint16_t)vraw[jj][0]);
      } else {
#pragma unroll
        for (int e = 0; e < DPL / 2; ++e) {
          vv[2 * e] = ld16<DT>((uint16_t)(vraw[jj][e] & 0xffffu));
          vv[2 * e + 1] = ld16<DT>((uint16_t)(vraw[jj][e] >> 16));
        }
      }
#pragma unroll
      for (int g = 0; g < HPR; ++g) {
        const float p = s_p[j][g];
#pragma unroll
        for (int e = 0; e < DPL; ++e) o[g][e] = __builtin_fmaf(p, vv[e], o[g][e]);
      }
    }
    __syncthreads();
  }

  // Cross-wave sum of the partial outputs.
#pragma unroll
  for (int g = 0; g < HPR; ++g)
#pragma unroll
    for (int e = 0; e < DPL; ++e) s_o[wave][g][lane * DPL + e] = o[g][e];
  __syncthreads();
  for (int i = tid; i < HPR * D; i += kThreads) {
    const int g = i / D, d = i - g * D;
    const float sum = s_o[0][g][d] + s_o[1][g][d] + s_o[2][g][d] + s_o[3][g][d];
    const int h = h0 + g;
    const int64_t bh = (int64_t)b * a.Hq + h;
    if (a.nsplit == 1) {
      const float l = s_l[g];
      a.out[bh * D + d] = st16<DT>(l > 0.f ? sum / l : 0.f);
    } else {
      float* pp = a.part + (bh * a.nsplit + s) * (D + 2);
      if (d == 0) {
        pp[0] = s_m[g];
        pp[1] = s_l[g];
      }
      pp[2 + d] = sum;
    }
  }
}

// Merge split partials: out = sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
// One workgroup per (b, h).  Split weights are formed once in LDS; each
// output dim is then summed by 256/D threads over interleaved splits with
// independent loads, and the partial sums are folded through LDS.
template <int DT>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ part,
                                                           int nsplit, int D,
                                                           uint16_t* __restrict__ out) {
  __shared__ float s_w[1024];
  __shared__ float s_red[8];
  __shared__ float s_acc[256];
  const int bh = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* pp = part + (int64_t)bh * nsplit * (D + 2);
  // block max of m_s
  float mx = -INFINITY;
  for (int s = tid; s < nsplit; s += 256) mx = fmaxf(mx, pp[(int64_t)s * (D + 2)]);
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) mx = fmaxf(mx, __shfl_xor(mx, d, 64));
  if (lane == 0) s_red[wave] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  float lsum = 0.f;
  for (int s = tid; s < nsplit; s += 256) {
    const float ms = pp[(int64_t)s * (D + 2)];
    const float w = (ms == -INFINITY || M == -INFINITY) ? 0.f : exp2f(ms - M);
    s_w[s] = w;
    lsum += pp[(int64_t)s * (D + 2) + 1] * w;
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) lsum += __shfl_xor(lsum, d, 64);
  __syncthreads();
  if (lane == 0) s_red[4 + wave] = lsum;
  __syncthreads();
  const float l = s_red[4] + s_red[5] + s_red[6] + s_red[7];
  const int P = 256 / D;  // threads per output dim
  const int d = tid % D, part_id = tid / D;
  float acc = 0.f;
  if (part_id < P) {
#pragma unroll 8
    for (int s = part_id; s < nsplit; s += P)
      acc = __builtin_fmaf(pp[(int64_t)s * (D + 2) + 2 + d], s_w[s], acc);
  }
  s_acc[tid] = acc;
  __syncthreads();
  if (tid < D) {
    float sum = 0.f;
    for (int p2 = 0; p2 < P; ++p2) sum += s_acc[p2 * D + tid];
    out[(int64_t)bh * D + tid] = st16<DT>(l > 0.f ? sum / l : 0.f);
  }
}

int choose_nsplit(int rows, int L) {
  DevInfo di;
  if (device_info(&di) != LAP_OK) return -1;
  const int max_split = (L + kTile - 1) / kTile;
  int ns = (di.cu_count * 2 + rows - 1) / rows;
  if (ns > max_split) ns = max_split;
  if (ns > 1024) ns = 1024;
  return ns < 1 ? 1 : ns;
}

template <int DT, typename IT, int HPR>
hipError_t launch_attn_hpr(const AttnArgs& a, int D, hipStream_t st) {
  dim3 grid((unsigned)(a.B * a.H_idx * a.nsplit));
  if (D == 64) hipLaunchKernelGGL((attn_decode_kernel<DT, IT, HPR, 64>), grid, dim3(kThreads), 0, st, a);
  else if (D == 128) hipLaunchKernelGGL((attn_decode_kernel<DT, IT, HPR, 128>), grid, dim3(kThreads), 0, st, a);
  else hipLaunchKernelGGL((attn_decode_kernel<DT, IT, HPR, 256>), grid, dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

template <int DT, typename IT>
hipError_t launch_attn_dt(const AttnArgs& a, int hpr, int D, hipStream_t st) {
  switch (hpr) {
    case 1: return launch_attn_hpr<DT, IT, 1>(a, D, st);
    case 2: return launch_attn_hpr<DT, IT, 2>(a, D, st);
    case 4: return launch_attn_hpr<DT, IT, 4>(a, D, st);
    default: return launch_attn_hpr<DT, IT, 8>(a, D, st);
  }
}

int run_attn(AttnArgs a, int dtype, int idx_dtype, int D, void* workspace, size_t ws_bytes,
             hipStream_t st) {
  const int L = a.n_idx + a.sink + a.tail_count;
  const int G = a.Hq / a.Hkv;
  const int hpr = (a.H_idx == a.Hq) ? 1 : G;
  a.nsplit = choose_nsplit(a.B * a.H_idx, L > 0 ? L : 1);
  LAP_CHECK_CODE(a.nsplit > 0, LAP_ERR_HIP, "attention: device query failed");
  a.per_split = (L + a.nsplit - 1) / a.nsplit;
  a.per_split = (a.per_split + kTile - 1) / kTile * kTile;
  if (a.per_split < kTile) a.per_split = kTile;
  a.nsplit = L > 0 ? (L + a.per_split - 1) / a.per_split : 1;
  // Workspace: split partials [B][Hq][nsplit][D + 2], merged by a combine
  // kernel.  (An in-kernel merge by the last-arriving workgroup needs a
  // device-scope release per workgroup, which on the multi-XCD part writes
  // back the XCD's L2 and costs far more than the second launch.)
  if (a.nsplit > 1) {
    const size_t need = (size_t)a.B * a.Hq * a.nsplit * (D + 2) * sizeof(float);
    LAP_CHECK_CODE(workspace && ws_bytes >= need, LAP_ERR_WORKSPACE,
                   "attention decode: workspace of %zu bytes needed", need);
    a.part = static_cast<float*>(workspace);
  }
  hipError_t e;
  const bool i64 = idx_dtype == LAP_DTYPE_I64;
  if (dtype == LAP_DTYPE_F16)
    e = i64 ? launch_attn_dt<LAP_DTYPE_F16, int64_t>(a, hpr, D, st)
            : launch_attn_dt<LAP_DTYPE_F16, int32_t>(a, hpr, D, st);
  else
    e = i64 ? launch_attn_dt<LAP_DTYPE_BF16, int64_t>(a, hpr, D, st)
            : launch_attn_dt<LAP_DTYPE_BF16, int32_t>(a, hpr, D, st);
  LAP_HIP(e, "attn_decode_kernel launch");
  if (a.nsplit > 1) {
    if (dtype == LAP_DTYPE_F16)
      hipLaunchKernelGGL(attn_combine_kernel<LAP_DTYPE_F16>, dim3(a.B * a.Hq), dim3(256), 0, st,
                         a.part, a.nsplit, D, a.out);
    else
      hipLaunchKernelGGL(attn_combine_kernel<LAP_DTYPE_BF16>, dim3(a.B * a.Hq), dim3(256), 0, st,
                         a.part, a.nsplit, D, a.out);
    LAP_LAUNCH_CHECK("attn_combine_kernel");
  }
  return LAP_OK;
}

int check_common(const void* q, const void* keys, const void* vals, void* out, int dtype, int B,
                 int Hq, int Hkv, int T, int D, int64_t q_sh, int64_t k_st, int64_t v_st) {
  LAP_CHECK(q && keys && vals && out, "attention decode: null pointer");
  LAP_CHECK(dtype == LAP_DTYPE_F16 || dtype == LAP_DTYPE_BF16,
            "attention decode supports fp16/bf16");
  LAP_CHECK(B > 0 && Hq > 0 && Hkv > 0 && T > 0, "attention decode: bad sizes (T must be >= 1)");
  LAP_CHECK(Hq % Hkv == 0, "invalid GQA head counts: Hq=%d, Hkv=%d", Hq, Hkv);
  const int G = Hq / Hkv;
  LAP_CHECK_CODE(G == 1 || G == 2 || G == 4 || G == 8, LAP_ERR_UNSUPPORTED,
                 "attention decode: group size %d unsupported", G);
  LAP_CHECK_CODE(D == 64 || D == 128 || D == 256, LAP_ERR_UNSUPPORTED,
                 "attention decode: head dim %d unsupported (64/128/256)", D);
  LAP_CHECK(q_sh >= D && k_st >= D && v_st >= D, "attention decode: strides smaller than D");
  LAP_CHECK(k_st % 8 == 0 && v_st % 8 == 0 && (reinterpret_cast<uintptr_t>(keys) & 15) == 0 &&
                (reinterpret_cast<uintptr_t>(vals) & 15) == 0,
            "attention decode: K/V rows must be 16-byte aligned");
  return LAP_OK;
}

}  // namespace
}  // namespace lap

using namespace lap;

extern "C" int lap_attn_decode_workspace_size(int B, int Hq, int D, int max_keys, size_t* bytes) {
  clear_error();
  LAP_CHECK(bytes, "lap_attn_decode_workspace_size: null output");
  LAP_CHECK(B >= 0 && Hq >= 0 && D > 0 && max_keys >= 0, "bad sizes");
  int ns = (max_keys + kTile - 1) / kTile;
  if (ns > 1024) ns = 1024;
  if (ns < 1) ns = 1;
  *bytes = (size_t)B * Hq * ns * (D + 2) * sizeof(float);  // split partials
  return LAP_OK;
}

extern "C" int lap_sparse_attn_decode(const void* q, int64_t q_sb, int64_t q_sh, const void* keys,
                                      const void* vals, int dtype, int B, int Hq, int Hkv, int T,
                                      int D, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                      int64_t v_sb, int64_t v_sh, int64_t v_st,
                                      const void* indices, int idx_dtype, int H_idx, int n_idx,
                                      int sink_count, int tail_start, int tail_count,
                                      float scale, void* out, void* workspace,
                                      size_t workspace_bytes, lap_stream_t stream) {
  clear_error();
  int s = check_common(q, keys, vals, out, dtype, B, Hq, Hkv, T, D, q_sh, k_st, v_st);
  if (s != LAP_OK) return s;
  LAP_CHECK(H_idx == Hq || H_idx == Hkv, "sparse decode: H_idx must be Hq or Hkv");
  LAP_CHECK(n_idx >= 0 && sink_count >= 0 && tail_count >= 0, "sparse decode: negative count");
  LAP_CHECK(n_idx == 0 || indices, "sparse decode: indices required");
  LAP_CHECK(idx_dtype == LAP_DTYPE_I32 || idx_dtype == LAP_DTYPE_I64,
            "sparse decode: idx must be int64 or int32");
  if (tail_count > 0) LAP_CHECK(tail_start >= 0, "sparse decode: tail_start < 0");
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.k = static_cast<const uint16_t*>(keys);
  a.v = static_cast<const uint16_t*>(vals);
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.T = T;
  a.idx = indices;
  a.H_idx = H_idx; a.n_idx = n_idx; a.sink = sink_count;
  a.tail_start = tail_start; a.tail_count = tail_count;
  a.scale_log2 = scale * kLog2e;
  a.out = static_cast<uint16_t*>(out);
  return run_attn(a, dtype, idx_dtype, D, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int lap_dense_attn_decode(const void* q, int64_t q_sb, int64_t q_sh, const void* keys,
                                     const void* vals, int dtype, int B, int Hq, int Hkv, int T,
                                     int D, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                     int64_t v_sb, int64_t v_sh, int64_t v_st, float scale,
                                     void* out, void* workspace, size_t workspace_bytes,
                                     lap_stream_t stream) {
  clear_error();
  int s = check_common(q, keys, vals, out, dtype, B, Hq, Hkv, T, D, q_sh, k_st, v_st);
  if (s != LAP_OK) return s;
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.k = static_cast<const uint16_t*>(keys);
  a.v = static_cast<const uint16_t*>(vals);
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.T = T;
  a.idx = nullptr;
  a.H_idx = Hkv; a.n_idx = 0; a.sink = 0;
  a.tail_start = 0; a.tail_count = T;
  a.scale_log2 = scale * kLog2e;
  a.out = static_cast<uint16_t*>(out);
  return run_attn(a, dtype, LAP_DTYPE_I32, D, workspace, workspace_bytes, as_stream(stream));
}

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
// carries nh query heads (G when one list serves a KV group, 1 for per-head
// lists; the kernel is built for HPR = 1, 2, 4 or 8 heads and leaves the
// lanes past nh out) so K/V rows are read once per group.  Each wave runs its
// own online softmax over steps of 16 keys of the split (waves take steps
// round-robin); q.k and p.V of a step are 16x16x16 MFMAs (layouts below), so
// the VALU only does the softmax.  Memory is software-pipelined per wave: a
// step's keep-list positions are read two steps ahead and its K/V rows one
// step ahead, and nothing in the loop waits on the whole workgroup.  The
// waves' states merge through LDS at the end; splits are merged by a combine
// kernel.
#include "common.h"
#include "attn_core.h"

#include <cstdlib>
#include <cstring>

namespace lap {
namespace {

constexpr int kThreads = 256;

struct AttnArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
  int B, Hq, Hkv, T;
  const void* idx;
  int H_idx, n_idx, sink, tail_start, tail_count;
  int nh;            // query heads per index row (1, or G = Hq / Hkv), <= HPR
  float scale_log2;  // softmax scale * log2(e)
  int per_split, nsplit;
  uint16_t* out;     // [B][Hq][D]
  float* part;       // [B][Hq][nsplit][D + 2] (m, l, o...)
  const int32_t* plans;  // lap_row_plan[B] (ragged batches) or null
};

// The keep set of one sequence: [0, sink) ++ [tail_start, +tail_count) after
// the index list, rows bounded by T.  The call's scalars, or the sequence's
// plan with sink and tail clamped to the call's (which size the grid).
struct RowKeep {
  int sink, tail_start, tail_count, T;
};
__device__ __forceinline__ RowKeep row_keep(const AttnArgs& a, int b) {
  if (!a.plans) return RowKeep{a.sink, a.tail_start, a.tail_count, a.T};
  const int32_t* p = a.plans + (int64_t)b * kPlanInts;
  return RowKeep{min(max(p[5], 0), a.sink), p[6], min(max(p[7], 0), a.tail_count),
                 min(p[1], a.T)};
}

// Keep-list position j (0 <= j < n_idx + sink + tail_count) -> cache row, -1
// when outside [0, T).  Branch-free: with HAS_IDX the index load is always
// issued (clamped into the list), so every call issues the same number of
// loads and the compiler's wait counts stay exact through the software
// pipeline.
template <bool HAS_IDX, typename IT>
__device__ __forceinline__ int keep_token(const AttnArgs& a, const RowKeep& rk,
                                          const IT* idx_row, int j) {
  const int jt = j - a.n_idx;
  int64_t t = jt < rk.sink ? jt : (int64_t)rk.tail_start + (jt - rk.sink);
  if (HAS_IDX) {
    const int ji = j < a.n_idx ? j : a.n_idx - 1;
    const int64_t ti = (int64_t)idx_row[ji];
    t = j < a.n_idx ? ti : t;
  }
  return (t < 0 || t >= rk.T) ? -1 : (int)t;
}


template <int DT, typename IT, int HPR, int D, bool HAS_IDX>
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(AttnArgs a) {
  static_assert(D % 64 == 0 && HPR <= 8, "D must be a multiple of 64, HPR <= 8");
  __shared__ float s_m[4][HPR], s_l[4][HPR];
  __shared__ __attribute__((aligned(16))) float s_o[4][HPR][D];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int s = blockIdx.x % a.nsplit;
  const int br = blockIdx.x / a.nsplit;
  const int b = br / a.H_idx, ri = br - b * a.H_idx;
  const int G = a.Hq / a.Hkv;
  const int nh = a.nh;
  const int h0 = (a.H_idx == a.Hq) ? ri : ri * G;  // first query head of the row
  const int hkv = h0 / G;
  const RowKeep rk = row_keep(a, b);
  const int L = a.n_idx + rk.sink + rk.tail_count;
  const int lo = s * a.per_split;
  const int hi = min(L, lo + a.per_split);
  const IT* idx_row =
      a.idx ? static_cast<const IT*>(a.idx) + ((int64_t)b * a.H_idx + ri) * a.n_idx : nullptr;
  const uint16_t* kb = a.k + (int64_t)b * a.k_sb + (int64_t)hkv * a.k_sh;
  const uint16_t* vb = a.v + (int64_t)b * a.v_sb + (int64_t)hkv * a.v_sh;

  WaveState<DT, HPR, D> ws;
  {
    const int r = lane >> 4, c = lane & 15;
    const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)(h0 + (c < nh ? c : 0)) * a.q_sh;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const uint16_t* q4 = qp + r * (D / 4) + 4 * ks;  // q may be only 2-byte aligned
      i16x4 f;
#pragma unroll
      for (int e = 0; e < 4; ++e) f[e] = c < nh ? (short)q4[e] : (short)0;
      ws.qf[ks] = f;
      ws.acc[ks] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    ws.m = -INFINITY;
    ws.l = 0.f;
  }
  // This wave's steps: keys [lo + (w + 4i) * 16, +16) for i = 0, 1, ...
  const int nsteps = (hi - lo + kKeys - 1) / kKeys;
  const int mine = nsteps > wave ? (nsteps - wave + 3) / 4 : 0;
  const int jmax = hi > lo ? hi - 1 : 0;
  auto pos_tok = [&](int i) -> int {
    const int jpos = lo + (wave + 4 * i) * kKeys + (lane & 15);
    const int tk = keep_token<HAS_IDX, IT>(a, rk, idx_row, jpos < jmax ? jpos : jmax);
    return (i < mine && jpos < hi) ? tk : -1;
  };
  // Pipeline: keep-list rows two steps ahead, K/V one step ahead, ping-pong
  // buffers.  The steady-state loop issues unconditionally (exact wait
  // counts); the last steps run in the tail loop.
  KvStep<D> bufA, bufB;
  int tokA = pos_tok(0), tokB = pos_tok(1);
  kv_issue<D>(bufA, kb, vb, a.k_st, a.v_st, tokA, lane);
  int i = 0;
  for (; i + 3 < mine; i += 2) {
    const int tokC = pos_tok(i + 2);
    kv_issue<D>(bufB, kb, vb, a.k_st, a.v_st, tokB, lane);
    attn_step<DT, HPR, D>(ws, bufA, a.scale_log2, lane);
    const int tokD = pos_tok(i + 3);
    kv_issue<D>(bufA, kb, vb, a.k_st, a.v_st, tokC, lane);
    attn_step<DT, HPR, D>(ws, bufB, a.scale_log2, lane);
    tokA = tokC;
    tokB = tokD;
  }
  // Tail: steps i .. mine-1 (at most three); bufA holds step i when i < mine.
  if (i < mine) {
    if (i + 1 < mine) kv_issue<D>(bufB, kb, vb, a.k_st, a.v_st, tokB, lane);
    attn_step<DT, HPR, D>(ws, bufA, a.scale_log2, lane);
    if (i + 1 < mine) {
      const int tokC = pos_tok(i + 2);
      if (i + 2 < mine) kv_issue<D>(bufA, kb, vb, a.k_st, a.v_st, tokC, lane);
      attn_step<DT, HPR, D>(ws, bufB, a.scale_log2, lane);
      if (i + 2 < mine) attn_step<DT, HPR, D>(ws, bufA, a.scale_log2, lane);
    }
  }

  // Merge the four waves' states.
  {
    const int r = lane >> 4, c = lane & 15;
    if (lane < nh) {
      s_m[wave][lane] = ws.m;
      s_l[wave][lane] = ws.l;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int h = 4 * r + e;
      if (h < nh)
#pragma unroll
        for (int ch = 0; ch < D / 16; ++ch) s_o[wave][h][c * (D / 16) + ch] = ws.acc[ch][e];
    }
  }
  __syncthreads();
  for (int i = tid; i < nh * D; i += kThreads) {
    const int g = i / D, d = i - g * D;
    const float M = fmaxf(fmaxf(s_m[0][g], s_m[1][g]), fmaxf(s_m[2][g], s_m[3][g]));
    float l = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float wt = (M == -INFINITY || s_m[w][g] == -INFINITY) ? 0.f : exp2f(s_m[w][g] - M);
      l += s_l[w][g] * wt;
      o += s_o[w][g][d] * wt;
    }
    const int64_t bh = (int64_t)b * a.Hq + h0 + g;
    if (a.nsplit == 1) {
      a.out[bh * D + d] = st16<DT>(l > 0.f ? o / l : 0.f);
    } else {
      float* pp = a.part + (bh * a.nsplit + s) * (D + 2);
      if (d == 0) {
        pp[0] = M;
        pp[1] = l;
      }
      pp[2 + d] = o;
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
  // Workgroups per CU the splits aim at: one (A/B at C2 and C5 against two
  // and four: faster for the dense, group, per-head and ragged steps);
  // LAPRUNE_ATTN_WPC overrides.
  static const int wpc = [] {
    const char* e = getenv("LAPRUNE_ATTN_WPC");
    const int v = e ? atoi(e) : 0;
    return v >= 1 && v <= 16 ? v : 1;
  }();
  const int max_split = (L + kTile - 1) / kTile;
  int ns = (di.cu_count * wpc + rows - 1) / rows;
  if (ns > max_split) ns = max_split;
  if (ns > 1024) ns = 1024;
  return ns < 1 ? 1 : ns;
}

template <int DT, typename IT, int HPR>
hipError_t launch_attn_hpr(const AttnArgs& a, int D, hipStream_t st) {
  dim3 grid((unsigned)(a.B * a.H_idx * a.nsplit));
  const bool has_idx = a.idx && a.n_idx > 0;
#define LAP_ATTN(D_)                                                                        \
  if (has_idx)                                                                              \
    hipLaunchKernelGGL((attn_decode_kernel<DT, IT, HPR, D_, true>), grid, dim3(kThreads), 0, \
                       st, a);                                                              \
  else                                                                                      \
    hipLaunchKernelGGL((attn_decode_kernel<DT, IT, HPR, D_, false>), grid, dim3(kThreads), 0, \
                       st, a)
  if (D == 64) { LAP_ATTN(64); }
  else if (D == 128) { LAP_ATTN(128); }
  else { LAP_ATTN(256); }
#undef LAP_ATTN
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
  a.nh = (a.H_idx == a.Hq) ? 1 : G;
  // the kernel's head capacity per row: the next of 1, 2, 4, 8 (lanes past
  // nh compute on zero queries and write nothing)
  const int hpr = a.nh <= 1 ? 1 : a.nh <= 2 ? 2 : a.nh <= 4 ? 4 : 8;
  a.nsplit = choose_nsplit(a.B * a.H_idx, L > 0 ? L : 1);
  LAP_CHECK_CODE(a.nsplit > 0, LAP_ERR_HIP, "attention: device query failed");
  a.per_split = (L + a.nsplit - 1) / a.nsplit;
  a.per_split = (a.per_split + kTile - 1) / kTile * kTile;
  if (a.per_split < kTile) a.per_split = kTile;
  a.nsplit = L > 0 ? (L + a.per_split - 1) / a.per_split : 1;
  // Workspace: the split partials [B][Hq][nsplit][D + 2] (m, l, o...).
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
                 int Hq, int Hkv, int T, int D, int64_t q_sh, int64_t k_sb, int64_t k_sh,
                 int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st) {
  LAP_CHECK(q && keys && vals && out, "attention decode: null pointer");
  LAP_CHECK(dtype == LAP_DTYPE_F16 || dtype == LAP_DTYPE_BF16,
            "attention decode supports fp16/bf16");
  LAP_CHECK(B > 0 && Hq > 0 && Hkv > 0 && T > 0, "attention decode: bad sizes (T must be >= 1)");
  LAP_CHECK(Hq % Hkv == 0, "invalid GQA head counts: Hq=%d, Hkv=%d", Hq, Hkv);
  const int G = Hq / Hkv;
  LAP_CHECK_CODE(G >= 1 && G <= 8, LAP_ERR_UNSUPPORTED,
                 "attention decode: group size %d unsupported (1 to 8)", G);
  LAP_CHECK_CODE(D == 64 || D == 128 || D == 256, LAP_ERR_UNSUPPORTED,
                 "attention decode: head dim %d unsupported (64/128/256)", D);
  LAP_CHECK(q_sh >= D && k_st >= D && v_st >= D, "attention decode: strides smaller than D");
  // every K/V row is read as 16-byte vectors: base and all three strides
  LAP_CHECK(k_st % 8 == 0 && v_st % 8 == 0 && k_sh % 8 == 0 && v_sh % 8 == 0 &&
                k_sb % 8 == 0 && v_sb % 8 == 0 && (reinterpret_cast<uintptr_t>(keys) & 15) == 0 &&
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
  // the split partials
  *bytes = (size_t)B * Hq * ns * (D + 2) * sizeof(float);
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
  int s = check_common(q, keys, vals, out, dtype, B, Hq, Hkv, T, D, q_sh, k_sb, k_sh, k_st, v_sb,
                       v_sh, v_st);
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

extern "C" int lap_sparse_attn_decode_ragged(
    const void* q, int64_t q_sb, int64_t q_sh, const void* keys, const void* vals, int dtype,
    int B, int Hq, int Hkv, int T, int D, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t v_sb,
    int64_t v_sh, int64_t v_st, const void* indices, int idx_dtype, int H_idx, int k_cols,
    const lap_row_plan* plans, int max_sink, int max_tail, float scale, void* out,
    void* workspace, size_t workspace_bytes, lap_stream_t stream) {
  clear_error();
  int s = check_common(q, keys, vals, out, dtype, B, Hq, Hkv, T, D, q_sh, k_sb, k_sh, k_st, v_sb,
                       v_sh, v_st);
  if (s != LAP_OK) return s;
  LAP_CHECK(plans, "ragged decode: null plans");
  LAP_CHECK(H_idx == Hq || H_idx == Hkv, "ragged decode: H_idx must be Hq or Hkv");
  LAP_CHECK(k_cols >= 0 && max_sink >= 0 && max_tail >= 0, "ragged decode: negative count");
  LAP_CHECK(k_cols == 0 || indices, "ragged decode: indices required");
  LAP_CHECK(idx_dtype == LAP_DTYPE_I32 || idx_dtype == LAP_DTYPE_I64,
            "ragged decode: idx must be int64 or int32");
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
  a.H_idx = H_idx; a.n_idx = k_cols;
  // grid bounds; each sequence's own windows come from its plan
  a.sink = max_sink;
  a.tail_start = 0;
  a.tail_count = max_tail;
  a.plans = reinterpret_cast<const int32_t*>(plans);
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
  int s = check_common(q, keys, vals, out, dtype, B, Hq, Hkv, T, D, q_sh, k_sb, k_sh, k_st, v_sb,
                       v_sh, v_st);
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

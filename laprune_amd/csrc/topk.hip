// topk.hip — A3: exact top-k over fp16 scores by two radix levels.
//
// Replaces torch.topk(scores[..., cand_start:cand_end], k, sorted=False)
// (laprune/llm/modifiers/aq_evaluation.py:198-201).  Scores are fp16, so an
// orderable 16-bit key (common.h: f16_key / bf16_key_of_f16) ranks them
// exactly and two 8-bit radix levels find the k-th largest key tau:
//   level 1: histogram of key>>8 over the row (per chunk, summed) -> bin b1
//   level 2: histogram of key&255 among keys with key>>8 == b1    -> bin b2
// Selected = every key > tau, plus the `need` lowest-index keys == tau, so
// the result is deterministic (ties: lowest column wins) and emitted in
// ascending column order by an ordered per-chunk compaction.
//
// Kernels (grid = rows x chunks, 256 threads, chunk = 2048 candidates):
//   topk_prep_kernel   scores -> keys (group max) + level-1 chunk histograms
//                      (the fused scorer in score.hip produces the same)
//   topk_level2_kernel level-1 bin per row, level-2 chunk histograms
//   topk_select_kernel threshold, per-chunk output offsets, compaction
// No atomics touch global memory and nothing needs zero-initialised scratch.
#include "common.h"

namespace lap {

int launch_score_g4(const uint16_t* lut, bool lut_il, const uint8_t* codes, int64_t cs_b,
                    int64_t cs_h, int64_t cs_t, int B, int Hkv, int T, uint16_t* heads,
                    uint16_t* keys, uint32_t* hist, int key_mode, int cand_start, int cand_end,
                    int* nchunk_out, hipStream_t st);
bool score_g4_supported(const uint8_t* codes, int64_t cs_b, int64_t cs_h, int64_t cs_t);
int score_g4_nchunk(int R, int T);

namespace {

constexpr int kChunk = 2048;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// Inclusive suffix sums S(i) = sum_{j>=i} h[j] over 256 LDS bins, then the
// unique bin b with S(b) >= target > S(b+1).  Returns b and S(b+1) to every
// thread.  target must satisfy 1 <= target <= S(0).
__device__ void select_bin(const uint32_t* s_h, uint32_t target, uint32_t* s_wsum,
                           uint32_t* s_res) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  // Scan the reversed bins: x_tid = h[255 - tid]; P(tid) = S(255 - tid).
  uint32_t x = s_h[255 - tid];
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    uint32_t y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) s_wsum[wave] = x;
  __syncthreads();
  uint32_t add = 0;
  for (int w = 0; w < wave; ++w) add += s_wsum[w];
  const uint32_t S_i = x + add;                    // S(255 - tid)
  const uint32_t S_next = S_i - s_h[255 - tid];    // S(256 - tid)
  if (S_i >= target && S_next < target) {
    s_res[0] = 255 - tid;
    s_res[1] = S_next;
  }
  __syncthreads();
}

template <int KEYMODE>
__device__ __forceinline__ uint32_t key_of(uint16_t h) {
  return KEYMODE == LAP_KEY_BF16 ? bf16_key_of_f16(h) : f16_key(h);
}

template <int KEYMODE>
__global__ __launch_bounds__(kThreads) void topk_prep_kernel(
    const uint16_t* __restrict__ scores, int64_t row_stride, int R, int group, int cand_start,
    int n, int C, uint16_t* __restrict__ keys, uint32_t* __restrict__ hist1) {
  __shared__ uint32_t s_h[256];
  const int r = blockIdx.x % R, c = blockIdx.x / R;
  s_h[threadIdx.x] = 0;
  __syncthreads();
  const int e0 = c * kChunk, e1 = min(n, e0 + kChunk);
#pragma unroll 8
  for (int e = e0 + threadIdx.x; e < e1; e += kThreads) {
    uint32_t key = 0;
    for (int g = 0; g < group; ++g) {
      const uint16_t h = scores[(int64_t)(r * group + g) * row_stride + cand_start + e];
      key = max(key, key_of<KEYMODE>(h));
    }
    keys[(int64_t)r * n + e] = (uint16_t)key;
    atomicAdd(&s_h[key >> 8], 1u);
  }
  __syncthreads();
  hist1[((int64_t)r * C + c) * 256 + threadIdx.x] = s_h[threadIdx.x];
}

struct KeySrc {
  const uint16_t* keys;
  int64_t stride;  // row stride of keys
  int off;         // column of candidate 0
};

// Sum of n values p[0], p[stride], ... with 32 independent loads in flight
// (the chunk histograms live in L2; latency, not bandwidth, is the cost).
__device__ __forceinline__ void sum_strided2(const uint32_t* __restrict__ p, int n,
                                             int64_t stride, int split, uint32_t& tot,
                                             uint32_t& pre) {
  tot = 0;
  pre = 0;
  int i = 0;
  for (; i + 32 <= n; i += 32) {
    uint32_t v[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) v[u] = p[(int64_t)(i + u) * stride];
#pragma unroll
    for (int u = 0; u < 32; ++u) {
      tot += v[u];
      pre += (i + u) < split ? v[u] : 0u;
    }
  }
  for (; i < n; ++i) {
    const uint32_t v = p[(int64_t)i * stride];
    tot += v;
    pre += i < split ? v : 0u;
  }
}

// Exclusive prefix sum over the 256 threads of the block; returns the
// thread's prefix and writes the block total to *total.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t x, uint32_t* s_wsum,
                                                         uint32_t* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t inc = x;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t y = __shfl_up(inc, d, 64);
    if (lane >= d) inc += y;
  }
  if (lane == 63) s_wsum[wave] = inc;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const uint32_t v = s_wsum[w];
    before += w < wave ? v : 0u;
    all += v;
  }
  __syncthreads();
  *total = all;
  return before + inc - x;
}

constexpr int kPer = kChunk / kThreads;  // keys per thread, contiguous

__global__ __launch_bounds__(kThreads) void topk_level2_kernel(
    KeySrc ks, int R, int n, int k, const uint32_t* __restrict__ hist1, int C1, int C,
    uint32_t* __restrict__ hist2, uint32_t* __restrict__ gtc, uint32_t* __restrict__ info) {
  __shared__ uint32_t s_h[256], s_h2[256], s_wsum[kWaves], s_res[2], s_gt;
  const int r = blockIdx.x % R, c = blockIdx.x / R;
  const int tid = threadIdx.x;
  // this thread's keys first, so their latency overlaps the histogram sum
  const int e0 = c * kChunk, e1 = min(n, e0 + kChunk);
  const uint16_t* kr = ks.keys + (int64_t)r * ks.stride + ks.off;
  uint32_t kv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = e0 + tid * kPer + i;
    kv[i] = e < e1 ? (uint32_t)kr[e] : 0xffffffffu;
  }
  uint32_t tot, unused;
  sum_strided2(hist1 + (int64_t)r * C1 * 256 + tid, C1, 256, 0, tot, unused);
  s_h[tid] = tot;
  s_h2[tid] = 0;
  if (tid == 0) s_gt = 0;
  __syncthreads();
  select_bin(s_h, (uint32_t)k, s_wsum, s_res);
  const uint32_t b1 = s_res[0];
  if (c == 0 && tid == 0) {
    info[r * 4 + 0] = b1;
    info[r * 4 + 1] = s_res[1];
  }
  uint32_t gt = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    if (kv[i] == 0xffffffffu) continue;
    const uint32_t hi = kv[i] >> 8;
    if (hi == b1) atomicAdd(&s_h2[kv[i] & 255u], 1u);
    gt += hi > b1;
  }
  if (gt) atomicAdd(&s_gt, gt);
  __syncthreads();
  hist2[((int64_t)r * C + c) * 256 + tid] = s_h2[tid];
  if (tid == 0) gtc[(int64_t)r * C + c] = s_gt;
}

template <typename OUT_T>
__global__ __launch_bounds__(kThreads) void topk_select_kernel(
    KeySrc ks, int R, int n, int k, int C, const uint32_t* __restrict__ hist2,
    const uint32_t* __restrict__ gtc, const uint32_t* __restrict__ info, int cand_start,
    OUT_T* __restrict__ out, int64_t out_stride) {
  __shared__ uint32_t s_tot[256], s_pre[256], s_wsum[kWaves], s_res[2], s_red[kWaves];
  const int r = blockIdx.x % R, c = blockIdx.x / R;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int e0 = c * kChunk, e1 = min(n, e0 + kChunk);
  const uint16_t* kr = ks.keys + (int64_t)r * ks.stride + ks.off;
  uint32_t kv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = e0 + tid * kPer + i;
    kv[i] = e < e1 ? (uint32_t)kr[e] : 0u;
  }
  const uint32_t b1 = info[r * 4 + 0], gt1 = info[r * 4 + 1];
  uint32_t tot, pre;
  sum_strided2(hist2 + (int64_t)r * C * 256 + tid, C, 256, c, tot, pre);
  s_tot[tid] = tot;
  s_pre[tid] = pre;
  // Selected-above-threshold count of earlier chunks: gtc prefix.
  uint32_t g = 0;
  for (int cc = tid; cc < c; cc += kThreads) g += gtc[(int64_t)r * C + cc];
  __syncthreads();
  const uint32_t k2 = (uint32_t)k - gt1;
  select_bin(s_tot, k2, s_wsum, s_res);
  const uint32_t b2 = s_res[0];
  const uint32_t need = k2 - s_res[1];  // ties at tau to take, >= 1
  const uint32_t tau = (b1 << 8) | b2;
  const uint32_t ties_before = s_pre[b2];
  // base = gtc prefix + level-2 keys above b2 in earlier chunks + ties taken.
  uint32_t part = g + (tid > (int)b2 ? s_pre[tid] : 0u);
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) part += __shfl_xor(part, d, 64);
  if (lane == 0) s_red[wave] = part;
  __syncthreads();
  uint32_t base = 0;
  for (int w = 0; w < kWaves; ++w) base += s_red[w];
  base += min(need, ties_before);

  // Ordered compaction: each thread owns kPer consecutive candidates.
  uint32_t ntie = 0, ngt = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const bool valid = e0 + tid * kPer + i < e1;
    ntie += (valid && kv[i] == tau) ? 1u : 0u;
    ngt += (valid && kv[i] > tau) ? 1u : 0u;
  }
  uint32_t all_ties;
  const uint32_t tie_rank0 = ties_before + block_exclusive_scan(ntie, s_wsum, &all_ties);
  // ties this thread may take: ranks [tie_rank0, tie_rank0 + ntie) below need
  const uint32_t take = tie_rank0 >= need ? 0u : min(ntie, need - tie_rank0);
  uint32_t all_sel;
  uint32_t pos = base + block_exclusive_scan(ngt + take, s_wsum, &all_sel);
  OUT_T* orow = out + (int64_t)r * out_stride;
  uint32_t taken = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = e0 + tid * kPer + i;
    if (e >= e1) continue;
    bool sel = kv[i] > tau;
    if (kv[i] == tau && taken < take) {
      sel = true;
      ++taken;
    }
    if (sel) orow[pos++] = (OUT_T)(cand_start + e);
  }
}

struct Ws {
  uint16_t* keys;
  uint32_t* hist1;
  uint32_t* hist2;
  uint32_t* gtc;
  uint32_t* info;
  size_t bytes;
};

// Carve the workspace: keys [R][key_cols] u16, hist1 [R][C1][256],
// hist2 [R][C2][256], gtc [R][C2], info [R][4].
Ws carve(void* base, int R, int64_t key_cols, int C1, int C2) {
  Ws w{};
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) {
    char* q = p ? p + off : nullptr;
    off = align_up(off + bytes, 256);
    return q;
  };
  w.keys = reinterpret_cast<uint16_t*>(take((size_t)R * key_cols * 2));
  w.hist1 = reinterpret_cast<uint32_t*>(take((size_t)R * C1 * 256 * 4));
  w.hist2 = reinterpret_cast<uint32_t*>(take((size_t)R * C2 * 256 * 4));
  w.gtc = reinterpret_cast<uint32_t*>(take((size_t)R * C2 * 4));
  w.info = reinterpret_cast<uint32_t*>(take((size_t)R * 4 * 4));
  w.bytes = off;
  return w;
}

int run_levels(const Ws& w, KeySrc ks, int R, int n, int k, int C1, int cand_start,
               void* out, int out_dtype, int64_t out_stride, hipStream_t st) {
  const int C2 = (n + kChunk - 1) / kChunk;
  hipLaunchKernelGGL(topk_level2_kernel, dim3(R * C2), dim3(kThreads), 0, st, ks, R, n, k,
                     w.hist1, C1, C2, w.hist2, w.gtc, w.info);
  LAP_LAUNCH_CHECK("topk_level2_kernel");
  if (out_dtype == LAP_DTYPE_I64)
    hipLaunchKernelGGL(topk_select_kernel<int64_t>, dim3(R * C2), dim3(kThreads), 0, st, ks, R,
                       n, k, C2, w.hist2, w.gtc, w.info, cand_start,
                       static_cast<int64_t*>(out), out_stride);
  else
    hipLaunchKernelGGL(topk_select_kernel<int32_t>, dim3(R * C2), dim3(kThreads), 0, st, ks, R,
                       n, k, C2, w.hist2, w.gtc, w.info, cand_start,
                       static_cast<int32_t*>(out), out_stride);
  LAP_LAUNCH_CHECK("topk_select_kernel");
  return LAP_OK;
}

// Upper bound on the scorer's workgroup chunks per row: a chunk holds at
// least one pass of the smallest launch shape (256 threads x 1 token).
int retrieve_chunk_bound(int T) { return (T + 255) / 256; }

}  // namespace
}  // namespace lap

using namespace lap;

extern "C" int lap_topk_workspace_size(int R, int cand_len, size_t* bytes) {
  clear_error();
  LAP_CHECK(bytes, "lap_topk_workspace_size: null output");
  LAP_CHECK(R >= 0 && cand_len >= 0, "lap_topk_workspace_size: negative size");
  const int C = (cand_len + kChunk - 1) / kChunk;
  *bytes = carve(nullptr, R, cand_len, C, C).bytes;
  return LAP_OK;
}

extern "C" int lap_topk_select(const void* scores, int64_t score_row_stride, int R, int group,
                               int T, int cand_start, int cand_end, int k, int key_mode,
                               void* out_idx, int out_dtype, void* workspace,
                               size_t workspace_bytes, lap_stream_t stream) {
  clear_error();
  LAP_CHECK(scores && out_idx, "lap_topk_select: null pointer");
  LAP_CHECK(R > 0 && group > 0 && T >= 0, "lap_topk_select: bad sizes");
  LAP_CHECK(cand_start >= 0 && cand_end <= T && cand_start <= cand_end,
            "lap_topk_select: candidate window [%d,%d) outside [0,%d)", cand_start, cand_end, T);
  LAP_CHECK(k >= 0, "lap_topk_select: k must be non-negative");
  LAP_CHECK(score_row_stride >= T, "lap_topk_select: row stride < T");
  LAP_CHECK(key_mode == LAP_KEY_F16 || key_mode == LAP_KEY_BF16, "lap_topk_select: bad key mode");
  LAP_CHECK(out_dtype == LAP_DTYPE_I32 || out_dtype == LAP_DTYPE_I64,
            "lap_topk_select: out dtype must be int32/int64");
  const int n = cand_end - cand_start;
  const int ke = std::min(k, n);
  if (ke == 0) return LAP_OK;
  const int C = (n + kChunk - 1) / kChunk;
  Ws w = carve(workspace, R, n, C, C);
  LAP_CHECK_CODE(workspace && workspace_bytes >= w.bytes, LAP_ERR_WORKSPACE,
                 "lap_topk_select: workspace of %zu bytes needed", w.bytes);
  hipStream_t st = as_stream(stream);
  const uint16_t* S = static_cast<const uint16_t*>(scores);
  if (key_mode == LAP_KEY_BF16)
    hipLaunchKernelGGL(topk_prep_kernel<LAP_KEY_BF16>, dim3(R * C), dim3(kThreads), 0, st, S,
                       score_row_stride, R, group, cand_start, n, C, w.keys, w.hist1);
  else
    hipLaunchKernelGGL(topk_prep_kernel<LAP_KEY_F16>, dim3(R * C), dim3(kThreads), 0, st, S,
                       score_row_stride, R, group, cand_start, n, C, w.keys, w.hist1);
  LAP_LAUNCH_CHECK("topk_prep_kernel");
  KeySrc ks{w.keys, n, 0};
  return run_levels(w, ks, R, n, ke, C, cand_start, out_idx, out_dtype, k, st);
}

extern "C" int lap_retrieve_workspace_size(int R, int T, size_t* bytes) {
  clear_error();
  LAP_CHECK(bytes, "lap_retrieve_workspace_size: null output");
  LAP_CHECK(R >= 0 && T >= 0, "lap_retrieve_workspace_size: negative size");
  const int C2 = (T + kChunk - 1) / kChunk;
  *bytes = carve(nullptr, R, T, retrieve_chunk_bound(T), C2).bytes;
  return LAP_OK;
}

static int retrieve_checks(const void* lut_gmkg, const uint8_t* codes, int64_t cs_b,
                           int64_t cs_h, int64_t cs_t, int B, int Hkv, int T, int cand_start,
                           int cand_end, int k, int key_mode) {
  LAP_CHECK(lut_gmkg && codes, "lap_retrieve: null pointer");
  LAP_CHECK(B > 0 && Hkv > 0 && T > 0, "lap_retrieve: bad sizes");
  LAP_CHECK(cand_start >= 0 && cand_end <= T && cand_start <= cand_end,
            "lap_retrieve: candidate window [%d,%d) outside [0,%d)", cand_start, cand_end, T);
  LAP_CHECK(k >= 0, "lap_retrieve: k must be non-negative");
  LAP_CHECK(key_mode == LAP_KEY_F16 || key_mode == LAP_KEY_BF16, "lap_retrieve: bad key mode");
  LAP_CHECK(cs_t >= 32, "lap_retrieve: codes token stride < M=32");
  LAP_CHECK_CODE(score_g4_supported(codes, cs_b, cs_h, cs_t), LAP_ERR_UNSUPPORTED,
                 "lap_retrieve: codes base and strides must be 16-byte aligned");
  return LAP_OK;
}

extern "C" int lap_retrieve_score(const void* lut_gmkg, const uint8_t* codes,
                                  int64_t codes_stride_b, int64_t codes_stride_h,
                                  int64_t codes_stride_t, int B, int Hkv, int T, int cand_start,
                                  int cand_end, int key_mode, void* scores_out,
                                  void* workspace, size_t workspace_bytes,
                                  lap_stream_t stream) {
  clear_error();
  int s = retrieve_checks(lut_gmkg, codes, codes_stride_b, codes_stride_h, codes_stride_t, B,
                          Hkv, T, cand_start, cand_end, 0, key_mode);
  if (s != LAP_OK) return s;
  const int R = B * Hkv;
  const int C2 = (T + kChunk - 1) / kChunk;
  Ws w = carve(workspace, R, T, retrieve_chunk_bound(T), C2);
  LAP_CHECK_CODE(workspace && workspace_bytes >= w.bytes, LAP_ERR_WORKSPACE,
                 "lap_retrieve_score: workspace of %zu bytes needed", w.bytes);
  int C1 = 0;
  s = launch_score_g4(static_cast<const uint16_t*>(lut_gmkg), true, codes, codes_stride_b,
                      codes_stride_h, codes_stride_t, B, Hkv, T,
                      static_cast<uint16_t*>(scores_out), w.keys, w.hist1, key_mode,
                      cand_start, cand_end, &C1, as_stream(stream));
  if (s != LAP_OK) return s;
  LAP_CHECK_CODE(C1 <= retrieve_chunk_bound(T), LAP_ERR_INVALID,
                 "lap_retrieve_score: internal chunk bound exceeded");
  return LAP_OK;
}

extern "C" int lap_retrieve_select(int B, int Hkv, int T, int cand_start, int cand_end, int k,
                                   void* out_idx, int out_dtype, void* workspace,
                                   size_t workspace_bytes, lap_stream_t stream) {
  clear_error();
  LAP_CHECK(out_idx, "lap_retrieve_select: null output");
  LAP_CHECK(B > 0 && Hkv > 0 && T > 0, "lap_retrieve_select: bad sizes");
  LAP_CHECK(cand_start >= 0 && cand_end <= T && cand_start <= cand_end,
            "lap_retrieve_select: candidate window [%d,%d) outside [0,%d)", cand_start, cand_end,
            T);
  LAP_CHECK(k >= 0, "lap_retrieve_select: k must be non-negative");
  LAP_CHECK(out_dtype == LAP_DTYPE_I32 || out_dtype == LAP_DTYPE_I64,
            "lap_retrieve_select: out dtype must be int32/int64");
  const int R = B * Hkv;
  const int n = cand_end - cand_start;
  const int ke = std::min(k, n);
  if (ke == 0) return LAP_OK;
  const int C2 = (T + kChunk - 1) / kChunk;
  Ws w = carve(workspace, R, T, retrieve_chunk_bound(T), C2);
  LAP_CHECK_CODE(workspace && workspace_bytes >= w.bytes, LAP_ERR_WORKSPACE,
                 "lap_retrieve_select: workspace of %zu bytes needed", w.bytes);
  const int C1 = score_g4_nchunk(R, T);
  LAP_CHECK_CODE(C1 > 0 && C1 <= retrieve_chunk_bound(T), LAP_ERR_HIP,
                 "lap_retrieve_select: device query failed");
  KeySrc ks{w.keys, T, cand_start};
  return run_levels(w, ks, R, n, ke, C1, cand_start, out_idx, out_dtype, k, as_stream(stream));
}

extern "C" int lap_retrieve_topk(const void* lut_gmkg, const uint8_t* codes,
                                 int64_t codes_stride_b, int64_t codes_stride_h,
                                 int64_t codes_stride_t, int B, int Hkv, int T, int cand_start,
                                 int cand_end, int k, int key_mode, void* scores_out,
                                 void* out_idx, int out_dtype, void* workspace,
                                 size_t workspace_bytes, lap_stream_t stream) {
  clear_error();
  LAP_CHECK(out_idx || k == 0, "lap_retrieve_topk: null output");
  int s = lap_retrieve_score(lut_gmkg, codes, codes_stride_b, codes_stride_h, codes_stride_t, B,
                             Hkv, T, cand_start, cand_end, key_mode, scores_out, workspace,
                             workspace_bytes, stream);
  if (s != LAP_OK) return s;
  return lap_retrieve_select(B, Hkv, T, cand_start, cand_end, k, out_idx, out_dtype, workspace,
                             workspace_bytes, stream);
}

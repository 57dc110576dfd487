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
#include "topk_core.h"

#include <cstdlib>
#include <cstring>
#include <type_traits>

namespace lap {

int launch_score_g4(const uint16_t* lut, bool lut_il, const uint8_t* codes, int64_t cs_b,
                    int64_t cs_h, int64_t cs_t, int B, int Hkv, int T, uint16_t* heads,
                    uint16_t* keys, uint32_t* hist, int key_mode, bool per_head,
                    int cand_start, int cand_end, const int32_t* plans, int* nchunk_out,
                    hipStream_t st);
bool score_g4_supported(const uint8_t* codes, int64_t cs_b, int64_t cs_h, int64_t cs_t);
int score_g4_nchunk(int R, int T);

namespace {

constexpr int kChunk = 2048;   // prep chunk; the smallest level chunk (workspace sizing)
constexpr int kThreads = 256;  // prep and small-level workgroups
constexpr int kPer = 8;        // keys per thread in the level kernels, contiguous

template <int KEYMODE>
__device__ __forceinline__ uint32_t key_of(uint16_t h) {
  return KEYMODE == LAP_KEY_BF16 ? bf16_key_of_f16(h) : f16_key(h);
}

// Candidate window [cs, cs + n) and budget k of one top-k row.
struct SelRow {
  int n, k, cs;
};

// Window and budget of every row: one for all rows, or per sequence from
// lap_row_plan (ragged batches; row r belongs to sequence r / rows_per_plan).
struct SelSpec {
  int n, k, cs;              // uniform window and budget (k <= n)
  const int32_t* plans;      // lap_row_plan[B] or null
  int rows_per_plan;
  int k_cols;                // output row width when plans are given
  int t_cols;                // columns available; plans are clamped to them
  __device__ __forceinline__ SelRow row(int r) const {
    if (!plans) return SelRow{n, k, cs};
    const int32_t* p = plans + (int64_t)(r / rows_per_plan) * kPlanInts;
    const int te = min(max(p[0], 0), t_cols);
    const int c0 = min(max(p[2], 0), te), c1 = min(max(p[3], c0), te);
    const int nn = c1 - c0;
    return SelRow{nn, max(0, min(min(p[4], nn), k_cols)), c0};
  }
};

template <int KEYMODE>
__global__ __launch_bounds__(kThreads) void topk_prep_kernel(
    const uint16_t* __restrict__ scores, int64_t row_stride, int R, int group, SelSpec sp,
    int64_t key_stride, int C, uint16_t* __restrict__ keys, uint32_t* __restrict__ hist1) {
  __shared__ uint32_t s_h[256];
  const int r = blockIdx.x % R, c = blockIdx.x / R;
  const SelRow sr = sp.row(r);
  s_h[threadIdx.x] = 0;
  __syncthreads();
  const int e0 = c * kChunk, e1 = min(sr.n, e0 + kChunk);
#pragma unroll 8
  for (int e = e0 + threadIdx.x; e < e1; e += kThreads) {
    uint32_t key = 0;
    for (int g = 0; g < group; ++g) {
      const uint16_t h = scores[(int64_t)(r * group + g) * row_stride + sr.cs + e];
      key = max(key, key_of<KEYMODE>(h));
    }
    keys[(int64_t)r * key_stride + e] = (uint16_t)key;
    atomicAdd(&s_h[key >> 8], 1u);
  }
  __syncthreads();
  hist1[((int64_t)r * C + c) * 256 + threadIdx.x] = s_h[threadIdx.x];
}

// Keys of a row: candidate e of row r is keys[r * stride + e] when the keys
// were stored window-relative (topk_prep_kernel), keys[r * stride + cs + e]
// when they are indexed by column (the fused scorer).
struct KeySrc {
  const uint16_t* keys;
  int64_t stride;
  bool by_column;
  __device__ __forceinline__ const uint16_t* row(int r, const SelRow& sr) const {
    return keys + (int64_t)r * stride + (by_column ? sr.cs : 0);
  }
};

// Sum of n values p[0], p[stride], ... (and of those with index < split),
// NB independent loads in flight per round (the chunk histograms live in
// L2: latency, not bandwidth, is the cost).
template <int NB>
__device__ __forceinline__ void sum_strided(const uint32_t* __restrict__ p, int n,
                                            int64_t stride, int split, uint32_t& tot,
                                            uint32_t& pre) {
  tot = 0;
  pre = 0;
  for (int i0 = 0; i0 < n; i0 += NB) {
    uint32_t v[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) v[u] = p[(int64_t)min(i0 + u, n - 1) * stride];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const bool ok = i0 + u < n;
      tot += ok ? v[u] : 0u;
      pre += ok && i0 + u < split ? v[u] : 0u;
    }
  }
}

// Per-bin sums of a row's chunk histograms h[c][256] over c < C (tot) and
// c < split (pre): TH / 256 threads per bin, thread t taking chunks
// t / 256, t / 256 + TH / 256, ...; the partial sums meet in s_tot[0] and
// s_pre[0] (s_pre may be null).
template <int TH>
__device__ __forceinline__ void sum_chunk_hists(const uint32_t* __restrict__ h, int C, int split,
                                                uint32_t (*s_tot)[256], uint32_t (*s_pre)[256]) {
  constexpr int P = TH / 256;
  const int tid = threadIdx.x, bin = tid & 255, part = tid >> 8;
  uint32_t tot, pre;
  // 32 loads per round for one thread per bin (up to 64 chunks), 8 when four
  // threads share a bin's chunks
  sum_strided<P == 1 ? 32 : 8>(h + (int64_t)part * 256 + bin,
                               part < C ? (C - part + P - 1) / P : 0, P * 256,
                               split > part ? (split - part + P - 1) / P : 0, tot, pre);
  s_tot[part][bin] = tot;
  if (s_pre) s_pre[part][bin] = pre;
  __syncthreads();
  if (P > 1) {
    if (tid < 256) {
#pragma unroll
      for (int q = 1; q < P; ++q) {
        s_tot[0][tid] += s_tot[q][tid];
        if (s_pre) s_pre[0][tid] += s_pre[q][tid];
      }
    }
    __syncthreads();
  }
}

// Level 2 over chunks of kPer * TH candidates (TH = 256 or 1024): the
// threshold bin b1 from the row's level-1 histograms, then the low-byte
// histogram of this chunk's keys in b1 and its count of keys above b1.
template <int TH>
__global__ __launch_bounds__(TH) void topk_level2_kernel(
    KeySrc ks, int R, SelSpec sp, const uint32_t* __restrict__ hist1, int C1, int C,
    uint32_t* __restrict__ hist2, uint32_t* __restrict__ gtc, uint32_t* __restrict__ info) {
  constexpr int CH = kPer * TH;
  __shared__ uint32_t s_h[TH / 256][256], s_h2[256], s_wsum[TH / 64], s_res[2], s_gt;
  const int r = blockIdx.x % R, c = blockIdx.x / R;
  const int tid = threadIdx.x;
  const SelRow sr = sp.row(r);
  const int e0 = c * CH, e1 = min(sr.n, e0 + CH);
  if (sr.k == 0 || e0 >= e1) {  // nothing of this row here (ragged rows only)
    if (tid < 256) hist2[((int64_t)r * C + c) * 256 + tid] = 0u;
    if (tid == 0) gtc[(int64_t)r * C + c] = 0u;
    return;
  }
  // this thread's keys first (unconditional, clamped), so their latency
  // overlaps the histogram sum
  const uint16_t* kr = ks.row(r, sr);
  uint32_t kv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) kv[i] = kr[min(e0 + tid * kPer + i, e1 - 1)];
  if (tid < 256) s_h2[tid] = 0;
  if (tid == 0) s_gt = 0;
  sum_chunk_hists<TH>(hist1 + (int64_t)r * C1 * 256, C1, 0, s_h, nullptr);
  select_bin(s_h[0], (uint32_t)sr.k, s_wsum, s_res);
  const uint32_t b1 = s_res[0];
  if (c == 0 && tid == 0) {
    info[r * 4 + 0] = b1;
    info[r * 4 + 1] = s_res[1];
  }
  uint32_t gt = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    if (e0 + tid * kPer + i >= e1) continue;
    const uint32_t hi = kv[i] >> 8;
    if (hi == b1) atomicAdd(&s_h2[kv[i] & 255u], 1u);
    gt += hi > b1;
  }
  if (gt) atomicAdd(&s_gt, gt);
  __syncthreads();
  if (tid < 256) hist2[((int64_t)r * C + c) * 256 + tid] = s_h2[tid];
  if (tid == 0) gtc[(int64_t)r * C + c] = s_gt;
}

// Threshold tau and the ordered compaction of one chunk: keys above tau,
// then the `need` lowest-column ties, at the chunk's output offset.
template <int TH, typename OUT_T>
__global__ __launch_bounds__(TH) void topk_select_kernel(
    KeySrc ks, int R, SelSpec sp, int C, const uint32_t* __restrict__ hist2,
    const uint32_t* __restrict__ gtc, const uint32_t* __restrict__ info,
    OUT_T* __restrict__ out, int64_t out_stride) {
  constexpr int CH = kPer * TH, W = TH / 64;
  __shared__ uint32_t s_tot[TH / 256][256], s_pre[TH / 256][256], s_wsum[W], s_res[2], s_red[W];
  const int r = blockIdx.x % R, c = blockIdx.x / R;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const SelRow sr = sp.row(r);
  OUT_T* orow = out + (int64_t)r * out_stride;
  if (sp.plans && c == 0)  // ragged rows: pad past the row's k with -1
    for (int i = sr.k + tid; i < sp.k_cols; i += TH) orow[i] = (OUT_T)-1;
  const int e0 = c * CH, e1 = min(sr.n, e0 + CH);
  if (sr.k == 0 || e0 >= e1) return;
  const uint16_t* kr = ks.row(r, sr);
  uint32_t kv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) kv[i] = kr[min(e0 + tid * kPer + i, e1 - 1)];
  const uint32_t b1 = info[r * 4 + 0], gt1 = info[r * 4 + 1];
  // Selected-above-threshold count of earlier chunks (gtc prefix): the first
  // TH counts are requested before the histogram loads and added after them.
  uint32_t g = tid < c ? gtc[(int64_t)r * C + tid] : 0u;
  sum_chunk_hists<TH>(hist2 + (int64_t)r * C * 256, C, c, s_tot, s_pre);
  for (int cc = tid + TH; cc < c; cc += TH) g += gtc[(int64_t)r * C + cc];
  const uint32_t k2 = (uint32_t)sr.k - gt1;
  select_bin(s_tot[0], k2, s_wsum, s_res);
  const uint32_t b2 = s_res[0];
  const uint32_t need = k2 - s_res[1];  // ties at tau to take, >= 1
  const uint32_t tau = (b1 << 8) | b2;
  const uint32_t ties_before = s_pre[0][b2];
  // base = gtc prefix + level-2 keys above b2 in earlier chunks + ties taken.
  uint32_t acc = g + (tid < 256 && tid > (int)b2 ? s_pre[0][tid] : 0u);
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) acc += __shfl_xor(acc, d, 64);
  if (lane == 0) s_red[wave] = acc;
  __syncthreads();
  uint32_t base = 0;
  for (int w = 0; w < W; ++w) base += s_red[w];
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
  const uint32_t tie_rank0 = ties_before + block_exclusive_scan<TH>(ntie, s_wsum, &all_ties);
  // ties this thread may take: ranks [tie_rank0, tie_rank0 + ntie) below need
  const uint32_t take = tie_rank0 >= need ? 0u : min(ntie, need - tie_rank0);
  uint32_t all_sel;
  uint32_t pos = base + block_exclusive_scan<TH>(ngt + take, s_wsum, &all_sel);
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
    if (sel) orow[pos++] = (OUT_T)(sr.cs + e);
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

// Level 2 and the compaction over chunks of candidates; n_max is the widest
// row's window.  Each workgroup re-sums its row's chunk histograms, so more
// rows take longer chunks: 2048-key chunks on 256-thread workgroups while
// they make fewer than 512 workgroups, then 4096-key chunks on 512 threads
// (C2: 8 group rows or 32 per-head rows at 128k) up to 1024 workgroups, then
// 8192-key chunks on 1024 threads.  LAPRUNE_LEVEL_TH=256|512|1024 forces a
// shape.
template <int TH>
int run_levels_th(const Ws& w, KeySrc ks, int R, const SelSpec& sp, int n_max, int C1,
                  void* out, int out_dtype, int64_t out_stride, hipStream_t st) {
  const int C2 = (n_max + kPer * TH - 1) / (kPer * TH);
  if (C2 == 0) return LAP_OK;
  hipLaunchKernelGGL(topk_level2_kernel<TH>, dim3(R * C2), dim3(TH), 0, st, ks, R, sp, w.hist1,
                     C1, C2, w.hist2, w.gtc, w.info);
  LAP_LAUNCH_CHECK("topk_level2_kernel");
  if (out_dtype == LAP_DTYPE_I64)
    hipLaunchKernelGGL((topk_select_kernel<TH, int64_t>), dim3(R * C2), dim3(TH), 0, st, ks, R,
                       sp, C2, w.hist2, w.gtc, w.info, static_cast<int64_t*>(out), out_stride);
  else
    hipLaunchKernelGGL((topk_select_kernel<TH, int32_t>), dim3(R * C2), dim3(TH), 0, st, ks, R,
                       sp, C2, w.hist2, w.gtc, w.info, static_cast<int32_t*>(out), out_stride);
  LAP_LAUNCH_CHECK("topk_select_kernel");
  return LAP_OK;
}

int run_levels(const Ws& w, KeySrc ks, int R, const SelSpec& sp, int n_max, int C1,
               void* out, int out_dtype, int64_t out_stride, hipStream_t st) {
  static const int forced = [] {
    const char* e = getenv("LAPRUNE_LEVEL_TH");
    return e ? atoi(e) : 0;
  }();
  const int64_t small_wgs = (int64_t)R * ((n_max + kChunk - 1) / kChunk);
  const int64_t mid_wgs = (int64_t)R * ((n_max + 2 * kChunk - 1) / (2 * kChunk));
  int th = small_wgs < 512 ? kThreads : mid_wgs <= 1024 ? 512 : 1024;
  if (forced == 256 || forced == 512 || forced == 1024) th = forced;
  if (th == 1024)
    return run_levels_th<1024>(w, ks, R, sp, n_max, C1, out, out_dtype, out_stride, st);
  if (th == 512)
    return run_levels_th<512>(w, ks, R, sp, n_max, C1, out, out_dtype, out_stride, st);
  return run_levels_th<kThreads>(w, ks, R, sp, n_max, C1, out, out_dtype, out_stride, st);
}

// ---- One workgroup per row: level 2 and the compaction in one launch.
//
// Wave w owns the columns [w * 64 * KPT, (w + 1) * 64 * KPT) of the row
// (KPT <= 32, so up to 32768 columns); its lane l holds column
// w * 64 * KPT + 64 e + l as key e, so for every e the wave's 64 lanes cover
// 64 consecutive columns and a ballot orders them.  The level-1 histogram is
// the sum of the scorer's chunk histograms; its threshold bin b1 leaves few
// candidates (the keys of bins >= b1: fewer than k plus one bin), which every
// wave packs in column order into its own LDS segment.  The level-2
// histogram, the tie ranks and the ordered output then run over those
// segments only.  Same result as run_levels (threshold tau, then the `need`
// lowest-column ties).
constexpr int kRowThreads = 1024;
constexpr int kRowWaves = kRowThreads / 64;
constexpr int kRowMaxKpt = 32;

// Dynamic LDS of topk_row_kernel<KPT>: the candidate segments.
constexpr size_t row_kernel_lds(int kpt) { return (size_t)kRowThreads * kpt * sizeof(uint32_t); }

template <int KPT, typename OUT_T>
__global__ __launch_bounds__(kRowThreads) void topk_row_kernel(
    const uint16_t* __restrict__ keys, int64_t key_stride, int T,
    const uint32_t* __restrict__ hist1, int C1, SelSpec sp, OUT_T* __restrict__ out,
    int64_t out_stride) {
  static_assert(KPT % 8 == 0 && KPT <= kRowMaxKpt, "KPT must be 8, 16, 24 or 32");
  extern __shared__ uint32_t s_seg[];  // wave w: [w * 64 * KPT, +count), (key << 16) | column
  __shared__ uint32_t s_h[4][256], s_h2[256], s_wsum[kRowWaves], s_res[2];
  __shared__ uint32_t s_wgt[kRowWaves], s_wtie[kRowWaves];
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const SelRow sr = sp.row(r);
  OUT_T* orow = out + (int64_t)r * out_stride;
  if (sp.plans)  // ragged rows: pad past the row's k with -1
    for (int i = sr.k + tid; i < sp.k_cols; i += kRowThreads) orow[i] = (OUT_T)-1;
  if (sr.k == 0) return;
  const int c0 = sr.cs, c1 = sr.cs + sr.n;

  // Level 1: the scorer's chunk histograms summed per bin (4 partial sums).
  // Their loads go out first (loads retire in order), four at a time.
  const int bin = tid & 255, part = tid >> 8;
  const uint32_t* hp = hist1 + (int64_t)r * C1 * 256 + bin;
  uint32_t hv[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) hv[u] = hp[(int64_t)min(part + 4 * u, C1 - 1) * 256];

  // Keys, one 2-byte load each (64 lanes read 128 contiguous bytes); columns
  // past T load column T - 1 and fall outside the window.
  const int wcol = wave * 64 * KPT;
  const uint16_t* kr = keys + (int64_t)r * key_stride;
  uint32_t kv[KPT];
#pragma unroll
  for (int e = 0; e < KPT; ++e) kv[e] = kr[min(wcol + 64 * e + lane, T - 1)];

  {
    uint32_t a = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) a += part + 4 * u < C1 ? hv[u] : 0u;
    for (int c = part + 16; c < C1; c += 4) a += hp[(int64_t)c * 256];
    s_h[part][bin] = a;
    if (tid < 256) s_h2[tid] = 0;
  }
  __syncthreads();
  if (tid < 256) s_h[0][tid] += s_h[1][tid] + s_h[2][tid] + s_h[3][tid];
  __syncthreads();
  select_bin(s_h[0], (uint32_t)sr.k, s_wsum, s_res);
  const uint32_t b1 = s_res[0], gt1 = s_res[1];

  // Candidates (window keys in bins >= b1) into the wave's segment, in
  // column order.
  const uint32_t lo = b1 << 8;
  uint32_t* seg = s_seg + wcol;
  uint32_t cnt = 0;  // wave-uniform
  auto pack = [&](auto windowed) {
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      const int col = wcol + 64 * e + lane;
      const bool c = kv[e] >= lo && (!decltype(windowed)::value || (col >= c0 && col < c1));
      const uint64_t m = __ballot(c);
      if (c) seg[cnt + lanes_below(m)] = (kv[e] << 16) | (uint32_t)col;
      cnt += (uint32_t)__popcll(m);
    }
  };
  // Wave-uniform: columns all inside the window (no per-key window test),
  // all outside (no candidates), or straddling an edge.
  const int wend = wcol + 64 * KPT;
  if (wcol >= c0 && wend <= c1) pack(std::false_type{});
  else if (wend > c0 && wcol < c1) pack(std::true_type{});
  // Level 2 over this segment's keys of bin b1 (each lane reads what other
  // lanes of its wave wrote: a wavefront-scope fence orders them).
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (uint32_t i = lane; i < cnt; i += 64) {
    const uint32_t key = seg[i] >> 16;
    if ((key >> 8) == b1) atomicAdd(&s_h2[key & 255u], 1u);
  }
  __syncthreads();
  const uint32_t k2 = (uint32_t)sr.k - gt1;
  select_bin(s_h2, k2, s_wsum, s_res);
  const uint32_t tau = (b1 << 8) | s_res[0];
  const uint32_t need = k2 - s_res[1];  // ties at tau to take, >= 1

  // Keys above tau and ties at tau per segment, then each wave's output
  // offset: the selections of the segments before it.
  uint32_t ngt = 0, ntie = 0;
  for (uint32_t i0 = 0; i0 < cnt; i0 += 64) {
    const uint32_t i = i0 + lane;
    const uint32_t key = i < cnt ? seg[i] >> 16 : 0u;
    ngt += (uint32_t)__popcll(__ballot(i < cnt && key > tau));
    ntie += (uint32_t)__popcll(__ballot(i < cnt && key == tau));
  }
  if (lane == 0) {
    s_wgt[wave] = ngt;
    s_wtie[wave] = ntie;
  }
  __syncthreads();
  uint32_t gt_before = 0, tie_before = 0;
  for (int w = 0; w < wave; ++w) {
    gt_before += s_wgt[w];
    tie_before += s_wtie[w];
  }
  uint32_t pos = gt_before + min(tie_before, need);
  uint32_t tie_rank = tie_before;
  for (uint32_t i0 = 0; i0 < cnt; i0 += 64) {
    const uint32_t i = i0 + lane;
    const uint32_t v = i < cnt ? seg[i] : 0u;
    const uint32_t key = v >> 16;
    const bool is_tie = i < cnt && key == tau;
    const uint64_t mt = __ballot(is_tie);
    const bool sel = (i < cnt && key > tau) || (is_tie && tie_rank + lanes_below(mt) < need);
    const uint64_t ms = __ballot(sel);
    if (sel) orow[pos + lanes_below(ms)] = (OUT_T)(v & 0xffffu);
    pos += (uint32_t)__popcll(ms);
    tie_rank += (uint32_t)__popcll(mt);
  }
}

// Keys per thread of topk_row_kernel for a row of T columns, or 0 for the
// two-kernel path.  One workgroup per row pays off up to 32 keys per thread
// (T <= 32768: batched decode rows); longer rows take the chunked levels.
// LAPRUNE_TOPK=levels|row forces a path (row: whenever T fits).
int row_kernel_kpt(int T) {
  static const int mode = [] {
    const char* e = getenv("LAPRUNE_TOPK");
    if (!e) return 0;
    return strcmp(e, "levels") == 0 ? 1 : strcmp(e, "row") == 0 ? 2 : 0;
  }();
  if (mode == 1 || T < 1) return 0;
  for (int kpt = 8; kpt <= kRowMaxKpt; kpt *= 2)
    if ((int64_t)kpt * kRowThreads >= T) return kpt;
  return 0;
}

template <typename OUT_T>
void launch_row_kernel(int kpt, const uint16_t* keys, int64_t key_stride, int T,
                       const uint32_t* hist1, int C1, const SelSpec& sp, int R, OUT_T* out,
                       int64_t out_stride, hipStream_t st) {
  switch (kpt) {
#define LAP_ROWK(K)                                                                      \
  case K:                                                                                \
    hipLaunchKernelGGL((topk_row_kernel<K, OUT_T>), dim3(R), dim3(kRowThreads),          \
                       row_kernel_lds(K), st, keys, key_stride, T, hist1, C1, sp, out,   \
                       out_stride);                                                      \
    break;
    LAP_ROWK(8) LAP_ROWK(16) LAP_ROWK(32)
#undef LAP_ROWK
  }
}

// Upper bound on the scorer's workgroup chunks per row: a chunk holds at
// least one pass of the smallest launch shape (256 threads x 1 token).
int retrieve_chunk_bound(int T) { return (T + 255) / 256; }

}  // namespace
}  // namespace lap

using namespace lap;

namespace {

SelSpec uniform_spec(int cand_start, int n, int k_eff) {
  SelSpec sp{};
  sp.n = n;
  sp.k = k_eff;
  sp.cs = cand_start;
  sp.rows_per_plan = 1;
  sp.k_cols = k_eff;
  return sp;
}

SelSpec ragged_spec(const lap_row_plan* plans, int rows_per_plan, int k_cols, int T) {
  SelSpec sp{};
  sp.plans = reinterpret_cast<const int32_t*>(plans);
  sp.rows_per_plan = rows_per_plan;
  sp.k_cols = k_cols;
  sp.t_cols = T;
  return sp;
}

// fp16 scores -> window-relative keys (row stride n_max) and level-1
// histograms, then the two levels.
int select_from_scores(const void* scores, int64_t row_stride, int R, int group, int key_mode,
                       const SelSpec& sp, int n_max, void* out_idx, int out_dtype,
                       int64_t out_stride, void* workspace, size_t ws_bytes, const char* who,
                       hipStream_t st) {
  const int C = (n_max + kChunk - 1) / kChunk;
  Ws w = carve(workspace, R, n_max, C, C);
  LAP_CHECK_CODE(workspace && ws_bytes >= w.bytes, LAP_ERR_WORKSPACE,
                 "%s: workspace of %zu bytes needed", who, w.bytes);
  const uint16_t* S = static_cast<const uint16_t*>(scores);
  if (key_mode == LAP_KEY_BF16)
    hipLaunchKernelGGL(topk_prep_kernel<LAP_KEY_BF16>, dim3(R * C), dim3(kThreads), 0, st, S,
                       row_stride, R, group, sp, (int64_t)n_max, C, w.keys, w.hist1);
  else
    hipLaunchKernelGGL(topk_prep_kernel<LAP_KEY_F16>, dim3(R * C), dim3(kThreads), 0, st, S,
                       row_stride, R, group, sp, (int64_t)n_max, C, w.keys, w.hist1);
  LAP_LAUNCH_CHECK("topk_prep_kernel");
  KeySrc ks{w.keys, n_max, false};
  return run_levels(w, ks, R, sp, n_max, C, out_idx, out_dtype, out_stride, st);
}

int check_key_and_out(int key_mode, int out_dtype, const char* who) {
  LAP_CHECK(key_mode == LAP_KEY_F16 || key_mode == LAP_KEY_BF16, "%s: bad key mode", who);
  LAP_CHECK(out_dtype == LAP_DTYPE_I32 || out_dtype == LAP_DTYPE_I64,
            "%s: out dtype must be int32/int64", who);
  return LAP_OK;
}

}  // namespace

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
  int s = check_key_and_out(key_mode, out_dtype, "lap_topk_select");
  if (s != LAP_OK) return s;
  const int n = cand_end - cand_start;
  const int ke = std::min(k, n);
  if (ke == 0) return LAP_OK;
  return select_from_scores(scores, score_row_stride, R, group, key_mode,
                            uniform_spec(cand_start, n, ke), n, out_idx, out_dtype, k, workspace,
                            workspace_bytes, "lap_topk_select", as_stream(stream));
}

extern "C" int lap_topk_select_ragged(const void* scores, int64_t score_row_stride, int R,
                                      int group, int rows_per_plan, int T,
                                      const lap_row_plan* plans, int k_cols, int key_mode,
                                      void* out_idx, int out_dtype, void* workspace,
                                      size_t workspace_bytes, lap_stream_t stream) {
  clear_error();
  LAP_CHECK(scores && plans && (out_idx || k_cols == 0), "lap_topk_select_ragged: null pointer");
  LAP_CHECK(R > 0 && group > 0 && T > 0 && k_cols >= 0, "lap_topk_select_ragged: bad sizes");
  LAP_CHECK(rows_per_plan > 0 && R % rows_per_plan == 0,
            "lap_topk_select_ragged: R=%d is not a multiple of rows_per_plan=%d", R,
            rows_per_plan);
  LAP_CHECK(score_row_stride >= T, "lap_topk_select_ragged: row stride < T");
  int s = check_key_and_out(key_mode, out_dtype, "lap_topk_select_ragged");
  if (s != LAP_OK) return s;
  if (k_cols == 0) return LAP_OK;
  return select_from_scores(scores, score_row_stride, R, group, key_mode,
                            ragged_spec(plans, rows_per_plan, k_cols, T), T, out_idx, out_dtype,
                            k_cols, workspace, workspace_bytes, "lap_topk_select_ragged",
                            as_stream(stream));
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
                           int64_t cs_h, int64_t cs_t, int B, int Hkv, int T, int key_mode,
                           const char* who) {
  LAP_CHECK(lut_gmkg && codes, "%s: null pointer", who);
  LAP_CHECK(B > 0 && Hkv > 0 && T > 0, "%s: bad sizes", who);
  const int km = key_mode & ~LAP_SELECT_PER_HEAD;
  LAP_CHECK(km == LAP_KEY_F16 || km == LAP_KEY_BF16, "%s: bad key mode", who);
  LAP_CHECK(cs_t >= 32, "%s: codes token stride < M=32", who);
  LAP_CHECK_CODE(score_g4_supported(codes, cs_b, cs_h, cs_t), LAP_ERR_UNSUPPORTED,
                 "%s: codes base and strides must be 16-byte aligned", who);
  return LAP_OK;
}

// Selection rows per KV row: 4 (one per query head) with LAP_SELECT_PER_HEAD,
// else 1 (the group max).
static int rows_per_kv(int key_mode) { return (key_mode & LAP_SELECT_PER_HEAD) ? 4 : 1; }

// The fused scorer: per-head scores (optional), column-indexed selection
// keys and level-1 histograms in the workspace (B * Hkv * rows_per_kv rows).
static int retrieve_score_impl(const void* lut_gmkg, const uint8_t* codes, int64_t cs_b,
                               int64_t cs_h, int64_t cs_t, int B, int Hkv, int T, int cand_start,
                               int cand_end, const lap_row_plan* plans, int key_mode,
                               void* scores_out, void* workspace, size_t workspace_bytes,
                               const char* who, hipStream_t st) {
  const int R = B * Hkv * rows_per_kv(key_mode);
  const int C2 = (T + kChunk - 1) / kChunk;
  Ws w = carve(workspace, R, T, retrieve_chunk_bound(T), C2);
  LAP_CHECK_CODE(workspace && workspace_bytes >= w.bytes, LAP_ERR_WORKSPACE,
                 "%s: workspace of %zu bytes needed", who, w.bytes);
  int C1 = 0;
  int s = launch_score_g4(static_cast<const uint16_t*>(lut_gmkg), true, codes, cs_b, cs_h, cs_t,
                          B, Hkv, T, static_cast<uint16_t*>(scores_out), w.keys, w.hist1,
                          key_mode & ~LAP_SELECT_PER_HEAD, rows_per_kv(key_mode) == 4,
                          cand_start, cand_end, reinterpret_cast<const int32_t*>(plans), &C1,
                          st);
  if (s != LAP_OK) return s;
  LAP_CHECK_CODE(C1 <= retrieve_chunk_bound(T), LAP_ERR_INVALID,
                 "%s: internal chunk bound exceeded", who);
  return LAP_OK;
}

// Levels over the keys and histograms retrieve_score_impl left, for the
// B * Hkv * rpk selection rows (rpk as the scorer ran: 1 or 4).
static int retrieve_select_impl(int B, int Hkv, int rpk, int T, const SelSpec& sp, int n_max,
                                void* out_idx, int out_dtype, int64_t out_stride,
                                void* workspace, size_t workspace_bytes, const char* who,
                                hipStream_t st) {
  const int R = B * Hkv * rpk;
  const int C2 = (T + kChunk - 1) / kChunk;
  Ws w = carve(workspace, R, T, retrieve_chunk_bound(T), C2);
  LAP_CHECK_CODE(workspace && workspace_bytes >= w.bytes, LAP_ERR_WORKSPACE,
                 "%s: workspace of %zu bytes needed", who, w.bytes);
  const int C1 = score_g4_nchunk(B * Hkv, T);  // the scorer's chunks per KV row
  LAP_CHECK_CODE(C1 > 0 && C1 <= retrieve_chunk_bound(T), LAP_ERR_HIP,
                 "%s: device query failed", who);
  const int kpt = row_kernel_kpt(T);
  if (kpt > 0) {
    if (out_dtype == LAP_DTYPE_I64)
      launch_row_kernel<int64_t>(kpt, w.keys, T, T, w.hist1, C1, sp, R,
                                 static_cast<int64_t*>(out_idx), out_stride, st);
    else
      launch_row_kernel<int32_t>(kpt, w.keys, T, T, w.hist1, C1, sp, R,
                                 static_cast<int32_t*>(out_idx), out_stride, st);
    LAP_LAUNCH_CHECK("topk_row_kernel");
    return LAP_OK;
  }
  KeySrc ks{w.keys, T, true};
  return run_levels(w, ks, R, sp, n_max, C1, out_idx, out_dtype, out_stride, st);
}

extern "C" int lap_retrieve_score(const void* lut_gmkg, const uint8_t* codes,
                                  int64_t codes_stride_b, int64_t codes_stride_h,
                                  int64_t codes_stride_t, int B, int Hkv, int T, int cand_start,
                                  int cand_end, int key_mode, void* scores_out,
                                  void* workspace, size_t workspace_bytes,
                                  lap_stream_t stream) {
  clear_error();
  int s = retrieve_checks(lut_gmkg, codes, codes_stride_b, codes_stride_h, codes_stride_t, B,
                          Hkv, T, key_mode, "lap_retrieve_score");
  if (s != LAP_OK) return s;
  LAP_CHECK(cand_start >= 0 && cand_end <= T && cand_start <= cand_end,
            "lap_retrieve_score: candidate window [%d,%d) outside [0,%d)", cand_start, cand_end,
            T);
  return retrieve_score_impl(lut_gmkg, codes, codes_stride_b, codes_stride_h, codes_stride_t, B,
                             Hkv, T, cand_start, cand_end, nullptr, key_mode, scores_out,
                             workspace, workspace_bytes, "lap_retrieve_score", as_stream(stream));
}

static int retrieve_select_uniform(int B, int Hkv, int rpk, int T, int cand_start, int cand_end,
                                   int k, void* out_idx, int out_dtype, void* workspace,
                                   size_t workspace_bytes, const char* who, hipStream_t st) {
  LAP_CHECK(out_idx, "%s: null output", who);
  LAP_CHECK(B > 0 && Hkv > 0 && T > 0, "%s: bad sizes", who);
  LAP_CHECK(cand_start >= 0 && cand_end <= T && cand_start <= cand_end,
            "%s: candidate window [%d,%d) outside [0,%d)", who, cand_start, cand_end, T);
  LAP_CHECK(k >= 0, "%s: k must be non-negative", who);
  LAP_CHECK(out_dtype == LAP_DTYPE_I32 || out_dtype == LAP_DTYPE_I64,
            "%s: out dtype must be int32/int64", who);
  const int n = cand_end - cand_start;
  const int ke = std::min(k, n);
  if (ke == 0) return LAP_OK;
  return retrieve_select_impl(B, Hkv, rpk, T, uniform_spec(cand_start, n, ke), n, out_idx,
                              out_dtype, k, workspace, workspace_bytes, who, st);
}

extern "C" int lap_retrieve_select(int B, int Hkv, int T, int cand_start, int cand_end, int k,
                                   void* out_idx, int out_dtype, void* workspace,
                                   size_t workspace_bytes, lap_stream_t stream) {
  clear_error();
  return retrieve_select_uniform(B, Hkv, 1, T, cand_start, cand_end, k, out_idx, out_dtype,
                                 workspace, workspace_bytes, "lap_retrieve_select",
                                 as_stream(stream));
}

extern "C" int lap_retrieve_select_heads(int B, int Hkv, int T, int cand_start, int cand_end,
                                         int k, void* out_idx, int out_dtype, void* workspace,
                                         size_t workspace_bytes, lap_stream_t stream) {
  clear_error();
  return retrieve_select_uniform(B, Hkv, 4, T, cand_start, cand_end, k, out_idx, out_dtype,
                                 workspace, workspace_bytes, "lap_retrieve_select_heads",
                                 as_stream(stream));
}

extern "C" int lap_retrieve_topk(const void* lut_gmkg, const uint8_t* codes,
                                 int64_t codes_stride_b, int64_t codes_stride_h,
                                 int64_t codes_stride_t, int B, int Hkv, int T, int cand_start,
                                 int cand_end, int k, int key_mode, void* scores_out,
                                 void* out_idx, int out_dtype, void* workspace,
                                 size_t workspace_bytes, lap_stream_t stream) {
  clear_error();
  LAP_CHECK(out_idx || k == 0, "lap_retrieve_topk: null output");
  LAP_CHECK(k >= 0, "lap_retrieve_topk: k must be non-negative");
  int s = lap_retrieve_score(lut_gmkg, codes, codes_stride_b, codes_stride_h, codes_stride_t, B,
                             Hkv, T, cand_start, cand_end, key_mode, scores_out, workspace,
                             workspace_bytes, stream);
  if (s != LAP_OK || k == 0) return s;
  return retrieve_select_uniform(B, Hkv, rows_per_kv(key_mode), T, cand_start, cand_end, k,
                                 out_idx, out_dtype, workspace, workspace_bytes,
                                 "lap_retrieve_topk", as_stream(stream));
}

extern "C" int lap_retrieve_topk_ragged(const void* lut_gmkg, const uint8_t* codes,
                                        int64_t codes_stride_b, int64_t codes_stride_h,
                                        int64_t codes_stride_t, int B, int Hkv, int T,
                                        const lap_row_plan* plans, int k_cols, int key_mode,
                                        void* scores_out, void* out_idx, int out_dtype,
                                        void* workspace, size_t workspace_bytes,
                                        lap_stream_t stream) {
  clear_error();
  const char* who = "lap_retrieve_topk_ragged";
  int s = retrieve_checks(lut_gmkg, codes, codes_stride_b, codes_stride_h, codes_stride_t, B,
                          Hkv, T, key_mode, who);
  if (s != LAP_OK) return s;
  LAP_CHECK(plans, "%s: null plans", who);
  LAP_CHECK(k_cols >= 0 && (out_idx || k_cols == 0), "%s: bad output", who);
  LAP_CHECK(out_dtype == LAP_DTYPE_I32 || out_dtype == LAP_DTYPE_I64,
            "%s: out dtype must be int32/int64", who);
  hipStream_t st = as_stream(stream);
  s = retrieve_score_impl(lut_gmkg, codes, codes_stride_b, codes_stride_h, codes_stride_t, B, Hkv,
                          T, 0, 0, plans, key_mode, scores_out, workspace, workspace_bytes, who,
                          st);
  if (s != LAP_OK || k_cols == 0) return s;
  const int rpk = rows_per_kv(key_mode);
  return retrieve_select_impl(B, Hkv, rpk, T, ragged_spec(plans, Hkv * rpk, k_cols, T), T,
                              out_idx, out_dtype, k_cols, workspace, workspace_bytes, who, st);
}

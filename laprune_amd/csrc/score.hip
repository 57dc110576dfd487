// score.hip — A2: AQ LUT scoring of cached keys.
//
// Accumulation contract shared by every scorer here and by the reference
// kernels (aq_kernels/aq_lut_gqa.cu:69-74, :134-147, :195-210):
//     acc = 0.0f;  for m ascending: acc += (float)lut_fp16[h, m, code_m];
//     score = fp16_rne(acc)
//
// Fast path (G = 4, M = 32, K = 256; Llama-3.1 GQA): one KV group's table
// [M][K][G] fp16 = 64 KiB sits in LDS, so the four query heads of a code are
// one 8-byte LDS read.  Each 32-byte code row arrives as two 16-byte loads.
// The per-head add is one v_fma_mix_f32 (exact fp16->fp32 widening fused
// with the fp32 add).  The grid is 1-D with the KV row in the low bits of the
// block id: workgroups are dealt round-robin to the 8 XCDs, so with 8 KV rows
// each XCD scores one KV group and its 64 KiB table stays in that XCD's L2.
// The table comes from either LUT layout: the interleaved [Hkv][M][K][G]
// is copied, the reference's [Hkv*G][M][K] is interleaved while it is
// loaded.  Optionally the kernel also emits selection keys (the group max of
// the four fp16 head scores, or each head's own score, as orderable 16-bit
// keys) and per-workgroup 256-bin histograms of the keys' high byte over the
// candidate window, the first radix level of the top-k (topk.hip).
#include "common.h"
#include "score_core.h"

#include <cstdlib>
#include <cstring>

namespace lap {

namespace {

struct ScoreOut {
  uint16_t* heads;   // [R*4][T] fp16 or null
  uint16_t* keys;    // [R][T] u16 (group max), [R*4][T] with per_head; or null
  uint32_t* hist;    // [R][nchunk][256], [R*4][nchunk][256] with per_head; or null
  int key_mode;
  int cand_start, cand_end;
  const int32_t* plans;  // lap_row_plan[B] (ragged batches) or null
  int per_head;          // keys and histograms per query head instead of per KV row
};

// Selection rows a KV row feeds: its four query heads, or itself.
__device__ __forceinline__ int key_rows(const ScoreOut& so) { return so.per_head ? kG : 1; }

// Columns a row scores, [0, t_end), and its histogram window [cs, ce): the
// call's scalars, or the sequence's plan clamped to the T scored columns.
struct RowCols {
  int t_end, cs, ce;
};
__device__ __forceinline__ RowCols row_cols(const ScoreOut& so, int b, int T) {
  if (!so.plans) return RowCols{T, so.cand_start, so.cand_end};
  const int32_t* p = so.plans + (int64_t)b * kPlanInts;
  return RowCols{min(max(p[0], 0), T), p[2], p[3]};
}


// Copy the workgroup's level-1 histograms (one per selection row of KV row
// r, the sum of its copies) to [row][nchunk][256]; with s_hist null, zeros
// (a chunk past the row's columns).
template <int HC>
__device__ __forceinline__ void write_hists(const ScoreOut& so, HistRows<HC> s_hist, int r,
                                            int R, int chunk, int tid, int threads) {
  if (!so.hist) return;
  const int nchunk = gridDim.x / R, rows = key_rows(so);
  for (int i = tid; i < rows * 256; i += threads) {
    const int g = i >> 8, bin = i & 255;
    uint32_t v = 0;
    if (s_hist) {
#pragma unroll
      for (int c = 0; c < HC; ++c) v += s_hist[g][c * kHPitch + bin];
    }
    so.hist[(((int64_t)r * rows + g) * nchunk + chunk) * 256 + bin] = v;
  }
}
__device__ __forceinline__ void write_empty_hist(const ScoreOut& so, int r, int R, int chunk,
                                                 int tid, int threads) {
  write_hists<1>(so, nullptr, r, R, chunk, tid, threads);
}

// Selection keys.  A group row keys fp16(max of its four fp32 head scores),
// which equals the max of the four fp16 scores' keys since fp16 rounding is
// monotone; per-head rows key each head's own score.  bf16 keys rank the
// model-dtype cast of the fp16 score (aq_evaluation.py:166).  The key mode is
// a uniform select, not a branch: this runs once or four times per token.
__device__ __forceinline__ uint32_t key_of_score(float e, bool kbf) {
  const uint16_t h = f2h(e);
  return kbf ? bf16_key_of_f16(h) : f16_key(h);
}

// Pipelined fused scorer (either table layout).  A workgroup owns THREADS * TOK
// consecutive tokens of one KV row; thread tid scores tokens
// t0 + j * THREADS + tid, j < TOK, as TOK stages.  Every CU of the chip
// starts at once, so requesting all code rows up front lets the memory
// system share bandwidth evenly and complete every wave's rows near the end
// of the whole stream, after which all CUs compute with HBM idle.  Instead a
// thread keeps PREF stages in flight: it requests stage j + PREF only when
// stage j has arrived, so early stages complete early and the lookups of
// stage j overlap the stream of the later ones.  The table slice is
// requested first and the first stages only once it is in LDS: the lookups
// are the kernel's bound (random 8-byte LDS reads, about six cycles per wave
// instruction with bank conflicts), so the table, which every lookup needs,
// goes first.  The barrier after the fill orders LDS only, and the waves
// lower their priority stage by stage (stage_prio) so that they finish
// together.  The ordered loads and their waits are in score_core.h.
//
// PH: per-head selection keys (a template parameter, so the two key modes
// are separate kernels in traces and the key code folds).
// HC: level-1 histogram copies per selection row (see kHPitch).
template <int THREADS, int TOK, int PREF, bool IL, bool PH, int HC>
__global__ __launch_bounds__(THREADS) void score_g4p_kernel(
    const uint16_t* __restrict__ lut, const uint8_t* __restrict__ codes, int64_t cs_b,
    int64_t cs_h, int64_t cs_t, int Hkv, int R, int T, ScoreOut so_arg, _Float16 one) {
  ScoreOut so = so_arg;
  so.per_head = PH;
  constexpr int kFill = kLutBytes / 16 / THREADS;  // table uint4s per thread
  constexpr int kAhead = PREF < TOK ? PREF : TOK;  // stages requested up front
  static_assert(kFill * THREADS * 16 == kLutBytes && THREADS >= 256 && kFill % 4 == 0,
                "bad THREADS");
  static_assert(kFill <= 23 && 2 * kAhead <= 16, "vmcnt range");
  __shared__ __attribute__((aligned(16))) uint4 s_lut[kLutBytes / 16];
  __shared__ uint32_t s_hist[PH ? kG : 1][HC * kHPitch];

  // The table loads go out first, before anything else reads the kernel
  // arguments: they need only the row (lut and R), and everything after
  // them (the row's plan, a second round of argument loads) would otherwise
  // delay the table, which every lookup waits for, by a scalar-load round
  // trip or two (about 0.5 us at C2).
  const int r = blockIdx.x % R;
  const int tid = threadIdx.x;
  const uint4* src = reinterpret_cast<const uint4*>(lut + (int64_t)r * (kG * kM * kK));
  // The table: the interleaved layout is copied as is; the reference layout
  // [4][M][K] is read as 8 consecutive entries of each head per group of
  // four loads and interleaved in registers.
  u32x4 f[kFill];
  if constexpr (IL) {
#pragma unroll
    for (int i = 0; i < kFill; ++i) f[i] = gload16_ordered(src + i * THREADS + tid);
  } else {
    const uint16_t* hsrc = lut + (int64_t)r * (kG * kM * kK);
#pragma unroll
    for (int j = 0; j < kFill / 4; ++j) {
      const int e0 = (j * THREADS + tid) * 8;
#pragma unroll
      for (int g = 0; g < kG; ++g) f[4 * j + g] = gload16_ordered(hsrc + g * (kM * kK) + e0);
    }
  }

  const int chunk = blockIdx.x / R;
  const int b = r / Hkv, hkv = r - b * Hkv;
  const RowCols rc = row_cols(so, b, T);
  const int t0 = chunk * (THREADS * TOK);
  const int t1 = min(rc.t_end, t0 + THREADS * TOK);  // without plans t1 > t0 by the grid
  if (t0 >= t1) {
    vm_wait(0, f[0]);  // the table loads drain before the wave ends
    write_empty_hist(so, r, R, chunk, tid, THREADS);
    return;
  }

  // Rows past the chunk end load the chunk's last row (always in bounds) and
  // are discarded after scoring.
  const uint8_t* crow = codes + (int64_t)b * cs_b + (int64_t)hkv * cs_h;
  u32x4 c[TOK][2];
  auto request = [&](int j) {
    const int t = min(t0 + j * THREADS + tid, t1 - 1);
    const uint8_t* p = crow + (int64_t)t * cs_t;
    c[j][0] = gload16_stream(p);
    c[j][1] = gload16_stream(p + 16);
  };

  if constexpr (IL) {
#pragma unroll
    for (int i = 0; i < kFill; ++i) {
      vm_wait(kFill - 1 - i, f[i]);
      s_lut[i * THREADS + tid] = as_uint4(f[i]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < kFill / 4; ++j) {
      vm_wait(kFill - 4 - 4 * j, f[4 * j], f[4 * j + 1], f[4 * j + 2], f[4 * j + 3]);
      interleave_heads(f[4 * j], f[4 * j + 1], f[4 * j + 2], f[4 * j + 3],
                       &s_lut[(j * THREADS + tid) * 4]);
    }
  }
  // The first code rows are requested once the table is in: issued together
  // with the table they compete with it for the memory system, and the table
  // (which every lookup needs) then arrives later than the rows do.
#pragma unroll
  for (int j = 0; j < kAhead; ++j) request(j);
  for (int i = tid; i < (PH ? kG : 1) * HC * kHPitch; i += THREADS)
    s_hist[i / (HC * kHPitch)][i % (HC * kHPitch)] = 0;
  lds_barrier();

  // The scores and keys stay in registers until every stage is in: a store
  // issued between two stage waits would count in the next wait (stores and
  // loads share vmcnt), which would then wait for the store's
  // acknowledgement as well as for the stage.
  const char* lds = reinterpret_cast<const char*>(s_lut);
  const uint32_t copy = (uint32_t)(__lane_id() % HC) * kHPitch;
  const int lo = max(rc.cs, 0), hi = min(rc.ce, t1);  // histogram window in this chunk
  const bool kbf = so.key_mode == LAP_KEY_BF16;
  float sc[TOK][kG];
  uint32_t kw[TOK][PH ? 2 : 1];  // group key, or the four heads' keys two per word
  auto count = [&](int j) {
    if constexpr (PH) {
      atomicAdd(&s_hist[0][copy + ((kw[j][0] & 0xffffu) >> 8)], 1u);
      atomicAdd(&s_hist[1][copy + (kw[j][0] >> 24)], 1u);
      atomicAdd(&s_hist[2][copy + ((kw[j][1] & 0xffffu) >> 8)], 1u);
      atomicAdd(&s_hist[3][copy + (kw[j][1] >> 24)], 1u);
    } else {
      atomicAdd(&s_hist[0][copy + (kw[j][0] >> 8)], 1u);
    }
  };
#pragma unroll
  for (int j = 0; j < TOK; ++j) {
    // Stages requested after stage j so far: j+1 .. min(j+kAhead-1, TOK-1).
    const int later = (j + kAhead - 1 < TOK - 1 ? j + kAhead - 1 : TOK - 1) - j;
    vm_wait(2 * later, c[j][0], c[j][1]);
    stage_prio(j, TOK);
    if (j + kAhead < TOK) request(j + kAhead);
    float e0 = 0.f, e1 = 0.f, e2 = 0.f, e3 = 0.f;
    score_token(lds, as_uint4(c[j][0]), as_uint4(c[j][1]), one, e0, e1, e2, e3);
    sc[j][0] = e0;
    sc[j][1] = e1;
    sc[j][2] = e2;
    sc[j][3] = e3;
    if constexpr (PH) {
      kw[j][0] = key_of_score(e0, kbf) | (key_of_score(e1, kbf) << 16);
      kw[j][1] = key_of_score(e2, kbf) | (key_of_score(e3, kbf) << 16);
    } else {
      kw[j][0] = key_of_score(fmaxf(fmaxf(e0, e1), fmaxf(e2, e3)), kbf);
    }
    if (so.hist) {
      // a stage wholly inside the window (the common case) counts without a
      // per-lane test
      const int ts = t0 + j * THREADS, t = ts + tid;
      if (ts >= lo && ts + THREADS <= hi) count(j);
      else if (t >= lo && t < hi) count(j);
    }
  }
#pragma unroll
  for (int j = 0; j < TOK; ++j) {
    const int t = t0 + j * THREADS + tid;
    if (t >= t1) continue;
    if (so.heads) {
      uint16_t* hp = so.heads + (int64_t)(r * kG) * T + t;
#pragma unroll
      for (int g = 0; g < kG; ++g) hp[g * (int64_t)T] = f2h(sc[j][g]);
    }
    if (so.keys) {
      if constexpr (PH) {
        uint16_t* kp = so.keys + (int64_t)r * kG * T + t;
        kp[0] = (uint16_t)kw[j][0];
        kp[T] = (uint16_t)(kw[j][0] >> 16);
        kp[2 * (int64_t)T] = (uint16_t)kw[j][1];
        kp[3 * (int64_t)T] = (uint16_t)(kw[j][1] >> 16);
      } else {
        so.keys[(int64_t)r * T + t] = (uint16_t)kw[j][0];
      }
    }
  }

  if (so.hist) {
    __syncthreads();
    write_hists<HC>(so, s_hist, r, R, chunk, tid, THREADS);
  }
}

// Generic grouped scorer: G <= 4, any M, K.  Table [G][M][K] fp16 in LDS.
__global__ __launch_bounds__(256) void score_grouped_generic_kernel(
    const uint16_t* __restrict__ lut, int lut_layout, const uint8_t* __restrict__ codes,
    int64_t cs_h, int64_t cs_t, int G, int T, int M, int K, uint16_t* __restrict__ out,
    _Float16 one) {
  extern __shared__ __attribute__((aligned(16))) uint16_t s_tab[];  // [G][M][K]
  const int hkv = blockIdx.x;
  const int MK = M * K;
  for (int i = threadIdx.x; i < G * MK; i += blockDim.x) {
    uint16_t v;
    if (lut_layout == LAP_LUT_HMK) {
      v = lut[(int64_t)hkv * G * MK + i];
    } else {  // [Hkv][M][K][G] -> [G][M][K]
      const int g = i / MK, mk = i - g * MK;
      v = lut[((int64_t)hkv * MK + mk) * G + g];
    }
    s_tab[i] = v;
  }
  __syncthreads();
  const uint8_t* crow = codes + (int64_t)hkv * cs_h;
  for (int t = blockIdx.y * blockDim.x + threadIdx.x; t < T; t += gridDim.y * blockDim.x) {
    const uint8_t* cp = crow + (int64_t)t * cs_t;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int m = 0; m < M; ++m) {
      const int code = cp[m];
#pragma unroll
      for (int g = 0; g < 4; ++g)
        if (g < G) acc[g] = acc_f16(acc[g], __builtin_bit_cast(_Float16, s_tab[(g * M + m) * K + code]), one);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g)
      if (g < G) out[((int64_t)hkv * G + g) * T + t] = f2h(acc[g]);
  }
}

// Per-query-head scorer over an M sub-range, dense or over an index list
// (reference aq_kernels/aq_lut_gqa.cu:20-76).
__global__ __launch_bounds__(256) void score_gqa_kernel(
    const uint16_t* __restrict__ lut, const uint8_t* __restrict__ codes, int64_t cs_h,
    int64_t cs_t, int G, int T, int N, int M_start, int M_range, int M_stride, int K,
    const int64_t* __restrict__ indices, uint16_t* __restrict__ out, _Float16 one) {
  extern __shared__ __attribute__((aligned(16))) uint16_t s_tab[];  // [M_range][K]
  const int h = blockIdx.x;
  const int hkv = h / G;
  const uint16_t* src = lut + ((int64_t)h * M_stride + M_start) * K;
  for (int i = threadIdx.x; i < M_range * K; i += blockDim.x) s_tab[i] = src[i];
  __syncthreads();
  for (int n = blockIdx.y * blockDim.x + threadIdx.x; n < N; n += gridDim.y * blockDim.x) {
    int64_t t = n;
    if (indices) {
      t = indices[(int64_t)h * N + n];
      if (t < 0 || t >= T) {
        out[(int64_t)h * N + n] = 0;
        continue;
      }
    }
    const uint8_t* cp = codes + (int64_t)hkv * cs_h + t * cs_t + M_start;
    float acc = 0.f;
    for (int m = 0; m < M_range; ++m)
      acc = acc_f16(acc, __builtin_bit_cast(_Float16, s_tab[m * K + cp[m]]), one);
    out[(int64_t)h * N + n] = f2h(acc);
  }
}

template <typename CT>
__device__ __forceinline__ int code_index(CT v, int K) {
  int c = (int)(uint8_t)(v);  // low 8 bits as an unsigned code
  return c >= K ? K - 1 : c;  // c >= 0 by construction
}

// Non-GQA scorer (reference aq_kernels/aq_lut.cu:581-639).
template <typename CT, bool F32>
__global__ __launch_bounds__(256) void score_mha_kernel(const void* __restrict__ lut,
                                                        const CT* __restrict__ codes, int Q,
                                                        int N, int M, int K,
                                                        void* __restrict__ out, _Float16 one) {
  const int q = blockIdx.x;
  const int n = blockIdx.y * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const CT* cp = codes + ((int64_t)q * N + n) * M;
  const int64_t lrow = (int64_t)q * M * K;
  float acc = 0.f;
  if (F32) {
    const float* L = static_cast<const float*>(lut) + lrow;
    for (int m = 0; m < M; ++m) acc = acc + L[m * K + code_index(cp[m], K)];
    static_cast<float*>(out)[(int64_t)q * N + n] = acc;
  } else {
    const uint16_t* L = static_cast<const uint16_t*>(lut) + lrow;
    for (int m = 0; m < M; ++m)
      acc = acc_f16(acc, __builtin_bit_cast(_Float16, L[m * K + code_index(cp[m], K)]), one);
    static_cast<uint16_t*>(out)[(int64_t)q * N + n] = f2h(acc);
  }
}

// Direct scorer without a table (reference aq_kernels/aq_lut.cu:37-149).
template <typename CT, bool F32>
__global__ __launch_bounds__(256) void aq_direct_kernel(const void* __restrict__ qv,
                                                        const void* __restrict__ cbv,
                                                        const CT* __restrict__ codes, int Q,
                                                        int N, int M, int K, int D,
                                                        void* __restrict__ out) {
  const int q = blockIdx.x;
  const int n = blockIdx.y * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const CT* cp = codes + ((int64_t)q * N + n) * M;
  float acc = 0.f;
  if (F32) {
    const float* qq = static_cast<const float*>(qv) + (int64_t)q * D;
    const float* cb = static_cast<const float*>(cbv);
    for (int m = 0; m < M; ++m) {
      const int c = (int)(uint8_t)cp[m];
      if (c >= K) continue;
      const float* row = cb + ((int64_t)m * K + c) * D;
      for (int i = 0; i < D; ++i) acc = __builtin_fmaf(qq[i], row[i], acc);
    }
    static_cast<float*>(out)[(int64_t)q * N + n] = acc;
  } else {
    const _Float16* qq = static_cast<const _Float16*>(qv) + (int64_t)q * D;
    const _Float16* cb = static_cast<const _Float16*>(cbv);
    for (int m = 0; m < M; ++m) {
      const int c = (int)(uint8_t)cp[m];
      if (c >= K) continue;
      const _Float16* row = cb + ((int64_t)m * K + c) * D;
      int i = 0;
      for (; i + 1 < D; i += 2) {
        const float p0 = (float)(_Float16)(qq[i] * row[i]);
        const float p1 = (float)(_Float16)(qq[i + 1] * row[i + 1]);
        acc = acc + (p0 + p1);
      }
      for (; i < D; ++i) acc = acc + (float)qq[i] * (float)row[i];
    }
    static_cast<uint16_t*>(out)[(int64_t)q * N + n] = f2h(acc);
  }
}

inline _Float16 f16_one() { return (_Float16)1.0f; }

}  // namespace

// Launch plan of the fast G=4 scorer, score_g4p_kernel<threads, tok, pref>.
struct G4Plan {
  int threads, tok, pref, chunk_tokens, nchunk;
};

// Launch shapes of score_g4p_kernel, largest chunk first: {threads, tokens
// per thread, stages in flight}.
static const int kG4Shapes[][3] = {{1024, 4, 1}, {512, 4, 1}, {512, 2, 1}, {256, 2, 1},
                                   {256, 1, 1}};

// LAPRUNE_SCORE_CFG overrides the choice for measurements: one of the
// shapes above as "<threads>x<tok>p<pref>".
static bool score_cfg_override(int* threads, int* tok, int* pref) {
  static const char* e = getenv("LAPRUNE_SCORE_CFG");
  if (!e || !*e) return false;
  int th = 0, tk = 0, pf = 0;
  if (sscanf(e, "%dx%dp%d", &th, &tk, &pf) != 3) return false;
  bool known = false;
  for (const auto& sh : kG4Shapes) known |= sh[0] == th && sh[1] == tk && sh[2] == pf;
  if (!known) return false;
  *threads = th;
  *tok = tk;
  *pref = pf;
  return true;
}

static int g4_plan(int R, int T, G4Plan* p) {
  DevInfo di;
  int s = device_info(&di);
  if (s != LAP_OK) return s;
  int th = 0, tk = 0, pf = 1;
  const bool forced = score_cfg_override(&th, &tk, &pf);
  if (!forced) {
    // Largest chunk that still gives every CU a workgroup; the smallest
    // shape when even that cannot.
    th = 256;
    tk = 1;
    pf = 1;
    for (const auto& sh : kG4Shapes) {
      const int ct = sh[0] * sh[1];
      if ((int64_t)R * ((T + ct - 1) / ct) >= di.cu_count) {
        th = sh[0];
        tk = sh[1];
        pf = sh[2];
        break;
      }
    }
  }
  const int ct = th * tk;
  *p = G4Plan{th, tk, pf, ct, (T + ct - 1) / ct};
  return LAP_OK;
}

// Histogram copies: with at most one workgroup per CU, 16 per group row (80
// KiB of LDS) and 8 per per-head row (97 KiB); with two workgroups per CU,
// 4 per group row (68 KiB each) and 2 per per-head row (72 KiB).  The keys
// of one launch fall in a few high-byte bins, so a wave's 64 atomics land on
// a few addresses, and the copies spread them (16 copies measured 0.2 us
// faster than 4 at C2).
template <int TH, int TK, int PF>
static void launch_g4p(dim3 grid, hipStream_t st, const uint16_t* lut, bool lut_il,
                       const uint8_t* codes, int64_t cs_b, int64_t cs_h, int64_t cs_t, int Hkv,
                       int R, int T, const ScoreOut& so, bool one_per_cu) {
#define LAP_G4P_LAUNCH(IL, PH, HC)                                                          \
  hipLaunchKernelGGL((score_g4p_kernel<TH, TK, PF, IL, PH, HC>), grid, dim3(TH), 0, st, lut,  \
                     codes, cs_b, cs_h, cs_t, Hkv, R, T, so, f16_one())
  if (lut_il) {
    if (!so.per_head && one_per_cu) LAP_G4P_LAUNCH(true, false, 16);
    else if (!so.per_head) LAP_G4P_LAUNCH(true, false, 4);
    else if (one_per_cu) LAP_G4P_LAUNCH(true, true, 8);
    else LAP_G4P_LAUNCH(true, true, 2);
  } else {
    if (so.per_head) LAP_G4P_LAUNCH(false, true, 2);
    else if (one_per_cu) LAP_G4P_LAUNCH(false, false, 16);
    else LAP_G4P_LAUNCH(false, false, 4);
  }
#undef LAP_G4P_LAUNCH
}

// Launch the fast G=4 scorer.  Exposed to the fused retrieval entry point.
int launch_score_g4(const uint16_t* lut, bool lut_il, const uint8_t* codes, int64_t cs_b,
                    int64_t cs_h, int64_t cs_t, int B, int Hkv, int T, uint16_t* heads,
                    uint16_t* keys, uint32_t* hist, int key_mode, bool per_head,
                    int cand_start, int cand_end, const int32_t* plans, int* nchunk_out,
                    hipStream_t st) {
  const int R = B * Hkv;
  G4Plan pl;
  int s = g4_plan(R, T, &pl);
  if (s != LAP_OK) return s;
  ScoreOut so{heads, keys, hist, key_mode, cand_start, cand_end, plans, per_head ? 1 : 0};
  dim3 grid((unsigned)(R * pl.nchunk));
  DevInfo di;
  s = device_info(&di);
  if (s != LAP_OK) return s;
  const bool one_per_cu = (int64_t)grid.x <= di.cu_count;
  {
    const int key = (pl.threads * 16 + pl.tok) * 16 + pl.pref;
    switch (key) {
#define LAP_G4P(TH, TK, PF)                                                               \
  case (TH * 16 + TK) * 16 + PF:                                                          \
    launch_g4p<TH, TK, PF>(grid, st, lut, lut_il, codes, cs_b, cs_h, cs_t, Hkv, R, T, so, \
                           one_per_cu);                                                      \
    break;
      LAP_G4P(1024, 4, 1) LAP_G4P(512, 4, 1) LAP_G4P(512, 2, 1) LAP_G4P(256, 2, 1)
      LAP_G4P(256, 1, 1)
#undef LAP_G4P
      default:
        set_error("score_g4: no kernel for %d threads x %d tokens (prefetch %d)", pl.threads,
                  pl.tok, pl.pref);
        return LAP_ERR_INVALID;
    }
  }
  LAP_LAUNCH_CHECK("score_g4p_kernel");
  if (nchunk_out) *nchunk_out = pl.nchunk;
  return LAP_OK;
}

// Number of workgroup chunks launch_score_g4 uses for the GMKG table with T
// tokens and R rows (the level-1 histogram count of the fused top-k).
int score_g4_nchunk(int R, int T) {
  G4Plan pl;
  if (g4_plan(R, T, &pl) != LAP_OK) return -1;
  return pl.nchunk;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool score_g4_supported(const uint8_t* codes, int64_t cs_b, int64_t cs_h, int64_t cs_t) {
  return aligned16(codes) && cs_t % 16 == 0 && cs_h % 16 == 0 && cs_b % 16 == 0;
}

}  // namespace lap

using namespace lap;

extern "C" int lap_lut_score_grouped(const void* lut, int lut_layout, const uint8_t* codes,
                                     int64_t codes_stride_h, int64_t codes_stride_t, int Hkv,
                                     int G, int T, int M, int K, void* out,
                                     lap_stream_t stream) {
  clear_error();
  LAP_CHECK(lut && codes && out, "lap_lut_score_grouped: null pointer");
  LAP_CHECK(lut_layout == LAP_LUT_HMK || lut_layout == LAP_LUT_GMKG,
            "lap_lut_score_grouped: bad lut layout");
  LAP_CHECK(G > 0 && G <= 4, "grouped kernel supports G<=4");
  LAP_CHECK(Hkv > 0 && T >= 0 && M > 0 && K > 0 && K <= 256,
            "lap_lut_score_grouped: bad sizes Hkv=%d T=%d M=%d K=%d", Hkv, T, M, K);
  LAP_CHECK(codes_stride_t >= M && codes_stride_h >= 0,
            "lap_lut_score_grouped: codes strides must cover M");
  if (T == 0) return LAP_OK;
  hipStream_t st = as_stream(stream);
  const uint16_t* L = static_cast<const uint16_t*>(lut);
  if (G == 4 && M == kM && K == kK && score_g4_supported(codes, 0, codes_stride_h, codes_stride_t)) {
    return launch_score_g4(L, lut_layout == LAP_LUT_GMKG, codes, 0, codes_stride_h,
                           codes_stride_t, 1, Hkv, T, static_cast<uint16_t*>(out), nullptr,
                           nullptr, LAP_KEY_F16, false, 0, 0, nullptr, nullptr, st);
  }
  DevInfo di;
  int s = device_info(&di);
  if (s != LAP_OK) return s;
  const size_t smem = (size_t)G * M * K * 2;
  LAP_CHECK_CODE(smem <= (size_t)di.lds_per_block, LAP_ERR_UNSUPPORTED,
                 "grouped LUT shared-memory request is too large (%zu > %d bytes)", smem,
                 di.lds_per_block);
  const int gy = std::min((T + 255) / 256, std::max(1, di.cu_count * 2 / Hkv));
  hipLaunchKernelGGL(score_grouped_generic_kernel, dim3(Hkv, gy), dim3(256), smem, st, L,
                     lut_layout, codes, codes_stride_h, codes_stride_t, G, T, M, K,
                     static_cast<uint16_t*>(out), f16_one());
  LAP_LAUNCH_CHECK("score_grouped_generic_kernel");
  return LAP_OK;
}

extern "C" int lap_lut_score_gqa(const void* lut, const uint8_t* codes, int64_t codes_stride_h,
                                 int64_t codes_stride_t, int Hkv, int G, int T, int M_stride,
                                 int K, int M_start, int M_end, const int64_t* indices, int N,
                                 void* out, lap_stream_t stream) {
  clear_error();
  LAP_CHECK(lut && codes && out, "lap_lut_score_gqa: null pointer");
  LAP_CHECK(G > 0 && Hkv > 0, "H must equal Hkv * G");
  LAP_CHECK(M_end <= M_stride && M_start >= 0 && M_end - M_start > 0,
            "lap_lut_score_gqa: bad M range [%d,%d) of %d", M_start, M_end, M_stride);
  LAP_CHECK(K > 0 && K <= 256, "lap_lut_score_gqa: K=%d out of range", K);
  LAP_CHECK(T >= 0 && N >= 0, "lap_lut_score_gqa: negative size");
  if (!indices) LAP_CHECK(N == T, "lap_lut_score_gqa: dense mode needs N == T");
  if (N == 0) return LAP_OK;
  DevInfo di;
  int s = device_info(&di);
  if (s != LAP_OK) return s;
  const int M_range = M_end - M_start;
  const size_t smem = (size_t)M_range * K * 2;
  LAP_CHECK_CODE(smem <= (size_t)di.lds_per_block, LAP_ERR_UNSUPPORTED,
                 "lap_lut_score_gqa: table of %zu bytes exceeds LDS", smem);
  const int H = Hkv * G;
  const int gy = std::min((N + 255) / 256, std::max(1, di.cu_count * 4 / H));
  hipLaunchKernelGGL(score_gqa_kernel, dim3(H, gy), dim3(256), smem, as_stream(stream),
                     static_cast<const uint16_t*>(lut), codes, codes_stride_h, codes_stride_t, G,
                     T, N, M_start, M_range, M_stride, K, indices,
                     static_cast<uint16_t*>(out), f16_one());
  LAP_LAUNCH_CHECK("score_gqa_kernel");
  return LAP_OK;
}

extern "C" int lap_lut_score_mha(const void* lut, int lut_dtype, const void* codes,
                                 int codes_dtype, int Q, int N, int M, int K, void* out,
                                 lap_stream_t stream) {
  clear_error();
  LAP_CHECK(lut && codes && out, "lap_lut_score_mha: null pointer");
  LAP_CHECK(lut_dtype == LAP_DTYPE_F16 || lut_dtype == LAP_DTYPE_F32, "lut must be fp16 or fp32");
  LAP_CHECK(codes_dtype == LAP_DTYPE_U8 || codes_dtype == LAP_DTYPE_I8 ||
                codes_dtype == LAP_DTYPE_I64,
            "codes must be int64 (Long) or uint8 (Byte) or int8 (Char)");
  LAP_CHECK(Q > 0 && M > 0 && K > 0 && N >= 0, "lap_lut_score_mha: bad sizes");
  if (N == 0) return LAP_OK;
  dim3 grid(Q, (N + 255) / 256);
  hipStream_t st = as_stream(stream);
  const bool f32 = lut_dtype == LAP_DTYPE_F32;
#define LAP_MHA(CT)                                                                          \
  do {                                                                                       \
    if (f32)                                                                                 \
      hipLaunchKernelGGL((score_mha_kernel<CT, true>), grid, dim3(256), 0, st, lut,          \
                         static_cast<const CT*>(codes), Q, N, M, K, out, f16_one());         \
    else                                                                                     \
      hipLaunchKernelGGL((score_mha_kernel<CT, false>), grid, dim3(256), 0, st, lut,         \
                         static_cast<const CT*>(codes), Q, N, M, K, out, f16_one());         \
  } while (0)
  if (codes_dtype == LAP_DTYPE_U8) LAP_MHA(uint8_t);
  else if (codes_dtype == LAP_DTYPE_I8) LAP_MHA(int8_t);
  else LAP_MHA(int64_t);
#undef LAP_MHA
  LAP_LAUNCH_CHECK("score_mha_kernel");
  return LAP_OK;
}

extern "C" int lap_aq_lut_direct(const void* q, const void* codebooks, int dtype,
                                 const void* codes, int codes_dtype, int Q, int N, int M, int K,
                                 int D, void* out, lap_stream_t stream) {
  clear_error();
  LAP_CHECK(q && codebooks && codes && out, "lap_aq_lut_direct: null pointer");
  LAP_CHECK(dtype == LAP_DTYPE_F32 || dtype == LAP_DTYPE_F16,
            "lap_aq_lut_direct: dtype must be fp32 or fp16");
  LAP_CHECK(codes_dtype == LAP_DTYPE_U8 || codes_dtype == LAP_DTYPE_I8 ||
                codes_dtype == LAP_DTYPE_I64,
            "codes must be int64 (Long) or uint8 (Byte) or int8 (Char)");
  LAP_CHECK(Q > 0 && M > 0 && K > 0 && D > 0 && N >= 0, "lap_aq_lut_direct: bad sizes");
  if (N == 0) return LAP_OK;
  dim3 grid(Q, (N + 255) / 256);
  hipStream_t st = as_stream(stream);
  const bool f32 = dtype == LAP_DTYPE_F32;
#define LAP_DIRECT(CT)                                                                       \
  do {                                                                                       \
    if (f32)                                                                                 \
      hipLaunchKernelGGL((aq_direct_kernel<CT, true>), grid, dim3(256), 0, st, q, codebooks, \
                         static_cast<const CT*>(codes), Q, N, M, K, D, out);                 \
    else                                                                                     \
      hipLaunchKernelGGL((aq_direct_kernel<CT, false>), grid, dim3(256), 0, st, q,           \
                         codebooks, static_cast<const CT*>(codes), Q, N, M, K, D, out);      \
  } while (0)
  if (codes_dtype == LAP_DTYPE_U8) LAP_DIRECT(uint8_t);
  else if (codes_dtype == LAP_DTYPE_I8) LAP_DIRECT(int8_t);
  else LAP_DIRECT(int64_t);
#undef LAP_DIRECT
  LAP_LAUNCH_CHECK("aq_direct_kernel");
  return LAP_OK;
}

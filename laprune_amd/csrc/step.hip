// step.hip — the fused decode step: A2 scoring, A3 selection and A5
// attention, with the split merge, in one launch.
//
// Replaces, for one layer and one decode token, the chain of the reference's
// _decode_attention (laprune/llm/modifiers/aq_evaluation.py:146-253):
// grouped LUT scoring (aq_kv.py:684 -> aq_lut_gqa.cu:460-534), the candidate
// window and torch.topk (aq_evaluation.py:185-205), the keep set (:210-237)
// and SDPA over the kept rows (:251).  The LUT itself is built by the
// launch before (lut.hip), which is the only other kernel of the step.
//
// Work shape.  Selection is per KV group (the group max of its four query
// heads' scores).  Each KV row r (batch row b, KV head h) is served by WR
// workgroups of 1024 threads, all on the same XCD: the hardware deals a
// launch's workgroups to the XCDs round-robin by block id (block i runs on
// XCD (i + s) % nxcc, where the start s can differ from launch to launch),
// and the blocks of row r are the ones with i % nxcc == r % nxcc.  The last
// workgroup of each row checks, from the XCC_ID registers its row's
// workgroups recorded, that they did share one XCD, and counts any row that
// did not in the status word.  The workgroups of a row share one L2, and the data they pass
// each other (histograms, level-2 tables, attention partials) never leaves it:
// a producer's plain stores are complete in L2 once its vmcnt drains, and a
// consumer reads them with device-scope loads, which miss the L1 (where a
// stale copy could sit) and hit the shared L2.  No cache write-back or
// invalidate is needed, which is what makes the two in-kernel barriers cost
// well under a kernel boundary.
//
// Phases of the workgroup owning chunk c of row r (TOK * 1024 tokens):
//   S  score its tokens (the scorer's pipeline, score_core.h): selection keys
//      stay in registers, and the level-1 histogram of the keys' top ten
//      bits over the candidate window is added to the row's histogram (L2
//      atomics);
//   B1 row barrier;
//   H  the row's threshold bin b1 and the count above it; the chunk
//      publishes its own count above b1 and the level-2 histogram (low six
//      bits) of its keys in b1;
//   B2 row barrier;
//   H2 the row's level-2 tables give the threshold tau, the ties at tau to
//      take (lowest columns first) and where this chunk's selection starts;
//      the chunk compacts its own selection in column order, writes those
//      indices and keeps them in LDS;
//   A  attention of the group's four query heads over its selection and its
//      share of the sink and local tail (the MFMA wave step of attn_core.h),
//      one (m, l, o) partial per head;
//   E  the last workgroup of the row to arrive merges the partials and
//      writes the output.
// Selection results equal the two-level top-k of topk.hip bit for bit: the
// same keys, threshold and tie rule (the radix split is 10 + 6 bits here,
// 8 + 8 there).
//
// Barriers spin a bounded number of polls; a spin that gives up counts a
// time-out in the status word and lets the kernel finish (results of that
// call are then undefined, and the caller must re-zero the workspace).
#include "common.h"
#include "attn_core.h"
#include "score_core.h"
#include "topk_core.h"

#include <algorithm>
#include <cstdlib>
#include <mutex>

namespace lap {

bool score_g4_supported(const uint8_t* codes, int64_t cs_b, int64_t cs_h, int64_t cs_t);

namespace {

constexpr int kTH = 1024;
constexpr int kWaves = kTH / 64;
constexpr int kMaxTok = 16;         // tokens per thread (chunk = TOK * 1024)
constexpr int kMaxTokPH = 8;        // the same with per-head selection
constexpr int kHC = 16;             // level-1 histogram copies (group selection)
constexpr int kHCph = 4;            // the same per query head (per-head selection)
constexpr int kDh = 128;            // head dim of the fused path
constexpr int kKeepMax = 8192;      // a workgroup's own selection (32 KiB of LDS)
constexpr int kSpin = 1 << 21;      // polls before a barrier gives up
constexpr int kBarWords = 16;       // one 64-byte line per barrier
constexpr int kStatusBytes = 256;
constexpr int kMaxWR = 32;          // workgroups per row (one per CU of an XCD)
// Rows the persistent head of a workspace (status words, row barriers, row
// histograms) is laid out for, whatever the call's B * Hkv: a caller may size
// one workspace for its largest batch and call with any smaller one, and
// every call finds row r's persistent words at the same address.  The fused
// kernel serves at most one row per CU (R <= 256 on MI355X).
constexpr int kHeadRows = 256;

struct StepArgs {
  const uint16_t* lut;   // [R][M][K][4] fp16 (GMKG)
  const uint8_t* codes;
  int64_t cs_b, cs_h, cs_t;
  int B, Hkv, T;         // T: code columns the grid covers
  const int32_t* plans;  // lap_row_plan[B] or null (then the scalars below)
  int cand_start, cand_end, k, sink, tail_start, tail_count;
  int k_cols;            // index row stride; rows pad [k, k_cols) with -1
  int max_sink, max_tail;
  int key_bf16;
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
  int T_kv;              // K/V rows available
  float scale_log2;
  void* idx;
  int idx_i64;
  uint16_t* out;         // [B][Hkv * 4][128]
  uint32_t* status;      // [0] rows spread over XCDs, [1] barrier time-outs
  uint32_t* bar;         // [R][3][kBarWords]
  uint32_t* hist;        // [R][4][1024] level-1 counts of the row's selection rows
                         // (row r only, or its 4 heads with per-head selection;
                         // zero between calls)
  uint32_t* t2;          // [R][WR][4][kT2] per chunk and selection row: level-2
                         // counts, keys above b1
  float* part;           // [R][WR][4][kDh + 2] (m, l, o)
  int nxcc, RX, WR;
  _Float16 one;
};

// One row's windows: the call's scalars, or its sequence's plan clamped to
// the grid (as the scorer, top-k and attention kernels clamp them).
struct StepRow {
  int t_end, cs, ce, k, sink, tail_start, tail_count, t_total;
};
__device__ __forceinline__ StepRow step_row(const StepArgs& a, int b) {
  if (!a.plans)
    return StepRow{a.T, a.cand_start, a.cand_end, a.k, a.sink, a.tail_start, a.tail_count,
                   a.T_kv};
  const int32_t* p = a.plans + (int64_t)b * kPlanInts;
  const int te = min(max(p[0], 0), a.T);
  const int c0 = min(max(p[2], 0), te), c1 = min(max(p[3], c0), te);
  return StepRow{te,
                 c0,
                 c1,
                 max(0, min(min(p[4], c1 - c0), a.k_cols)),
                 min(max(p[5], 0), a.max_sink),
                 p[6],
                 min(max(p[7], 0), a.max_tail),
                 min(p[1], a.T_kv)};
}

__device__ __forceinline__ unsigned xcc_id() {
  return __builtin_amdgcn_s_getreg((20) | (0 << 6) | (15 << 11));  // HW_REG_XCC_ID[15:0]
}

// Device-scope loads of what other workgroups of the row wrote (they miss
// the L1 and are served by the XCD's L2).
template <typename T>
__device__ __forceinline__ T ld_dev(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint2 ld_dev2(const uint2* p) {
  const uint64_t v = ld_dev(reinterpret_cast<const uint64_t*>(p));
  return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
}

// Arrival on a row counter: blk holds a 64-bit count that only grows and
// that every call advances by exactly kMaxWR (the call's n <= kMaxWR
// arrivals, then kMaxWR - n added by the last), so calls with different n
// can share it and nothing is reset.  Returns the count that ends this call
// and whether this arrival was the call's last.
__device__ __forceinline__ uint64_t row_arrive(uint32_t* blk, int n, bool* last) {
  uint64_t* cnt = reinterpret_cast<uint64_t*>(blk);
  const uint64_t old = __hip_atomic_fetch_add(cnt, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t pos = old % (uint64_t)kMaxWR;
  *last = pos == (uint64_t)n - 1;
  if (*last && n < kMaxWR)
    __hip_atomic_fetch_add(cnt, (uint64_t)(kMaxWR - n), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return old - pos + (uint64_t)kMaxWR;
}

// Barrier of the n workgroups of one row, run by one thread of each after
// its workgroup's stores have drained: arrive, then poll the count (one
// device-scope atomic and polls of the same line; no second word for the
// last arrival to publish).
__device__ void row_barrier(uint32_t* blk, int n, uint32_t* status) {
  bool last;
  const uint64_t target = row_arrive(blk, n, &last);
  if (last) return;
  const uint64_t* cnt = reinterpret_cast<const uint64_t*>(blk);
  for (int s = 0; s < kSpin; ++s) {
    if (ld_dev(cnt) >= target) return;
    __builtin_amdgcn_s_sleep(1);
  }
  __hip_atomic_fetch_add(status + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// All of the workgroup's global stores complete, then one barrier arrival.
__device__ __forceinline__ void wg_row_barrier(const StepArgs& a, int r, int which) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) row_barrier(a.bar + ((int64_t)r * 3 + which) * kBarWords, a.WR, a.status);
  __syncthreads();
}

// Record the XCD this workgroup runs on in its row's mask (word 2 of the
// merge counter's line), which the row's last merge arrival checks.
__device__ __forceinline__ void record_xcd(const StepArgs& a, int r) {
  __hip_atomic_fetch_or(a.bar + ((int64_t)r * 3 + 2) * kBarWords + 2, 1u << (xcc_id() & 31u),
                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t key_of_score(float e, int key_bf16) {
  const uint16_t h = f2h(e);
  return key_bf16 ? bf16_key_of_f16(h) : f16_key(h);
}

template <typename IT>
__device__ __forceinline__ void put_idx(void* idx, int64_t i, int v) {
  static_cast<IT*>(idx)[i] = (IT)v;
}

// Radix split of the 16-bit selection keys: level 1 on bits 15..6 (1024
// bins, one per thread of the workgroup), level 2 on bits 5..0, so the
// level-2 table every chunk publishes is 64 counts and reading all of a
// row's tables after B2 is a few loads per thread.
constexpr int kL1 = 1024, kLoBits = 6, kL2 = 1 << kLoBits;
constexpr int kH1Pitch = kL1 + 1;  // copies of one bin in different banks
constexpr int kT2 = kL2 + 4;       // per-chunk table: level-2 counts, keys above b1
constexpr uint32_t kNoKey = 0xffffffffu;  // a thread's token outside the window

// Inclusive prefix sum within each row of 16 lanes (DPP row shifts); the
// rows must be whole (all 16 lanes active).
__device__ __forceinline__ uint32_t row16_inclusive_scan(uint32_t x) {
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, true);  // row_shr:1
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, true);  // row_shr:2
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, true);  // row_shr:4
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, true);  // row_shr:8
  return x;
}

// x of lane (i + N) mod 16 in lane i's 16-lane row (DPP row_ror:N, every
// lane active).
template <int N>
__device__ __forceinline__ float row_ror(float x) {
  static_assert(N >= 1 && N <= 15, "row_ror:1..15");
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + N, 0xf, 0xf, false));
}

// The sum of x over the wave's 64 lanes (every lane active), in every lane:
// a DPP scan read at lane 63 (no LDS permutes).
__device__ __forceinline__ uint32_t wave_sum(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_readlane((int)wave_inclusive_scan(x), 63);
}

// w[0] + ... + w[wave - 1] of kWaves words in LDS, in every lane of the
// wave (every lane active).
__device__ __forceinline__ uint32_t waves_before(const uint32_t* w, int wave, int lane) {
  const int l = lane & (kWaves - 1);
  const uint32_t v = l < wave ? w[l] : 0u;
  return (uint32_t)__builtin_amdgcn_readlane((int)row16_inclusive_scan(v), kWaves - 1);
}

// The unique bin b of h[0..1023] with S(b) >= target > S(b+1), S(i) =
// sum_{j >= i} h[j]: s_res = {b, S(b+1)}.  1024 threads, thread tid holding
// x = h[1023 - tid]; 1 <= target <= S(0).
__device__ __forceinline__ void select_bin1024(uint32_t x, uint32_t target, uint32_t* s_wsum,
                                               uint32_t* s_res) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t inc = wave_inclusive_scan(x);
  if (lane == 63) s_wsum[wave] = inc;
  __syncthreads();
  const uint32_t above = waves_before(s_wsum, wave, lane) + inc - x;
  if (above + x >= target && above < target) {
    s_res[0] = kL1 - 1 - tid;
    s_res[1] = above;
  }
  __syncthreads();
}
// Per-wave counts of TOK-stage token lists to positions: s_wcnt[l][w] holds
// list l's count in wave w; afterwards it holds the exclusive prefix over
// the waves, and s_ltot[l] the list's total.  One 16-lane row per list.
template <int LISTS>
__device__ __forceinline__ void scan_wave_counts(uint32_t* s_wcnt, uint32_t* s_ltot) {
  static_assert(kWaves == 16, "one 16-lane row per list");
  const int tid = threadIdx.x;
  __syncthreads();
  if (tid < LISTS * kWaves) {
    const uint32_t xw = s_wcnt[tid];
    const uint32_t inc = row16_inclusive_scan(xw);
    s_wcnt[tid] = inc - xw;
    if ((tid & (kWaves - 1)) == kWaves - 1) s_ltot[tid / kWaves] = inc;
  }
  __syncthreads();
}

// LDS carve of the 64 KiB region that holds the table during S.
struct Lds {
  uint4* lut;                // S: [kLutBytes / 16]
  int* keep;                 // H2, A: [kKeepMax]
  float* o;                  // A: [kWaves][4][kDh]
};

// The row a workgroup serves (KV row r, its chunk c of the row's TOK * 1024
// columns), or false when the grid has no row for it.
struct StepPos {
  int r, c, b, hkv, h0, t0, t1;
  StepRow pr;
};
template <int TOK>
__device__ __forceinline__ bool step_pos(const StepArgs& a, StepPos* p) {
  const int nx = a.nxcc;
  const int x = blockIdx.x % nx, slot = blockIdx.x / nx;
  const int rs = slot / a.WR, c = slot - rs * a.WR;
  const int r = rs * nx + x;
  if (rs >= a.RX || r >= a.B * a.Hkv) return false;
  p->r = r;
  p->c = c;
  p->b = r / a.Hkv;
  p->hkv = r - p->b * a.Hkv;
  p->h0 = p->hkv * kG;
  p->pr = step_row(a, p->b);
  p->t0 = c * TOK * kTH;
  p->t1 = min(p->pr.t_end, p->t0 + TOK * kTH);
  return true;
}

// The query fragments of the attention phase (A-operand layout of
// attn_core.h), requested at the start so that their latency hides behind S.
__device__ __forceinline__ void load_q_frags(const StepArgs& a, int b, int h0, int lane,
                                             i16x4 (&qpre)[kDh / 16]) {
  const int rq = lane >> 4, cq = lane & 15;
  const uint16_t* qp =
      a.q + (int64_t)b * a.q_sb + (int64_t)(h0 + (cq < kG ? cq : 0)) * a.q_sh + rq * (kDh / 4);
#pragma unroll
  for (int ks = 0; ks < kDh / 16; ++ks) {
    const uint2 w = *reinterpret_cast<const uint2*>(qp + 4 * ks);  // 8-byte aligned (host check)
    qpre[ks] = cq < kG ? __builtin_bit_cast(i16x4, w) : i16x4{0, 0, 0, 0};
  }
}

// S: the row's table into LDS, then TOK stages of 1024 tokens scored with one
// stage's code rows in flight ahead (the scorer's pipeline, score_core.h);
// body(j, t, e0, e1, e2, e3) gets stage j's token t and its four head scores.
// Tokens past the chunk end load its last row (in bounds); the body sees
// their column t >= t1.
template <int TOK, typename Body>
__device__ __forceinline__ void score_chunk(const StepArgs& a, const StepPos& p,
                                            uint4* __restrict__ lut_lds, Body&& body) {
  const int tid = threadIdx.x;
  constexpr int kFill = kLutBytes / 16 / kTH;
  const uint4* src = reinterpret_cast<const uint4*>(a.lut + (int64_t)p.r * (kG * kM * kK));
  u32x4 f[kFill];
#pragma unroll
  for (int i = 0; i < kFill; ++i) f[i] = gload16_ordered(src + i * kTH + tid);
  const uint8_t* crow = a.codes + (int64_t)p.b * a.cs_b + (int64_t)p.hkv * a.cs_h;
  u32x4 cc[TOK][2];
  auto request = [&](int j) {
    const int t = min(p.t0 + j * kTH + tid, p.t1 - 1);
    const uint8_t* q = crow + (int64_t)t * a.cs_t;
    cc[j][0] = gload16_stream(q);
    cc[j][1] = gload16_stream(q + 16);
  };
#pragma unroll
  for (int i = 0; i < kFill; ++i) {
    vm_wait(kFill - 1 - i, f[i]);
    lut_lds[i * kTH + tid] = as_uint4(f[i]);
  }
  request(0);  // after the table, as in the scorer (score.hip)
  lds_barrier();
  const char* tab = reinterpret_cast<const char*>(lut_lds);
#pragma unroll
  for (int j = 0; j < TOK; ++j) {
    vm_wait(0, cc[j][0], cc[j][1]);
    if (j + 1 < TOK) request(j + 1);
    stage_prio(j, TOK);
    float e0 = 0.f, e1 = 0.f, e2 = 0.f, e3 = 0.f;
    score_token(tab, as_uint4(cc[j][0]), as_uint4(cc[j][1]), a.one, e0, e1, e2, e3);
    body(j, p.t0 + j * kTH + tid, e0, e1, e2, e3);
  }
  __builtin_amdgcn_s_setprio(0);
}

// The end of a row's step, shared by both fused kernels: the waves' (m, l,
// o) combined in LDS into the workgroup's partial, then the row's last
// workgroup to arrive merges the partials (E) and writes the output.  Waves
// nw.. ran no attention step (their state is empty) and are left out.
// out_stores(last) issues the stores nothing in the launch reads (index rows
// and the like); every workgroup calls it once, after its merge arrival (the
// merging workgroup: with EARLY, as soon as its partial loads are out), and
// `last` is true for the row's last arrival (or its only workgroup), which
// clears the row histogram: every workgroup of the row has added to it and
// read it before arriving, so the clear follows them all even when a barrier
// of the call timed out.
template <int DT, bool EARLY, typename Stores>
__device__ __forceinline__ void finish_row(const StepArgs& a, WaveState<DT, kG, kDh>& ws,
                                           const Lds& lds, float (&s_m)[kWaves][4],
                                           float (&s_l)[kWaves][4], uint32_t& s_flag, int r,
                                           int c, int b, int h0, bool select, int nw,
                                           Stores&& out_stores) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  lds_barrier();  // every wave's attention is done; lds.o (after the keep list) is free
  if (wave < nw) {
    const int rq = lane >> 4, cq = lane & 15;
    if (lane < kG) {
      s_m[wave][lane] = ws.m;
      s_l[wave][lane] = ws.l;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int g = 4 * rq + e;
      if (g < kG)
#pragma unroll
        for (int ch = 0; ch < kDh / 16; ++ch)
          lds.o[(wave * kG + g) * kDh + cq * (kDh / 16) + ch] = ws.acc[ch][e];
    }
  }
  lds_barrier();
  float* mypart = a.part + ((int64_t)r * a.WR + c) * kG * (kDh + 2);
  if (tid < kG * kDh) {
    const int g = tid / kDh, d = tid - g * kDh;
    float M = -INFINITY, l = 0.f, o = 0.f;
    auto add = [&](int w) {
      const float wt = (M == -INFINITY || s_m[w][g] == -INFINITY) ? 0.f : exp2f(s_m[w][g] - M);
      l += s_l[w][g] * wt;
      o += lds.o[(w * kG + g) * kDh + d] * wt;
    };
    if (nw == kWaves) {  // every wave attended: unrolled, the LDS reads batched
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][g]);
#pragma unroll
      for (int w = 0; w < kWaves; ++w) add(w);
    } else {
      for (int w = 0; w < nw; ++w) M = fmaxf(M, s_m[w][g]);
      for (int w = 0; w < nw; ++w) add(w);
    }
    if (a.WR == 1) {
      a.out[((int64_t)b * a.Hkv * kG + h0 + g) * kDh + d] = st16<DT>(l > 0.f ? o / l : 0.f);
    } else {
      float* pp = mypart + g * (kDh + 2);
      if (d == 0) {
        pp[0] = M;
        pp[1] = l;
      }
      pp[2 + d] = o;
    }
  }
  if (a.WR == 1) {
    out_stores(true);
    return;
  }

  // ---------------------------------------------------------------- E
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    // blk[0..1]: the row counter of row_arrive; blk[2] collects the XCDs
    // the row ran on, which the last arrival checks and clears
    uint32_t* blk = a.bar + ((int64_t)r * 3 + 2) * kBarWords;
    if (!select) {  // rows that select recorded it before B1
      record_xcd(a, r);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // recorded before arriving
    }
    bool last;
    row_arrive(blk, a.WR, &last);
    if (last) {
      const uint32_t seen = ld_dev(blk + 2);
      if (__popc(seen) > 1)
        __hip_atomic_fetch_add(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(blk + 2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    s_flag = last ? 1u : 0u;
  }
  __syncthreads();
  if (!s_flag) {
    out_stores(false);
    return;
  }
  // The row's partials: thread t < 128 holds (m, l) of split t / 4, head
  // t % 4 (waves 0 and 1); per head, the max M over the splits and the sum
  // of l * 2^(m - M) are reduced over the lanes of one head and then over
  // the two waves.  o is summed over the splits by two threads per output
  // (each with its splits' loads all in flight).
  static_assert(kMaxWR * kG == 128, "waves 0 and 1 hold the (split, head) records");
  const float* rp = a.part + (int64_t)r * a.WR * kG * (kDh + 2);
  float* sw = lds.o;                  // [kMaxWR * 4] weights (0 past WR)
  float* so = sw + kMaxWR * kG;       // [kTH] half sums of o
  float* sx = so + kTH;               // [2][4] per-wave max of m
  float* slw = sx + 2 * kG;           // [2][4] per-wave sum of l * weight
  // o's loads go out with (m, l)'s, so the merge waits for one round trip
  constexpr int kHalf = kMaxWR / 2;
  const int half = tid / (kG * kDh), e = tid % (kG * kDh);
  const int g_o = e / kDh, d_o = e - g_o * kDh;
  float v[kHalf];
#pragma unroll
  for (int u = 0; u < kHalf; ++u) {
    const int s2 = min(half * kHalf + u, a.WR - 1);
    v[u] = ld_dev(rp + ((int64_t)s2 * kG + g_o) * (kDh + 2) + 2 + d_o);
  }
  // EARLY: this workgroup's own output stores go out behind the loads, so
  // that their acknowledgements overlap the merge instead of following it
  // (a kernel that stores little here; per-head selection clears four
  // histograms, whose stores would hold up the merge's waits instead)
  if (EARLY) out_stores(true);
  float mt = -INFINITY, lt = 0.f;
  if (tid < kMaxWR * kG) {
    // (m, l) as one 8-byte load (a partial's head record starts 8-byte
    // aligned): two loads would each be waited for in turn
    const bool in = tid < a.WR * kG;
    const int sg = min(tid, a.WR * kG - 1);
    const uint2 ml = ld_dev2(reinterpret_cast<const uint2*>(rp + (int64_t)sg * (kDh + 2)));
    mt = in ? __uint_as_float(ml.x) : -INFINITY;
    lt = in ? __uint_as_float(ml.y) : 0.f;
    // lanes that share the head lane % 4: rotations by 4 and 8 inside each
    // 16-lane row (DPP), then across rows
    float mx = fmaxf(mt, row_ror<4>(mt));
    mx = fmaxf(mx, row_ror<8>(mx));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (lane < kG) sx[wave * kG + lane] = mx;
  }
  __syncthreads();
  if (tid < kMaxWR * kG) {
    const int g = tid % kG;
    const float M = fmaxf(sx[g], sx[kG + g]);
    const float wt = (mt == -INFINITY || M == -INFINITY) ? 0.f : exp2f(mt - M);
    sw[tid] = wt;
    float lw = lt * wt;
    lw += row_ror<4>(lw);
    lw += row_ror<8>(lw);
    lw += __shfl_xor(lw, 16, 64);
    lw += __shfl_xor(lw, 32, 64);
    if (lane < kG) slw[wave * kG + lane] = lw;
  }
  __syncthreads();
  {
    float o = 0.f;
#pragma unroll
    for (int u = 0; u < kHalf; ++u)
      o = __builtin_fmaf(v[u], sw[(half * kHalf + u) * kG + g_o], o);
    so[tid] = o;
  }
  __syncthreads();
  if (tid < kG * kDh) {
    const int g = tid / kDh, d = tid - g * kDh;
    const float o = so[tid] + so[tid + kG * kDh];
    const float l = slw[g] + slw[kG + g];
    a.out[((int64_t)b * a.Hkv * kG + h0 + g) * kDh + d] = st16<DT>(l > 0.f ? o / l : 0.f);
  }
  if (!EARLY) out_stores(true);
}

template <int DT, int TOK>
__global__ __launch_bounds__(kTH) void step_fused_kernel(StepArgs a) {
  static_assert(TOK >= 1 && TOK <= kMaxTok, "TOK");
  static_assert(kKeepMax * 4 + kWaves * 4 * kDh * 4 <= kLutBytes, "LDS carve");
  static_assert(kMaxWR * 4 + kTH + 4 * kG <= kWaves * 4 * kDh && kG * kDh * 2 == kTH, "E carve");
  __shared__ __attribute__((aligned(16))) uint4 s_big[kLutBytes / 16];
  __shared__ uint32_t s_hist[kHC * kH1Pitch];
  __shared__ uint32_t s_h2[kL2], s_wsum[kWaves], s_res[4], s_gtw[kWaves];
  __shared__ uint32_t s_wcnt[kMaxTok * kWaves], s_ltot[kMaxTok];
  __shared__ uint32_t s_flag;
  __shared__ float s_m[kWaves][4], s_l[kWaves][4];

  Lds lds;
  lds.lut = s_big;
  lds.keep = reinterpret_cast<int*>(s_big);
  lds.o = reinterpret_cast<float*>(s_big) + kKeepMax;

  StepPos ps;
  if (!step_pos<TOK>(a, &ps)) return;  // no row here
  const int r = ps.r, c = ps.c, b = ps.b, hkv = ps.hkv, h0 = ps.h0, t0 = ps.t0, t1 = ps.t1;
  const StepRow pr = ps.pr;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool select = pr.k > 0;
  i16x4 qpre[kDh / 16];
  load_q_frags(a, b, h0, lane, qpre);

  // ---------------------------------------------------------------- S
  uint32_t kv[TOK];
#pragma unroll
  for (int j = 0; j < TOK; ++j) kv[j] = kNoKey;
  for (int i = tid; i < kHC * kH1Pitch; i += kTH) s_hist[i] = 0;
  if (select && t0 < t1) {
    const int copy = (int)(__lane_id() % kHC) * kH1Pitch;
    score_chunk<TOK>(a, ps, lds.lut, [&](int j, int t, float e0, float e1, float e2, float e3) {
      if (t < t1 && t >= pr.cs && t < pr.ce) {
        const uint32_t key = key_of_score(fmaxf(fmaxf(e0, e1), fmaxf(e2, e3)), a.key_bf16);
        kv[j] = key;
        atomicAdd(&s_hist[copy + (key >> kLoBits)], 1u);
      }
    });
  }
  __syncthreads();
  // The query fragments are waited for here, where nothing else is in
  // flight: left to the compiler, their first use in A waits for every
  // global operation issued before it.
#pragma unroll
  for (int ks = 0; ks < kDh / 16; ++ks) asm volatile("" : "+v"(qpre[ks]));
  // This chunk's level-1 count of bin tid (the sum of the copies), added to
  // the row's histogram.
  uint32_t h1 = 0;
  if (select) {
#pragma unroll
    for (int cp = 0; cp < kHC; ++cp) h1 += s_hist[cp * kH1Pitch + tid];
    if (h1)
      __hip_atomic_fetch_add(a.hist + (int64_t)r * kL1 + tid, h1, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---------------------------------------------------------------- B1, H
  // After B1 the row's level-1 histogram is whole: the threshold bin b1 and
  // the keys above it.  Each chunk then publishes, for its own keys, the
  // count above b1 and the level-2 histogram of its keys in b1.
  uint32_t tau = 0, take = 0, base = 0, n_sel = 0;
  if (select) {
    if (tid == 0) record_xcd(a, r);  // complete before B2's arrival
    wg_row_barrier(a, r, 0);
    const uint32_t hx = ld_dev(a.hist + (int64_t)r * kL1 + kL1 - 1 - tid);
    if (tid < kL2) s_h2[tid] = 0;  // ordered before H's adds by the selection's barriers
    select_bin1024(hx, (uint32_t)pr.k, s_wsum, s_res);
    const uint32_t b1 = s_res[0], gt1 = s_res[1];
#pragma unroll
    for (int j = 0; j < TOK; ++j)
      if (kv[j] != kNoKey && (kv[j] >> kLoBits) == b1) atomicAdd(&s_h2[kv[j] & (kL2 - 1)], 1u);
    const uint32_t gt = wave_sum((uint32_t)tid > b1 ? h1 : 0u);
    if (lane == 0) s_gtw[wave] = gt;
    __syncthreads();
    uint32_t* t2 = a.t2 + ((int64_t)r * a.WR + c) * kT2;
    if (tid < kL2) t2[tid] = s_h2[tid];
    if (tid == kL2) {
      uint32_t my_gt1 = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) my_gt1 += s_gtw[w];
      t2[kL2] = my_gt1;
    }
    wg_row_barrier(a, r, 1);
    // Every chunk has read the row histogram; the row's last merge arrival
    // clears it for the next call (out_stores).

    // ------------------------------------------------------------ H2
    // The row's level-2 tables: the threshold tau = (b1, b2), the ties at
    // tau to take, and where this chunk's selection starts in the row's.
    // Wave 0 alone: lane l holds bin 63 - l of every chunk's table (chunks
    // past WR read as zero) and, for l < WR, chunk l's count above b1.  The
    // row's level-2 histogram, its suffix sums and the per-chunk sums are
    // then register sums, one scan and two reductions, published with one
    // barrier.
    if (wave == 0) {
      const uint32_t k2 = (uint32_t)pr.k - gt1;  // keys to take from bin b1, >= 1
      const uint32_t* t2r = a.t2 + (int64_t)r * a.WR * kT2;
      const int bn = kL2 - 1 - lane;
      uint32_t vt[kMaxWR];
#pragma unroll
      for (int c2 = 0; c2 < kMaxWR; ++c2) vt[c2] = ld_dev(t2r + min(c2, a.WR - 1) * kT2 + bn);
      const uint32_t gt_l = ld_dev(t2r + min(lane, a.WR - 1) * kT2 + kL2);
      uint32_t tot = 0, before = 0, mine = 0;  // bin bn: the row's, chunks < c, chunk c
#pragma unroll
      for (int c2 = 0; c2 < kMaxWR; ++c2) {
        const uint32_t x = c2 < a.WR ? vt[c2] : 0u;
        tot += x;
        before += c2 < c ? x : 0u;
        mine += c2 == c ? x : 0u;
      }
      // S(bn) = keys in b1 with low bits >= bn; b2 = the bin with
      // S(b2) >= k2 > S(b2 + 1), lane L = 63 - b2
      const uint32_t inc = wave_inclusive_scan(tot);
      const uint64_t hit = __ballot(inc >= k2 && inc - tot < k2);
      const int L = hit ? __builtin_ctzll(hit) : kL2 - 1;
      const uint32_t need = k2 - (uint32_t)__builtin_amdgcn_readlane((int)(inc - tot), L);
      const uint32_t ts = (uint32_t)__builtin_amdgcn_readlane((int)before, L);  // ties before c
      const uint32_t my_ties = (uint32_t)__builtin_amdgcn_readlane((int)mine, L);
      // keys above tau (above b1, or in b1 with low bits above b2: lanes
      // below L) in the chunks before c, and in chunk c
      const uint32_t gs = wave_sum((lane < L ? before : 0u) + (lane < c ? gt_l : 0u));
      const uint32_t mg = wave_sum((lane < L ? mine : 0u) + (lane == c ? gt_l : 0u));
      if (lane == 0) {
        const uint32_t tk = ts >= need ? 0u : min(my_ties, need - ts);
        // ties taken by the earlier chunks, min(need, ts), from an explicit
        // instruction: hipcc 7.2 at -O3 folds this min (written as min() or
        // as a select) to ts here, which is wrong once the row's ties run out
        uint32_t taken_before;
        asm volatile("v_min_u32 %0, %1, %2" : "=v"(taken_before) : "v"(need), "v"(ts));
        s_res[0] = (uint32_t)(kL2 - 1 - L);
        s_res[1] = my_ties;
        s_res[2] = tk;
        s_res[3] = gs + taken_before;
        s_flag = mg + tk;
      }
    }
    __syncthreads();
    tau = (b1 << kLoBits) | s_res[0];
    take = s_res[2];
    base = s_res[3];
    n_sel = s_flag;
    const uint32_t my_ties = s_res[1];

    // Ordered compaction of this chunk's selection (column order: stage j,
    // then thread): keys above tau, and its first `take` ties at tau.  Only
    // the chunk where the row's ties run out takes some of its ties and
    // needs their ranks.
    bool sel[TOK];
    if (take == 0 || take >= my_ties) {
      const bool all_ties = take > 0;
#pragma unroll
      for (int j = 0; j < TOK; ++j)
        sel[j] = (kv[j] != kNoKey) & ((kv[j] > tau) | (all_ties & (kv[j] == tau)));
    } else {
#pragma unroll
      for (int j = 0; j < TOK; ++j) {
        const uint64_t mt = __ballot((kv[j] != kNoKey) & (kv[j] == tau));
        if (lane == 0) s_wcnt[j * kWaves + wave] = (uint32_t)__popcll(mt);
      }
      scan_wave_counts<TOK>(s_wcnt, s_ltot);
      uint32_t tie_base = 0;
#pragma unroll
      for (int j = 0; j < TOK; ++j) {
        const uint64_t mt = __ballot((kv[j] != kNoKey) & (kv[j] == tau));
        const uint32_t rank = tie_base + s_wcnt[j * kWaves + wave] + lanes_below(mt);
        sel[j] = (kv[j] != kNoKey) & ((kv[j] > tau) | ((kv[j] == tau) & (rank < take)));
        tie_base += s_ltot[j];
      }
      __syncthreads();  // the tie prefixes are read
    }
#pragma unroll
    for (int j = 0; j < TOK; ++j) {
      const uint64_t ms = __ballot(sel[j]);
      if (lane == 0) s_wcnt[j * kWaves + wave] = (uint32_t)__popcll(ms);
    }
    scan_wave_counts<TOK>(s_wcnt, s_ltot);
    uint32_t sel_base = 0;
#pragma unroll
    for (int j = 0; j < TOK; ++j) {
      const uint64_t ms = __ballot(sel[j]);
      const uint32_t q = sel_base + s_wcnt[j * kWaves + wave] + lanes_below(ms);
      if (sel[j] && q < (uint32_t)kKeepMax && base + q < (uint32_t)pr.k)
        lds.keep[q] = t0 + j * kTH + tid;
      sel_base += s_ltot[j];
    }
    n_sel = min(n_sel, (uint32_t)kKeepMax);
  }
  lds_barrier();  // the keep list

  // The stores nothing in this launch reads: this chunk's part of the index
  // row (from the keep list, which stays in LDS to the end), its share of a
  // ragged row's -1 padding, and (last arrival) the clearing of the row
  // histogram.  They are issued after the merge arrival, so that no wait on
  // the way there (every wait drains all earlier memory operations) includes
  // them.
  auto out_stores = [&](bool last) {
    const int64_t irow = ((int64_t)b * a.Hkv + hkv) * a.k_cols;
    for (int p = tid; p < (int)n_sel && base + (uint32_t)p < (uint32_t)pr.k; p += kTH) {
      if (a.idx_i64) put_idx<int64_t>(a.idx, irow + base + p, lds.keep[p]);
      else put_idx<int32_t>(a.idx, irow + base + p, lds.keep[p]);
    }
    if (a.plans) {  // ragged rows: pad [k, k_cols) with -1, split over the row's workgroups
      const int pad = a.k_cols - pr.k;
      const int ps = (pad + a.WR - 1) / a.WR;
      for (int i = c * ps + tid; i < min(pad, (c + 1) * ps); i += kTH) {
        if (a.idx_i64) put_idx<int64_t>(a.idx, irow + pr.k + i, -1);
        else put_idx<int32_t>(a.idx, irow + pr.k + i, -1);
      }
    }
    if (select && last) a.hist[(int64_t)r * kL1 + tid] = 0u;
  };

  // ---------------------------------------------------------------- A
  // This workgroup attends over its own selection and every WR-th entry
  // (from c) of the row's sink ++ local tail.
  const uint16_t* kb = a.kc + (int64_t)b * a.k_sb + (int64_t)hkv * a.k_sh;
  const uint16_t* vb = a.vc + (int64_t)b * a.v_sb + (int64_t)hkv * a.v_sh;
  WaveState<DT, kG, kDh> ws;
#pragma unroll
  for (int ks = 0; ks < kDh / 16; ++ks) {
    ws.qf[ks] = qpre[ks];
    ws.acc[ks] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  ws.m = -INFINITY;
  ws.l = 0.f;
  const int n_fix = pr.sink + pr.tail_count;
  const int n_st = n_fix > c ? (n_fix - c + a.WR - 1) / a.WR : 0;
  const int n_loc = (int)n_sel + n_st;
  // local keep position p -> cache row (-1 past the row's rows)
  // (kept: keep-list entry p when p < n_sel)
  auto keep_tok = [&](int p, int kept) -> int {
    if (p >= n_loc) return -1;
    int64_t t;
    if (p < (int)n_sel) t = kept;
    else {
      const int jt = c + (p - (int)n_sel) * a.WR;
      t = jt < pr.sink ? jt : (int64_t)pr.tail_start + (jt - pr.sink);
    }
    return (t < 0 || t >= pr.t_total) ? -1 : (int)t;
  };
  const int nsteps = (n_loc + kKeys - 1) / kKeys;
  const int p4r = 4 * (lane >> 4);
  for (int i = wave; i < nsteps; i += kWaves) {
    const int p = i * kKeys + (lane & 15);
    const int tok = keep_tok(p, lds.keep[min(p, kKeepMax - 1)]);
    // keys 4r .. 4r + 3 of this lane's row r: one 16-byte read (a start past
    // the keep list means every entry is past n_sel, so the clamp is unused)
    const int p4 = i * kKeys + p4r;
    const int4 kq = *reinterpret_cast<const int4*>(lds.keep + min(p4, kKeepMax - 4));
    const int tv[4] = {keep_tok(p4, kq.x), keep_tok(p4 + 1, kq.y), keep_tok(p4 + 2, kq.z),
                       keep_tok(p4 + 3, kq.w)};
    const int mk[4] = {0, 0, 0, 0};
    KvStep<kDh> st;
    kv_issue_rows<kDh>(st, kb, vb, a.k_st, a.v_st, tok, tv, mk, lane);
    attn_step<DT, kG, kDh>(ws, st, a.scale_log2, lane);
  }
  finish_row<DT, true>(a, ws, lds, s_m, s_l, s_flag, r, c, b, h0, select, min(nsteps, kWaves),
                 out_stores);
}

// The level-1 bins of four selection rows at once: per head h, the unique bin
// b of h[h][0..1023] with S(b) >= target > S(b+1); s_res[h] = {b, S(b+1)}.
// 1024 threads, thread tid holding x[h] = h[h][1023 - tid]; 1 <= target <=
// S(0) for every head.
__device__ __forceinline__ void select_bin1024x4(const uint32_t (&x)[kG], uint32_t target,
                                                 uint32_t (&s_wsum)[kG][kWaves],
                                                 uint32_t (&s_res)[kG][4]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t inc[kG];
#pragma unroll
  for (int g = 0; g < kG; ++g) {
    inc[g] = wave_inclusive_scan(x[g]);
    if (lane == 63) s_wsum[g][wave] = inc[g];
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < kG; ++g) {
    const uint32_t above = waves_before(s_wsum[g], wave, lane) + inc[g] - x[g];
    if (above + x[g] >= target && above < target) {
      s_res[g][0] = kL1 - 1 - tid;
      s_res[g][1] = above;
    }
  }
  __syncthreads();
}

// Per-head selection (LAP_SELECT_PER_HEAD, the reference's rule: each query
// head keeps its own top-k): the phases of step_fused_kernel with the four
// heads' selections side by side under the same two row barriers.  Scoring
// keeps four 16-bit keys per token and four level-1 histograms; H and H2
// resolve the four thresholds together; each head writes its own index row;
// A attends once over the union of the four selections, each key carrying
// the bits of the heads that keep it, so one MFMA pass serves every head.
// The split merge is the group kernel's.
template <int DT, int TOK>
__global__ __launch_bounds__(kTH) void step_fused_ph_kernel(StepArgs a) {
  static_assert(TOK >= 1 && TOK <= kMaxTokPH, "TOK");
  static_assert(kMaxTokPH * kTH <= kKeepMax, "a chunk's union fits the keep list");
  __shared__ __attribute__((aligned(16))) uint4 s_big[kLutBytes / 16];
  __shared__ uint32_t s_hist[kG * kHCph * kH1Pitch];
  __shared__ __attribute__((aligned(16))) uint8_t s_kmask[kKeepMax];
  __shared__ uint32_t s_h2[kG][kL2], s_wsum[kG][kWaves], s_res[kG][4], s_sel[kG][4];
  constexpr int kLists = (kG + 1) * TOK;
  static_assert(kWaves == 16, "one 16-lane row per list");
  __shared__ uint32_t s_wcnt[(kG + 1) * kMaxTokPH * kWaves], s_ltot[(kG + 1) * kMaxTokPH];
  __shared__ uint32_t s_gtw[kG][kWaves];
  __shared__ uint32_t s_flag;
  __shared__ float s_m[kWaves][4], s_l[kWaves][4];

  Lds lds;
  lds.lut = s_big;
  lds.keep = reinterpret_cast<int*>(s_big);
  lds.o = reinterpret_cast<float*>(s_big) + kKeepMax;

  StepPos ps;
  if (!step_pos<TOK>(a, &ps)) return;  // no row here
  const int r = ps.r, c = ps.c, b = ps.b, hkv = ps.hkv, h0 = ps.h0, t0 = ps.t0, t1 = ps.t1;
  const StepRow pr = ps.pr;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool select = pr.k > 0;
  i16x4 qpre[kDh / 16];
  load_q_frags(a, b, h0, lane, qpre);

  // ---------------------------------------------------------------- S
  // kp[j]: the four heads' keys of stage j's token (heads 0, 1 in .x, 2, 3
  // in .y); inw bit j: the token is a candidate.
  uint2 kp[TOK];
  uint32_t inw = 0;
  for (int i = tid; i < kG * kHCph * kH1Pitch; i += kTH) s_hist[i] = 0;
  if (select && t0 < t1) {
    const int copy = (int)(__lane_id() % kHCph) * kH1Pitch;
    score_chunk<TOK>(a, ps, lds.lut, [&](int j, int t, float e0, float e1, float e2, float e3) {
      kp[j] = make_uint2(0u, 0u);
      if (t < t1 && t >= pr.cs && t < pr.ce) {
        const uint32_t k0 = key_of_score(e0, a.key_bf16), k1 = key_of_score(e1, a.key_bf16);
        const uint32_t k2 = key_of_score(e2, a.key_bf16), k3 = key_of_score(e3, a.key_bf16);
        kp[j] = make_uint2(k0 | (k1 << 16), k2 | (k3 << 16));
        inw |= 1u << j;
        atomicAdd(&s_hist[(0 * kHCph) * kH1Pitch + copy + (k0 >> kLoBits)], 1u);
        atomicAdd(&s_hist[(1 * kHCph) * kH1Pitch + copy + (k1 >> kLoBits)], 1u);
        atomicAdd(&s_hist[(2 * kHCph) * kH1Pitch + copy + (k2 >> kLoBits)], 1u);
        atomicAdd(&s_hist[(3 * kHCph) * kH1Pitch + copy + (k3 >> kLoBits)], 1u);
      }
    });
  }
  __syncthreads();
#pragma unroll
  for (int ks = 0; ks < kDh / 16; ++ks) asm volatile("" : "+v"(qpre[ks]));
  auto key = [&](int j, int g) -> uint32_t {
    const uint32_t w = g < 2 ? kp[j].x : kp[j].y;
    return (g & 1) ? (w >> 16) : (w & 0xffffu);
  };
  // This chunk's level-1 counts of bin tid, added to the four rows' histograms.
  uint32_t h1[kG] = {0u, 0u, 0u, 0u};
  if (select) {
#pragma unroll
    for (int g = 0; g < kG; ++g) {
#pragma unroll
      for (int cp = 0; cp < kHCph; ++cp) h1[g] += s_hist[(g * kHCph + cp) * kH1Pitch + tid];
      if (h1[g])
        __hip_atomic_fetch_add(a.hist + ((int64_t)r * kG + g) * kL1 + tid, h1[g],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // ---------------------------------------------------------------- B1, H
  uint32_t n_sel = 0;
  uint32_t hbase[kG] = {0u, 0u, 0u, 0u};  // where each head's selection of this chunk starts
  if (select) {
    if (tid == 0) record_xcd(a, r);  // complete before B2's arrival
    wg_row_barrier(a, r, 0);
    uint32_t hv[kG];
#pragma unroll
    for (int g = 0; g < kG; ++g)
      hv[g] = ld_dev(a.hist + ((int64_t)r * kG + g) * kL1 + kL1 - 1 - tid);
    if (tid < kG * kL2) (&s_h2[0][0])[tid] = 0;  // ordered before H's adds, as above
    select_bin1024x4(hv, (uint32_t)pr.k, s_wsum, s_res);
    uint32_t b1[kG], gt1[kG];
#pragma unroll
    for (int g = 0; g < kG; ++g) {
      b1[g] = s_res[g][0];
      gt1[g] = s_res[g][1];
    }
#pragma unroll
    for (int j = 0; j < TOK; ++j)
      if ((inw >> j) & 1)
#pragma unroll
        for (int g = 0; g < kG; ++g)
          if ((key(j, g) >> kLoBits) == b1[g]) atomicAdd(&s_h2[g][key(j, g) & (kL2 - 1)], 1u);
#pragma unroll
    for (int g = 0; g < kG; ++g) {
      const uint32_t gt = wave_sum((uint32_t)tid > b1[g] ? h1[g] : 0u);
      if (lane == 0) s_gtw[g][wave] = gt;
    }
    __syncthreads();
    uint32_t* t2 = a.t2 + ((int64_t)r * a.WR + c) * kG * kT2;  // [kG][kT2] of this chunk
    if (tid < kG * kL2) t2[(tid / kL2) * kT2 + tid % kL2] = (&s_h2[0][0])[tid];
    if (tid >= kG * kL2 && tid < kG * kL2 + kG) {
      const int g = tid - kG * kL2;
      uint32_t my_gt1 = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) my_gt1 += s_gtw[g][w];
      t2[g * kT2 + kL2] = my_gt1;
    }
    wg_row_barrier(a, r, 1);

    // ------------------------------------------------------------ H2
    // Waves 0..3, wave g for head g: lane l holds bin 63 - l of every
    // chunk's level-2 table of head g (chunks past WR read as zero) and, for
    // l < WR, chunk l's count above b1; the sums are those of the group
    // step's H2, in registers, published with one barrier.
    if (wave < kG) {
      const int g = wave;
      const uint32_t k2 = (uint32_t)pr.k - gt1[g];  // keys to take from bin b1[g], >= 1
      const uint32_t* t2r = a.t2 + ((int64_t)r * a.WR * kG + g) * kT2;  // chunk stride kG * kT2
      const int bn = kL2 - 1 - lane;
      uint32_t vt[kMaxWR];
#pragma unroll
      for (int c2 = 0; c2 < kMaxWR; ++c2)
        vt[c2] = ld_dev(t2r + (int64_t)min(c2, a.WR - 1) * kG * kT2 + bn);
      const uint32_t gt_l = ld_dev(t2r + (int64_t)min(lane, a.WR - 1) * kG * kT2 + kL2);
      uint32_t tot = 0, before = 0, mine = 0;  // bin bn: the row's, chunks < c, chunk c
#pragma unroll
      for (int c2 = 0; c2 < kMaxWR; ++c2) {
        const uint32_t x = c2 < a.WR ? vt[c2] : 0u;
        tot += x;
        before += c2 < c ? x : 0u;
        mine += c2 == c ? x : 0u;
      }
      const uint32_t inc = wave_inclusive_scan(tot);
      const uint64_t hit = __ballot(inc >= k2 && inc - tot < k2);
      const int L = hit ? __builtin_ctzll(hit) : kL2 - 1;
      const uint32_t need = k2 - (uint32_t)__builtin_amdgcn_readlane((int)(inc - tot), L);
      const uint32_t ts = (uint32_t)__builtin_amdgcn_readlane((int)before, L);
      const uint32_t my_ties = (uint32_t)__builtin_amdgcn_readlane((int)mine, L);
      const uint32_t gs = wave_sum((lane < L ? before : 0u) + (lane < c ? gt_l : 0u));
      if (lane == 0) {
        const uint32_t tk = ts >= need ? 0u : min(my_ties, need - ts);
        uint32_t taken_before;  // min(need, ts), explicit (see step_fused_kernel)
        asm volatile("v_min_u32 %0, %1, %2" : "=v"(taken_before) : "v"(need), "v"(ts));
        s_res[g][2] = (uint32_t)(kL2 - 1 - L);
        s_sel[g][0] = tk;
        s_sel[g][1] = gs + taken_before;
        s_sel[g][2] = my_ties;
      }
    }
    __syncthreads();
    uint32_t tau[kG];
#pragma unroll
    for (int g = 0; g < kG; ++g) tau[g] = (b1[g] << kLoBits) | s_res[g][2];

    // Ordered compaction, per head (its index row) and of the union (the
    // keep list of A, with each key's head bits).
    uint32_t take[kG], base[kG], ties[kG];
    bool partial = false;
#pragma unroll
    for (int g = 0; g < kG; ++g) {
      take[g] = s_sel[g][0];
      base[g] = s_sel[g][1];
      hbase[g] = base[g];
      ties[g] = s_sel[g][2];
      partial |= take[g] > 0 && take[g] < ties[g];
    }
    // Positions come from per-wave counts: list l = g * TOK + j (g < 4: head
    // g's selection, or its ties at tau; g = 4: the union) counts its
    // stage-j tokens per wave, then one 16-lane row scan per list gives each
    // wave's exclusive prefix and the list's total.
    auto scan_lists = [&]() { scan_wave_counts<kLists>(s_wcnt, s_ltot); };
    // the chunk's ties at tau, for heads that take only some of them (their
    // ranks, lowest columns first)
    if (partial) {
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        if (!(take[g] > 0 && take[g] < ties[g])) continue;
#pragma unroll
        for (int j = 0; j < TOK; ++j) {
          const uint64_t mt = __ballot(((inw >> j) & 1u) & (key(j, g) == tau[g]));
          if (lane == 0) s_wcnt[(g * TOK + j) * kWaves + wave] = (uint32_t)__popcll(mt);
        }
      }
      scan_lists();
    }
    uint32_t selb = 0;  // bit 4 j + g: stage j's token selected by head g
#pragma unroll
    for (int g = 0; g < kG; ++g) {
      const bool part = take[g] > 0 && take[g] < ties[g];
      uint32_t tie_base = 0;
#pragma unroll
      for (int j = 0; j < TOK; ++j) {
        const bool in = (inw >> j) & 1;
        const uint32_t kj = key(j, g);
        bool sj;
        if (part) {
          const uint64_t mt = __ballot(in & (kj == tau[g]));
          const uint32_t rank = tie_base + s_wcnt[(g * TOK + j) * kWaves + wave] + lanes_below(mt);
          sj = in & ((kj > tau[g]) | ((kj == tau[g]) & (rank < take[g])));
          tie_base += s_ltot[g * TOK + j];
        } else {
          sj = in & ((kj > tau[g]) | ((take[g] > 0) & (kj == tau[g])));
        }
        selb |= (sj ? 1u : 0u) << (4 * j + g);
      }
    }
    if (partial) __syncthreads();  // the tie prefixes are read
    // The union (keys any head keeps) in column order, with each key's head
    // bits: the keep list of A, and the source of the four index rows, which
    // out_stores writes after the merge arrival (head g's row is the union's
    // keys with bit g, in order).
#pragma unroll
    for (int j = 0; j < TOK; ++j) {
      const uint64_t m = __ballot(((selb >> (4 * j)) & 0xfu) != 0u);
      if (lane == 0) s_wcnt[j * kWaves + wave] = (uint32_t)__popcll(m);
    }
    scan_wave_counts<TOK>(s_wcnt, s_ltot);
    uint32_t ubase = 0;
#pragma unroll
    for (int j = 0; j < TOK; ++j) {
      const uint32_t bits = (selb >> (4 * j)) & 0xfu;
      const uint64_t m = __ballot(bits != 0u);
      const uint32_t q = ubase + s_wcnt[j * kWaves + wave] + lanes_below(m);
      if (bits) {
        lds.keep[q] = t0 + j * kTH + tid;
        s_kmask[q] = (uint8_t)bits;
      }
      ubase += s_ltot[j];
    }
    n_sel = ubase;
  }
  lds_barrier();  // the keep list

  // The stores nothing in this launch reads, after the merge arrival: the
  // chunk's part of the four index rows, ragged rows' padding, and (last
  // arrival) the histogram clear.  Thread t takes union entries [t E, t E +
  // E); its rank among each head's keys comes from a block scan of
  // per-thread counts (two heads per word, 16 bits each: a chunk keeps at
  // most 8192 keys).
  auto out_stores = [&](bool last) {
    if (n_sel > 0) {
      const int E = ((int)n_sel + kTH - 1) / kTH;
      const int p0 = min(tid * E, (int)n_sel), p1 = min(p0 + E, (int)n_sel);
      uint32_t c01 = 0, c23 = 0;
      for (int p = p0; p < p1; ++p) {
        const uint32_t m = s_kmask[p];
        c01 += (m & 1u) | ((m & 2u) << 15);
        c23 += ((m >> 2) & 1u) | ((m & 8u) << 13);
      }
      const uint32_t i01 = wave_inclusive_scan(c01), i23 = wave_inclusive_scan(c23);
      __syncthreads();  // s_wsum is free again
      if (lane == 63) {
        s_wsum[0][wave] = i01;
        s_wsum[1][wave] = i23;
      }
      __syncthreads();
      if (tid < 2 * kWaves) {  // the waves' sums to their exclusive prefix, one row per pair
        uint32_t* f = &s_wsum[tid / kWaves][tid % kWaves];
        const uint32_t v = *f;
        *f = row16_inclusive_scan(v) - v;
      }
      __syncthreads();
      const uint32_t e01 = s_wsum[0][wave] + i01 - c01, e23 = s_wsum[1][wave] + i23 - c23;
      uint32_t rk[kG] = {e01 & 0xffffu, e01 >> 16, e23 & 0xffffu, e23 >> 16};
      for (int p = p0; p < p1; ++p) {
        const uint32_t m = s_kmask[p];
        const int col = lds.keep[p];
#pragma unroll
        for (int g = 0; g < kG; ++g) {
          if (!((m >> g) & 1u)) continue;
          const uint32_t q = hbase[g] + rk[g]++;
          if (q < (uint32_t)pr.k) {
            const int64_t i = ((int64_t)b * a.Hkv * kG + h0 + g) * a.k_cols + q;
            if (a.idx_i64) put_idx<int64_t>(a.idx, i, col);
            else put_idx<int32_t>(a.idx, i, col);
          }
        }
      }
    }
    if (a.plans) {  // pad [k, k_cols) of the four rows with -1, split over the workgroups
      const int pad = a.k_cols - pr.k;
      const int ps = (pad + a.WR - 1) / a.WR;
      for (int i = c * ps + tid; i < min(pad, (c + 1) * ps); i += kTH) {
#pragma unroll
        for (int g = 0; g < kG; ++g) {
          const int64_t irow = ((int64_t)b * a.Hkv * kG + h0 + g) * a.k_cols + pr.k;
          if (a.idx_i64) put_idx<int64_t>(a.idx, irow + i, -1);
          else put_idx<int32_t>(a.idx, irow + i, -1);
        }
      }
    }
    if (select && last) {
#pragma unroll
      for (int g = 0; g < kG; ++g) a.hist[((int64_t)r * kG + g) * kL1 + tid] = 0u;
    }
  };

  // ---------------------------------------------------------------- A
  // This workgroup attends over the union of its heads' selections (each
  // head scores only its own keys) and every WR-th entry (from c) of the
  // row's sink ++ local tail, which every head keeps.
  const uint16_t* kb = a.kc + (int64_t)b * a.k_sb + (int64_t)hkv * a.k_sh;
  const uint16_t* vb = a.vc + (int64_t)b * a.v_sb + (int64_t)hkv * a.v_sh;
  WaveState<DT, kG, kDh> ws;
#pragma unroll
  for (int ks = 0; ks < kDh / 16; ++ks) {
    ws.qf[ks] = qpre[ks];
    ws.acc[ks] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  ws.m = -INFINITY;
  ws.l = 0.f;
  const int n_fix = pr.sink + pr.tail_count;
  const int n_st = n_fix > c ? (n_fix - c + a.WR - 1) / a.WR : 0;
  const int n_loc = (int)n_sel + n_st;
  const int nsteps = (n_loc + kKeys - 1) / kKeys;
  // key p's cache row (kept: keep-list entry p when p < n_sel)
  auto keep_tok = [&](int p, int kept) -> int {
    int tok = -1;
    if (p < (int)n_sel) tok = kept;
    else if (p < n_loc) {
      const int jt = c + (p - (int)n_sel) * a.WR;
      tok = jt < pr.sink ? jt : pr.tail_start + (jt - pr.sink);
    }
    return (tok < 0 || tok >= pr.t_total) ? -1 : tok;
  };
  // key p's head bits (bits: its keep-mask byte when p < n_sel)
  auto keep_bits = [&](int p, uint32_t bits) -> int {
    return p < (int)n_sel ? (int)(bits & 0xfu) : (p < n_loc ? 0xf : 0);
  };
  const int p4r = 4 * (lane >> 4);
  for (int i = wave; i < nsteps; i += kWaves) {
    const int p = i * kKeys + (lane & 15);
    const int tok = keep_tok(p, lds.keep[min(p, kKeepMax - 1)]);
    // keys 4r .. 4r + 3 of this lane's row r: one 16-byte read of the keep
    // list and one word of the masks (clamped as in step_fused_kernel)
    const int p4 = i * kKeys + p4r, q4 = min(p4, kKeepMax - 4);
    const int4 kq = *reinterpret_cast<const int4*>(lds.keep + q4);
    const uint32_t mq = *reinterpret_cast<const uint32_t*>(s_kmask + q4);
    const int tv[4] = {keep_tok(p4, kq.x), keep_tok(p4 + 1, kq.y), keep_tok(p4 + 2, kq.z),
                       keep_tok(p4 + 3, kq.w)};
    const int mk[4] = {keep_bits(p4, mq), keep_bits(p4 + 1, mq >> 8), keep_bits(p4 + 2, mq >> 16),
                       keep_bits(p4 + 3, mq >> 24)};
    KvStep<kDh> st;
    kv_issue_rows<kDh>(st, kb, vb, a.k_st, a.v_st, tok, tv, mk, lane);
    attn_step<DT, kG, kDh, true>(ws, st, a.scale_log2, lane);
  }
  finish_row<DT, false>(a, ws, lds, s_m, s_l, s_flag, r, c, b, h0, select, min(nsteps, kWaves),
                 out_stores);
}

inline _Float16 f16_one() { return (_Float16)1.0f; }

// Device facts the fused launch needs: XCDs and CUs per device.
struct XcdInfo {
  int nxcc = 0, cu = 0;
};
int xcd_info(XcdInfo* out) {
  static XcdInfo cache[64];
  int dev = 0;
  LAP_HIP(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= 64) {
    set_error("device index %d out of range", dev);
    return LAP_ERR_HIP;
  }
  if (cache[dev].nxcc == 0) {
    int n = 0, cu = 0;
    LAP_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, dev), "XCC count");
    LAP_HIP(hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev), "CU count");
    cache[dev].cu = cu;
    cache[dev].nxcc = n < 1 ? 1 : n;
  }
  *out = cache[dev];
  return LAP_OK;
}

// Launch shape of the fused step, or false when it does not apply.
struct FusedPlan {
  int nxcc, RX, WR, tok, grid;
};
// k_sel bounds a workgroup's own selection (the call's k, or k_cols): a
// chunk longer than the LDS keep list needs k_sel <= kKeepMax.  Chunks of 9
// to 16 tokens per thread run as 16 (group selection only).
bool fused_plan(int R, int T, bool per_head, int k_sel, FusedPlan* p) {
  static const int mode = [] {
    const char* e = getenv("LAPRUNE_FUSED");
    return e ? atoi(e) : 1;
  }();
  if (mode == 0) return false;
  XcdInfo xi;
  if (xcd_info(&xi) != LAP_OK || xi.cu % xi.nxcc != 0) return false;
  const int per_xcd = xi.cu / xi.nxcc;
  const int RX = (R + xi.nxcc - 1) / xi.nxcc;
  int WR = std::min(per_xcd / RX, kMaxWR);
  WR = std::min(WR, std::max(1, (T + kTH - 1) / kTH));
  if (WR < 1) return false;
  const int ch = (T + WR - 1) / WR;
  int tok = (ch + kTH - 1) / kTH;
  if (tok > 8) tok = 16;
  if (tok < 1 || tok > (per_head ? kMaxTokPH : kMaxTok)) return false;
  if (tok * kTH > kKeepMax && k_sel > kKeepMax) return false;
  *p = FusedPlan{xi.nxcc, RX, WR, tok, xi.nxcc * RX * WR};
  return true;
}

struct StepWs {
  uint32_t* status;
  uint32_t* bar;
  uint32_t* hist;
  uint32_t* t2;
  float* part;
  size_t bytes;
};
// Workspace of the fused step for R rows and WR workgroups per row: status
// words, barrier lines and row histograms (these three must start zeroed,
// and every call leaves them zeroed), then the per-chunk level-2 tables and
// the attention partials.  The barrier lines and histograms are laid out for
// head_rows >= R rows, so that calls of different R on one buffer find
// their persistent words at the same addresses.  With WR = 0, the persistent
// head only.
StepWs carve_step(void* base, int R, int WR, int head_rows) {
  StepWs w{};
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) {
    char* q = p ? p + off : nullptr;
    off = align_up(off + bytes, 256);
    return q;
  };
  w.status = reinterpret_cast<uint32_t*>(take(kStatusBytes));
  w.bar = reinterpret_cast<uint32_t*>(take((size_t)head_rows * 3 * kBarWords * 4));
  w.hist = reinterpret_cast<uint32_t*>(take((size_t)head_rows * kG * kL1 * 4));
  w.t2 = reinterpret_cast<uint32_t*>(take((size_t)R * WR * kG * kT2 * 4));
  w.part = reinterpret_cast<float*>(take((size_t)R * WR * kG * (kDh + 2) * 4));
  w.bytes = off;
  return w;
}

template <int DT>
void launch_fused_dt(const StepArgs& a, int tok, int grid, bool per_head, hipStream_t st) {
  switch (tok) {
#define LAP_STEP(TK)                                                                       \
  case TK:                                                                                 \
    if (per_head)                                                                          \
      hipLaunchKernelGGL((step_fused_ph_kernel<DT, TK>), dim3(grid), dim3(kTH), 0, st, a); \
    else                                                                                   \
      hipLaunchKernelGGL((step_fused_kernel<DT, TK>), dim3(grid), dim3(kTH), 0, st, a);    \
    break;
    LAP_STEP(1) LAP_STEP(2) LAP_STEP(3) LAP_STEP(4) LAP_STEP(5) LAP_STEP(6) LAP_STEP(7)
    LAP_STEP(8)
#undef LAP_STEP
    case 16:  // group selection only (fused_plan)
      hipLaunchKernelGGL((step_fused_kernel<DT, 16>), dim3(grid), dim3(kTH), 0, st, a);
      break;
  }
}

}  // namespace

// Bytes at the start of a lap_decode_step workspace that only the fused
// kernel uses: the status words, barrier lines and row histograms (kept zero
// between calls, whatever path a call takes) and, when the fused kernel applies to this
// shape (with either selection), its level-2 tables and partials.
size_t decode_step_fused_bytes(int R, int T, int head_rows) {
  FusedPlan fp;
  if (!fused_plan(R, T, false, 0, &fp)) return carve_step(nullptr, R, 0, head_rows).bytes;
  return carve_step(nullptr, R, fp.WR, head_rows).bytes;
}

// Run the fused step; LAP_ERR_UNSUPPORTED when this shape must take the
// kernel chain instead.
int decode_step_fused(const void* lut_gmkg, const uint8_t* codes, int64_t cs_b, int64_t cs_h,
                      int64_t cs_t, const void* q, int64_t q_sb, int64_t q_sh, const void* keys,
                      const void* vals, int dtype, int B, int Hkv, int T_kv, int64_t k_sb,
                      int64_t k_sh, int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st,
                      int T, int cand_start, int cand_end, int k, int sink, int tail_start,
                      int tail_count, const lap_row_plan* plans, int k_cols, int max_sink,
                      int max_tail, int key_bf16, float scale, void* out_idx, int idx_dtype,
                      void* out, void* workspace, size_t ws_bytes, int head_rows,
                      bool per_head, const char* who, hipStream_t st) {
  const int R = B * Hkv;
  FusedPlan fp;
  if (R > head_rows) return LAP_ERR_UNSUPPORTED;  // more rows than the head holds: the chain
  if (!fused_plan(R, T, per_head, plans ? k_cols : k, &fp)) return LAP_ERR_UNSUPPORTED;
  if (!score_g4_supported(codes, cs_b, cs_h, cs_t)) return LAP_ERR_UNSUPPORTED;
  // query fragments are read as 8-byte vectors
  if ((reinterpret_cast<uintptr_t>(q) & 7) || (q_sb & 3) || (q_sh & 3)) return LAP_ERR_UNSUPPORTED;
  StepWs w = carve_step(workspace, R, fp.WR, head_rows);
  LAP_CHECK_CODE(workspace && ws_bytes >= w.bytes, LAP_ERR_WORKSPACE,
                 "%s: %zu bytes of workspace needed", who, w.bytes);
  StepArgs a{};
  a.lut = static_cast<const uint16_t*>(lut_gmkg);
  a.codes = codes;
  a.cs_b = cs_b; a.cs_h = cs_h; a.cs_t = cs_t;
  a.B = B; a.Hkv = Hkv; a.T = T;
  a.plans = reinterpret_cast<const int32_t*>(plans);
  a.cand_start = cand_start; a.cand_end = cand_end; a.k = k;
  a.sink = sink; a.tail_start = tail_start; a.tail_count = tail_count;
  a.k_cols = k_cols; a.max_sink = max_sink; a.max_tail = max_tail;
  a.key_bf16 = key_bf16;
  a.q = static_cast<const uint16_t*>(q); a.q_sb = q_sb; a.q_sh = q_sh;
  a.kc = static_cast<const uint16_t*>(keys); a.vc = static_cast<const uint16_t*>(vals);
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.T_kv = T_kv;
  a.scale_log2 = scale * kLog2e;
  a.idx = out_idx;
  a.idx_i64 = idx_dtype == LAP_DTYPE_I64;
  a.out = static_cast<uint16_t*>(out);
  a.status = w.status; a.bar = w.bar; a.hist = w.hist; a.t2 = w.t2; a.part = w.part;
  a.nxcc = fp.nxcc; a.RX = fp.RX; a.WR = fp.WR;
  a.one = f16_one();
  if (dtype == LAP_DTYPE_F16) launch_fused_dt<LAP_DTYPE_F16>(a, fp.tok, fp.grid, per_head, st);
  else launch_fused_dt<LAP_DTYPE_BF16>(a, fp.tok, fp.grid, per_head, st);
  LAP_LAUNCH_CHECK(per_head ? "step_fused_ph_kernel" : "step_fused_kernel");
  return LAP_OK;
}

}  // namespace lap

using namespace lap;

namespace {

// Rows a selection serves per KV row: 4 with LAP_SELECT_PER_HEAD, else 1.
// Selection rows per KV head: its G query heads (LAP_SELECT_PER_HEAD) or
// one group row.
int step_rows_per_kv(int key_mode, int G) { return (key_mode & LAP_SELECT_PER_HEAD) ? G : 1; }

// The chain's part of the workspace (after the fused part): the retrieve
// workspace, then the attention partials.
// The kernel chain's workspace: the retrieval part (G = 4: the fused
// scorer's keys and histograms; other G: fp16 per-head scores [B * Hq][T],
// `scores` bytes, then the top-k's workspace) and the attention's partials.
struct ChainWs {
  size_t ret, attn, scores;
};
int chain_ws(int B, int Hq, int Hkv, int T, int D, int keep_max, int key_mode, ChainWs* w) {
  const int G = Hq / Hkv;
  size_t r = 0, a = 0;
  w->scores = 0;
  if (G == 4) {
    int s = lap_retrieve_workspace_size(B * Hkv * step_rows_per_kv(key_mode, G), T, &r);
    if (s != LAP_OK) return s;
  } else {
    w->scores = align_up((size_t)B * Hq * T * sizeof(uint16_t), 256);
    int s = lap_topk_workspace_size(B * Hkv * step_rows_per_kv(key_mode, G), T, &r);
    if (s != LAP_OK) return s;
    r += w->scores;
  }
  int s = lap_attn_decode_workspace_size(B, Hq, D, keep_max, &a);
  if (s != LAP_OK) return s;
  w->ret = align_up(r, 256);
  w->attn = align_up(a, 256);
  return LAP_OK;
}

}  // namespace

namespace {

// One decode step after argument checks, on `workspace` of `ws_bytes`
// bytes whose persistent head is laid out for head_rows rows.  With
// need_all, the workspace must hold the fused part and the chain's part
// whatever path runs (lap_decode_step's contract); otherwise each path
// checks only what it uses.
int decode_step_run(const char* who, const void* lut_gmkg, const uint8_t* codes,
                    int64_t codes_stride_b, int64_t codes_stride_h, int64_t codes_stride_t, int T,
                    int cand_start, int cand_end, int k, int sink_count, int tail_start,
                    int tail_count, const lap_row_plan* plans, int k_cols, int max_sink,
                    int max_tail, int key_mode, const void* q, int64_t q_sb, int64_t q_sh,
                    const void* keys, const void* vals, int dtype, int B, int Hq, int Hkv,
                    int T_kv, int D, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t v_sb,
                    int64_t v_sh, int64_t v_st, float scale, void* out_idx, int idx_dtype,
                    void* out, void* workspace, size_t workspace_bytes, int head_rows,
                    bool need_all, lap_stream_t stream) {
  LAP_CHECK(lut_gmkg && q && keys && vals && out, "%s: null pointer", who);
  LAP_CHECK(B > 0 && Hq > 0 && Hkv > 0 && T > 0 && T_kv > 0 && D > 0, "%s: bad sizes", who);
  LAP_CHECK(Hq % Hkv == 0, "%s: Hq=%d is not a multiple of Hkv=%d", who, Hq, Hkv);
  const int G = Hq / Hkv;
  LAP_CHECK_CODE(G >= 1 && G <= 8, LAP_ERR_UNSUPPORTED,
                 "%s: group size %d unsupported (1 to 8 query heads per KV head)", who, G);
  LAP_CHECK(dtype == LAP_DTYPE_BF16 || dtype == LAP_DTYPE_F16, "%s: q/K/V must be bf16 or fp16",
            who);
  LAP_CHECK(idx_dtype == LAP_DTYPE_I32 || idx_dtype == LAP_DTYPE_I64,
            "%s: idx must be int32 or int64", who);
  const int km = key_mode & ~LAP_SELECT_PER_HEAD;
  LAP_CHECK(km == LAP_KEY_F16 || km == LAP_KEY_BF16, "%s: bad key mode", who);
  LAP_CHECK(!plans || (k_cols >= 0 && max_sink >= 0 && max_tail >= 0), "%s: negative bound",
            who);
  int keep_max = 0;
  int k_eff = 0;
  if (!plans) {
    LAP_CHECK(cand_start >= 0 && cand_end <= T && cand_start <= cand_end,
              "%s: candidate window [%d,%d) outside [0,%d)", who, cand_start, cand_end, T);
    LAP_CHECK(k >= 0 && sink_count >= 0 && tail_count >= 0, "%s: negative count", who);
    if (tail_count > 0) LAP_CHECK(tail_start >= 0, "%s: tail_start < 0", who);
    k_eff = std::min(k, cand_end - cand_start);
    keep_max = k_eff + sink_count + tail_count;
  } else {
    keep_max = k_cols + max_sink + max_tail;
  }
  const bool selects = plans ? k_cols > 0 : k_eff > 0;
  LAP_CHECK(out_idx || !selects, "%s: null index output", who);
  LAP_CHECK(codes || !selects, "%s: null pointer (codes)", who);
  ChainWs cw;
  int s = chain_ws(B, Hq, Hkv, T, D, keep_max, key_mode, &cw);
  if (s != LAP_OK) return s;
  const size_t fused = align_up(decode_step_fused_bytes(B * Hkv, T, head_rows), 256);
  if (need_all)
    LAP_CHECK_CODE(workspace && workspace_bytes >= fused + cw.ret + cw.attn, LAP_ERR_WORKSPACE,
                   "%s: workspace of %zu bytes needed", who, fused + cw.ret + cw.attn);
  hipStream_t st = as_stream(stream);
  if (D == 128 && G == 4) {
    s = decode_step_fused(lut_gmkg, codes, codes_stride_b, codes_stride_h, codes_stride_t, q, q_sb,
                          q_sh, keys, vals, dtype, B, Hkv, T_kv, k_sb, k_sh, k_st, v_sb, v_sh,
                          v_st, T, cand_start, cand_end, k_eff, sink_count, tail_start,
                          tail_count, plans, plans ? k_cols : k_eff, max_sink, max_tail,
                          km == LAP_KEY_BF16, scale, out_idx, idx_dtype, out, workspace,
                          std::min(workspace_bytes, fused), head_rows,
                          (key_mode & LAP_SELECT_PER_HEAD) != 0, who, st);
    if (s != LAP_ERR_UNSUPPORTED) return s;
    clear_error();
  }
  // the kernel chain: scorer + top-k, then the split-K attention and merge
  LAP_CHECK_CODE(workspace && workspace_bytes >= fused + cw.ret + cw.attn, LAP_ERR_WORKSPACE,
                 "%s: workspace of %zu bytes needed", who, fused + cw.ret + cw.attn);
  char* base = static_cast<char*>(workspace) + fused;
  void* ws_r = base;
  void* ws_a = base + cw.ret;
  const int rows = step_rows_per_kv(key_mode, G);
  const int H_idx = Hkv * rows;
  if (G != 4) {
    // Per-head fp16 scores of every code column (lap_lut_score_gqa over the
    // [B * Hq][32][256] table), then the top-k of the group max (group
    // selection) or of each head's row.
    if (selects) {
      uint16_t* sc = reinterpret_cast<uint16_t*>(base);
      const uint16_t* lut = static_cast<const uint16_t*>(lut_gmkg);
      for (int b = 0; b < B; ++b) {
        s = lap_lut_score_gqa(lut + (int64_t)b * Hq * kM * kK, codes + b * codes_stride_b,
                              codes_stride_h, codes_stride_t, Hkv, G, T, kM, kK, 0, kM, nullptr,
                              T, sc + (int64_t)b * Hq * T, stream);
        if (s != LAP_OK) return s;
      }
      void* ws_t = base + cw.scores;
      const size_t ws_t_bytes = cw.ret - cw.scores;
      if (!plans)
        s = lap_topk_select(sc, T, B * H_idx, G / rows, T, cand_start, cand_end, k_eff, km,
                            out_idx, idx_dtype, ws_t, ws_t_bytes, stream);
      else
        s = lap_topk_select_ragged(sc, T, B * H_idx, G / rows, H_idx, T, plans, k_cols, km,
                                   out_idx, idx_dtype, ws_t, ws_t_bytes, stream);
      if (s != LAP_OK) return s;
    }
  }
  if (!plans) {
    if (k_eff > 0 && G == 4) {
      s = lap_retrieve_topk(lut_gmkg, codes, codes_stride_b, codes_stride_h, codes_stride_t, B,
                            Hkv, T, cand_start, cand_end, k_eff, key_mode, nullptr, out_idx,
                            idx_dtype, ws_r, cw.ret, stream);
      if (s != LAP_OK) return s;
    }
    return lap_sparse_attn_decode(q, q_sb, q_sh, keys, vals, dtype, B, Hq, Hkv, T_kv, D, k_sb,
                                  k_sh, k_st, v_sb, v_sh, v_st, out_idx, idx_dtype, H_idx, k_eff,
                                  sink_count, tail_start, tail_count, scale, out, ws_a, cw.attn,
                                  stream);
  }
  if (k_cols > 0 && G == 4) {
    s = lap_retrieve_topk_ragged(lut_gmkg, codes, codes_stride_b, codes_stride_h,
                                 codes_stride_t, B, Hkv, T, plans, k_cols, key_mode, nullptr,
                                 out_idx, idx_dtype, ws_r, cw.ret, stream);
    if (s != LAP_OK) return s;
  }
  return lap_sparse_attn_decode_ragged(q, q_sb, q_sh, keys, vals, dtype, B, Hq, Hkv, T_kv, D,
                                       k_sb, k_sh, k_st, v_sb, v_sh, v_st, out_idx, idx_dtype,
                                       H_idx, k_cols, plans, max_sink, max_tail, scale, out, ws_a,
                                       cw.attn, stream);
}

}  // namespace

extern "C" int lap_decode_step_workspace_size(int B, int Hq, int Hkv, int T, int D, int keep_max,
                                              int key_mode, size_t* bytes) {
  clear_error();
  LAP_CHECK(bytes, "lap_decode_step_workspace_size: null output");
  LAP_CHECK(B > 0 && Hq > 0 && Hkv > 0 && T >= 0 && D > 0 && keep_max >= 0,
            "lap_decode_step_workspace_size: bad sizes");
  ChainWs cw;
  int s = chain_ws(B, Hq, Hkv, T, D, keep_max, key_mode, &cw);
  if (s != LAP_OK) return s;
  const size_t fused = align_up(decode_step_fused_bytes(B * Hkv, T, kHeadRows), 256);
  *bytes = fused + cw.ret + cw.attn;
  return LAP_OK;
}

extern "C" int lap_decode_step_status(const void* workspace, size_t workspace_bytes,
                                      uint32_t* split_rows, uint32_t* timeouts) {
  clear_error();
  LAP_CHECK(workspace && split_rows && timeouts, "lap_decode_step_status: null pointer");
  LAP_CHECK(workspace_bytes >= 8, "lap_decode_step_status: workspace too small");
  uint32_t h[2] = {0, 0};
  LAP_HIP(hipMemcpy(h, workspace, sizeof(h), hipMemcpyDeviceToHost), "status copy");
  *split_rows = h[0];
  *timeouts = h[1];
  return LAP_OK;
}

extern "C" int lap_decode_step(
    const void* lut_gmkg, const uint8_t* codes, int64_t codes_stride_b, int64_t codes_stride_h,
    int64_t codes_stride_t, int T, int cand_start, int cand_end, int k, int sink_count,
    int tail_start, int tail_count, const lap_row_plan* plans, int k_cols, int max_sink,
    int max_tail, int key_mode, const void* q, int64_t q_sb, int64_t q_sh, const void* keys,
    const void* vals, int dtype, int B, int Hq, int Hkv, int T_kv, int D, int64_t k_sb,
    int64_t k_sh, int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st, float scale,
    void* out_idx, int idx_dtype, void* out, void* workspace, size_t workspace_bytes,
    lap_stream_t stream) {
  clear_error();
  return decode_step_run("lap_decode_step", lut_gmkg, codes, codes_stride_b, codes_stride_h,
                         codes_stride_t, T, cand_start, cand_end, k, sink_count, tail_start,
                         tail_count, plans, k_cols, max_sink, max_tail, key_mode, q, q_sb, q_sh,
                         keys, vals, dtype, B, Hq, Hkv, T_kv, D, k_sb, k_sh, k_st, v_sb, v_sh,
                         v_st, scale, out_idx, idx_dtype, out, workspace, workspace_bytes,
                         kHeadRows, true, stream);
}

// ------------------------------------------------------------------------
// lap_decode_step_noalloc: the same step on a static per-device scratch
// array instead of a caller workspace, for callers that may not allocate.
//
// `scratch` is one file-scope device array; every GPU the library runs on
// holds its own copy (at its own address) until the process ends.  In host
// code its name is only a stand-in, so host code uses the address that
// hipGetSymbolAddress returns for the current device, taken once per device
// at the first call there.  Its persistent head (status words, row
// barriers, row histograms) is laid out for kScratchRows rows, so calls of
// any shape find those words in place; the fused kernel leaves them zeroed
// (counters at multiples of their per-call advance), and the first call on
// a device clears them with a fill kernel on the call's stream.
namespace {

constexpr size_t kScratchBytes = (size_t)64 << 20;
constexpr int kScratchRows = kHeadRows;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ void scratch_clear_kernel(uint4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

std::mutex g_scratch_mu;
void* g_scratch_dev[64];

int scratch_clear_head(void* p, hipStream_t st) {
  const size_t head = carve_step(nullptr, kScratchRows, 0, kScratchRows).bytes;
  hipLaunchKernelGGL(scratch_clear_kernel, dim3(64), dim3(256), 0, st, static_cast<uint4*>(p),
                     head / 16);
  LAP_LAUNCH_CHECK("scratch_clear_kernel");
  return LAP_OK;
}

int scratch_for_device(hipStream_t st, void** out) {
  int dev = 0;
  LAP_HIP(hipGetDevice(&dev), "hipGetDevice");
  LAP_CHECK_CODE(dev >= 0 && dev < 64, LAP_ERR_UNSUPPORTED, "device ordinal %d out of range",
                 dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    LAP_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    LAP_CHECK_CODE(p && (reinterpret_cast<uintptr_t>(p) & 255) == 0, LAP_ERR_HIP,
                   "scratch symbol address %p is not 256-byte aligned", p);
    const int s = scratch_clear_head(p, st);
    if (s != LAP_OK) return s;
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return LAP_OK;
}

}  // namespace

extern "C" int lap_decode_step_noalloc(
    const void* lut_gmkg, const uint8_t* codes, int64_t codes_stride_b, int64_t codes_stride_h,
    int64_t codes_stride_t, int T, int cand_start, int cand_end, int k, int sink_count,
    int tail_start, int tail_count, const lap_row_plan* plans, int k_cols, int max_sink,
    int max_tail, int key_mode, const void* q, int64_t q_sb, int64_t q_sh, const void* keys,
    const void* vals, int dtype, int B, int Hq, int Hkv, int T_kv, int D, int64_t k_sb,
    int64_t k_sh, int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st, float scale,
    void* out_idx, int idx_dtype, void* out, lap_stream_t stream) {
  clear_error();
  const char* who = "lap_decode_step_noalloc";
  LAP_CHECK(B > 0 && Hkv > 0, "%s: bad sizes", who);
  LAP_CHECK_CODE((int64_t)B * Hkv <= kScratchRows, LAP_ERR_WORKSPACE,
                 "%s: %d x %d KV rows exceed the static scratch's %d rows", who, B, Hkv,
                 kScratchRows);
  void* p = nullptr;
  int s = scratch_for_device(as_stream(stream), &p);
  if (s != LAP_OK) return s;
  s = decode_step_run(who, lut_gmkg, codes, codes_stride_b, codes_stride_h, codes_stride_t, T,
                      cand_start, cand_end, k, sink_count, tail_start, tail_count, plans, k_cols,
                      max_sink, max_tail, key_mode, q, q_sb, q_sh, keys, vals, dtype, B, Hq, Hkv,
                      T_kv, D, k_sb, k_sh, k_st, v_sb, v_sh, v_st, scale, out_idx, idx_dtype, out,
                      p, kScratchBytes, kScratchRows, false, stream);
  if (s == LAP_ERR_WORKSPACE)
    set_error("%s: this shape needs more than the static scratch of %zu bytes (%s)", who,
              kScratchBytes, lap_last_error());
  return s;
}

// Health counters of the static scratch on the current device (the same
// two words lap_decode_step_status reads from a workspace), after the device
// has finished its work; zeros before the first call on the device.
extern "C" int lap_decode_step_noalloc_status(uint32_t* split_rows, uint32_t* timeouts) {
  clear_error();
  LAP_CHECK(split_rows && timeouts, "lap_decode_step_noalloc_status: null pointer");
  void* p = nullptr;
  int s = scratch_for_device(nullptr, &p);
  if (s != LAP_OK) return s;
  LAP_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
  uint32_t h[2] = {0, 0};
  LAP_HIP(hipMemcpy(h, p, sizeof(h), hipMemcpyDeviceToHost), "status copy");
  *split_rows = h[0];
  *timeouts = h[1];
  return LAP_OK;
}

// Zero the static scratch's persistent head (counters, row barriers, row
// histograms) on the current device with a fill kernel on `stream`: the
// reset after an unhealthy call.  Allocates nothing.
extern "C" int lap_decode_step_noalloc_reset(lap_stream_t stream) {
  clear_error();
  void* p = nullptr;
  int s = scratch_for_device(as_stream(stream), &p);
  if (s != LAP_OK) return s;
  return scratch_clear_head(p, as_stream(stream));
}

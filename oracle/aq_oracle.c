/*
 * aq_oracle.c — CPU oracle for the decode-time retrieval path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain scalar C with an
 * explicit arithmetic order, what each hot-path function of LAPrune computes,
 * so that the gfx950 kernels can be checked bit for bit.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product path never does.  Build: oracle/build.py (gcc -O2
 * -ffp-contract=off), output oracle/_build/liboracle.so.
 *
 * Each function names the reference code it restates (paths relative to the
 * LAPrune tree).  How each function is pinned (closed forms, brute force,
 * independent numpy restatements) is listed in oracle/orc.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ fp16/bf16 */

/* fp16 bits -> float (exact). */
float orc_h2f(uint16_t h) {
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m | 0x400u), (int)e - 25);
  return (h & 0x8000u) ? -v : v;
}

/* float -> fp16 bits, round to nearest even (IEEE 754 binary16). */
uint16_t orc_f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return sign | 0x7e00u;  /* NaN */
  if (ax == 0x7f800000u) return sign | 0x7c00u; /* inf */
  if ((ax >> 23) == 0) return sign;             /* float subnormal -> 0 */
  const int e = (int)(ax >> 23) - 127;
  if (e >= 16) return sign | 0x7c00u;
  const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
  const int shift = e >= -14 ? 13 : 13 + (-14 - e);
  if (shift >= 25) return sign;
  uint32_t kept = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (kept & 1u))) kept++;
  if (e >= -14) {
    uint32_t eh = (uint32_t)(e + 15);
    if (kept == 0x800u) {
      kept = 0x400u;
      eh++;
    }
    if (eh >= 31) return sign | 0x7c00u;
    return (uint16_t)(sign | (eh << 10) | (kept & 0x3ffu));
  }
  return (uint16_t)(sign | kept);
}

/* float -> bf16 bits, round to nearest even. */
uint16_t orc_f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* ---------------------------------------------------------------- A1 LUT */

/* lut[h,m,k] = fp16(fmaf chain over d of q[h,d]*C[m,k,d]), layout [Hq][M][K].
 * Restates laprune/llm/aq_kv.py:681-682 / :620 with the explicit order. */
void orc_lut_build(const float* q, const float* cb, int Hq, int D, int M, int K,
                   uint16_t* out) {
  const int MK = M * K;
  for (int h = 0; h < Hq; ++h)
    for (int r = 0; r < MK; ++r) {
      float acc = 0.f;
      const float* qr = q + (int64_t)h * D;
      const float* c = cb + (int64_t)r * D;
      for (int d = 0; d < D; ++d) acc = fmaf(qr[d], c[d], acc);
      out[(int64_t)h * MK + r] = orc_f2h(acc);
    }
}

/* ------------------------------------------------------------- A2 scores */

/* Grouped scorer, aq_kernels/aq_lut_gqa.cu:111-149 / :157-212:
 * out[hkv*G+g, t] = fp16( sum_m (float)lut[(hkv*G+g), m, code] ), m ascending. */
void orc_score_grouped(const uint16_t* lut, const uint8_t* codes, int64_t cs_h, int64_t cs_t,
                       int Hkv, int G, int T, int M, int K, uint16_t* out) {
  for (int hkv = 0; hkv < Hkv; ++hkv)
    for (int g = 0; g < G; ++g) {
      const int h = hkv * G + g;
      const uint16_t* L = lut + (int64_t)h * M * K;
      for (int t = 0; t < T; ++t) {
        const uint8_t* cp = codes + (int64_t)hkv * cs_h + (int64_t)t * cs_t;
        float acc = 0.f;
        for (int m = 0; m < M; ++m) acc = acc + orc_h2f(L[m * K + cp[m]]);
        out[(int64_t)h * T + t] = orc_f2h(acc);
      }
    }
}

/* aq_kernels/aq_lut_gqa.cu:20-76: M sub-range, dense or indexed; an index
 * outside [0,T) scores 0. */
void orc_score_gqa(const uint16_t* lut, const uint8_t* codes, int64_t cs_h, int64_t cs_t,
                   int Hkv, int G, int T, int M_stride, int K, int M_start, int M_end,
                   const int64_t* indices, int N, uint16_t* out) {
  const int H = Hkv * G;
  for (int h = 0; h < H; ++h) {
    const int hkv = h / G;
    const uint16_t* L = lut + ((int64_t)h * M_stride + M_start) * K;
    for (int n = 0; n < N; ++n) {
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
      for (int m = 0; m < M_end - M_start; ++m) acc = acc + orc_h2f(L[m * K + cp[m]]);
      out[(int64_t)h * N + n] = orc_f2h(acc);
    }
  }
}

/* aq_kernels/aq_lut.cu:581-639: codes given as int64 (any source dtype,
 * sign-extended); the low 8 bits are the code, clamped to K-1.
 * lut_f32 != 0: fp32 LUT and fp32 output (float*), else fp16 bits. */
void orc_score_mha(const void* lut, int lut_f32, const int64_t* codes, int Q, int N, int M,
                   int K, void* out) {
  for (int q = 0; q < Q; ++q)
    for (int n = 0; n < N; ++n) {
      const int64_t* cp = codes + ((int64_t)q * N + n) * M;
      float acc = 0.f;
      for (int m = 0; m < M; ++m) {
        int c = (int)(uint8_t)(cp[m] & 0xff);
        if (c >= K) c = K - 1;
        const int64_t at = (int64_t)q * M * K + (int64_t)m * K + c;
        acc = acc + (lut_f32 ? ((const float*)lut)[at] : orc_h2f(((const uint16_t*)lut)[at]));
      }
      if (lut_f32) ((float*)out)[(int64_t)q * N + n] = acc;
      else ((uint16_t*)out)[(int64_t)q * N + n] = orc_f2h(acc);
    }
}

/* laprune/llm/aq_kv.py:431-457 (AQLayerCodebookManager.reconstruct):
 * recon = zeros; for m ascending: recon += C[m][codes[:, m]], elementwise in
 * fp32.  codes [N][M] as int64 (any source dtype); the low 8 bits are the
 * code, clamped to K-1 (the reference indexes with the code directly: a code
 * >= K is an indexing error there). */
void orc_reconstruct(const float* cb, const int64_t* codes, int N, int M, int K, int D,
                     float* out) {
  for (int n = 0; n < N; ++n) {
    float* o = out + (int64_t)n * D;
    for (int d = 0; d < D; ++d) o[d] = 0.f;
    for (int m = 0; m < M; ++m) {
      int c = (int)(uint8_t)(codes[(int64_t)n * M + m] & 0xff);
      if (c >= K) c = K - 1;
      const float* row = cb + ((int64_t)m * K + c) * D;
      for (int d = 0; d < D; ++d) o[d] = o[d] + row[d];
    }
  }
}

/* aq_kernels/aq_lut.cu:37-149 direct scoring.  f32: one fmaf chain over
 * (m, d); f16 (is_f16 != 0, q/cb given as fp16 bits): per pair
 * p = fp16(q*c) lanewise, acc += (p0 + p1).  Codes >= K are skipped. */
void orc_aq_direct(const void* q, const void* cb, int is_f16, const int64_t* codes, int Q,
                   int N, int M, int K, int D, void* out) {
  for (int qi = 0; qi < Q; ++qi)
    for (int n = 0; n < N; ++n) {
      const int64_t* cp = codes + ((int64_t)qi * N + n) * M;
      float acc = 0.f;
      for (int m = 0; m < M; ++m) {
        const int c = (int)(uint8_t)(cp[m] & 0xff);
        if (c >= K) continue;
        const int64_t row = ((int64_t)m * K + c) * D;
        if (!is_f16) {
          const float* qq = (const float*)q + (int64_t)qi * D;
          const float* cc = (const float*)cb + row;
          for (int i = 0; i < D; ++i) acc = fmaf(qq[i], cc[i], acc);
        } else {
          const uint16_t* qq = (const uint16_t*)q + (int64_t)qi * D;
          const uint16_t* cc = (const uint16_t*)cb + row;
          int i = 0;
          for (; i + 1 < D; i += 2) {
            const float p0 = orc_h2f(orc_f2h(orc_h2f(qq[i]) * orc_h2f(cc[i])));
            const float p1 = orc_h2f(orc_f2h(orc_h2f(qq[i + 1]) * orc_h2f(cc[i + 1])));
            acc = acc + (p0 + p1);
          }
          for (; i < D; ++i) acc = acc + orc_h2f(qq[i]) * orc_h2f(cc[i]);
        }
      }
      if (!is_f16) ((float*)out)[(int64_t)qi * N + n] = acc;
      else ((uint16_t*)out)[(int64_t)qi * N + n] = orc_f2h(acc);
    }
}

/* ---------------------------------------------------------------- A3 top-k */

static uint32_t key16(uint16_t h) {
  if ((h & 0x7fffu) == 0) h = 0;
  return (h & 0x8000u) ? (~(uint32_t)h & 0xffffu) : ((uint32_t)h | 0x8000u);
}

/* Selection of aq_evaluation.py:198-201 with a fixed tie rule: per row r,
 * key = max over g of key(score[r*group+g, t]) (key_bf16: ranked as
 * bf16(fp16 score)); keep the k largest over t in [cand_start, cand_end),
 * lowest t first among equal keys; write them ascending to out[r*k ...].
 * Returns k_eff = min(k, n). */
int orc_topk(const uint16_t* scores, int64_t row_stride, int R, int group, int cand_start,
             int cand_end, int k, int key_bf16, int64_t* out) {
  const int n = cand_end - cand_start;
  const int ke = k < n ? k : n;
  if (ke <= 0) return 0;
  uint32_t* keys = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)n);
  uint32_t* hist = (uint32_t*)malloc(sizeof(uint32_t) * 65536);
  for (int r = 0; r < R; ++r) {
    memset(hist, 0, sizeof(uint32_t) * 65536);
    for (int e = 0; e < n; ++e) {
      uint32_t best = 0;
      for (int g = 0; g < group; ++g) {
        uint16_t h = scores[(int64_t)(r * group + g) * row_stride + cand_start + e];
        if (key_bf16) h = orc_f2bf(orc_h2f(h));
        const uint32_t kk = key16(h);
        if (kk > best) best = kk;
      }
      keys[e] = best;
      hist[best]++;
    }
    /* threshold: largest tau with count(key >= tau) >= ke */
    uint32_t above = 0;
    int tau = 65535;
    for (; tau >= 0; --tau) {
      if (above + hist[tau] >= (uint32_t)ke) break;
      above += hist[tau];
    }
    uint32_t need = (uint32_t)ke - above, taken = 0;
    int w = 0;
    for (int e = 0; e < n; ++e) {
      if (keys[e] > (uint32_t)tau || (keys[e] == (uint32_t)tau && taken < need)) {
        if (keys[e] == (uint32_t)tau) taken++;
        out[(int64_t)r * k + w++] = cand_start + e;
      }
    }
  }
  free(keys);
  free(hist);
  return ke;
}

/* -------------------------------------------------------------- A6 encode */

/* dot16: 16 fmaf chains over consecutive blocks of L = D/16, folded
 * s[j] += s[j+w] for w = 8, 4, 2, 1. */
float orc_dot16(const float* a, const float* b, int D) {
  const int L = D / 16;
  float s[16];
  for (int j = 0; j < 16; ++j) {
    float acc = 0.f;
    for (int t = 0; t < L; ++t) acc = fmaf(a[j * L + t], b[j * L + t], acc);
    s[j] = acc;
  }
  for (int w = 8; w >= 1; w >>= 1)
    for (int j = 0; j < w; ++j) s[j] = s[j] + s[j + w];
  return s[0];
}

/* Greedy AQ encode, laprune/quantizer.py:346-355 with iters = 0:
 *   dist_k = (rn + cn[m,k]) - 2*dot(r, C[m,k]); code = first argmin;
 *   r -= C[m,code].  All dots by orc_dot16.  rnorm = sqrtf(dot16(r,r)).
 * Optional trace (may be NULL): dists of every stage, [N][M][K]. */
void orc_encode(const float* x, const float* cb, int N, int M, int K, int D, uint8_t* codes,
                float* rnorm, float* trace) {
  float* cn = (float*)malloc(sizeof(float) * (size_t)M * K);
  float* r = (float*)malloc(sizeof(float) * (size_t)D);
  for (int i = 0; i < M * K; ++i) cn[i] = orc_dot16(cb + (int64_t)i * D, cb + (int64_t)i * D, D);
  for (int n = 0; n < N; ++n) {
    memcpy(r, x + (int64_t)n * D, sizeof(float) * (size_t)D);
    for (int m = 0; m < M; ++m) {
      const float rn = orc_dot16(r, r, D);
      float best = INFINITY;
      int bk = 0;
      for (int k = 0; k < K; ++k) {
        const float* c = cb + ((int64_t)m * K + k) * D;
        const float dist = (rn + cn[m * K + k]) - 2.0f * orc_dot16(r, c, D);
        if (trace) trace[((int64_t)n * M + m) * K + k] = dist;
        if (dist < best) {
          best = dist;
          bk = k;
        }
      }
      codes[(int64_t)n * M + m] = (uint8_t)bk;
      const float* c = cb + ((int64_t)m * K + bk) * D;
      for (int d = 0; d < D; ++d) r[d] = r[d] - c[d];
    }
    if (rnorm) rnorm[n] = sqrtf(orc_dot16(r, r, D));
  }
  free(cn);
  free(r);
}

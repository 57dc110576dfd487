// cache.hip — N1/N2: the decode step's writes into the device-resident cache.
//
// lap_rope_append applies the rotary embedding to the step's query and key
// (HF apply_rotary_pos_emb as aq_evaluation.py:296-305 calls it, the
// rotate_half convention) and writes the rotated key and the value of one
// token per sequence into the K/V capacity buffers at device positions
// (the cache write of _kv_cache_append, aq_evaluation.py:65-112), in one
// launch instead of about a dozen element-wise kernels per layer.
//
// Arithmetic matches torch's element-wise ops in the model dtype: each
// product and the sum are computed in fp32 and rounded to the dtype,
//     out = rnd(rnd(x * cos) + rnd(rotate_half(x) * sin)),
// rotate_half(x) = cat(-x[D/2:], x[:D/2]), so the rotated tensors are
// bit-identical to the reference's.
#include "common.h"

namespace lap {
namespace {

template <int DT>
__device__ __forceinline__ float ld(const uint16_t* p, int64_t i) {
  return DT == LAP_DTYPE_F16 ? h2f(p[i]) : bf2f(p[i]);
}
template <int DT>
__device__ __forceinline__ uint16_t rnd(float f) {
  return DT == LAP_DTYPE_F16 ? f2h(f) : f2bf(f);
}
template <int DT>
__device__ __forceinline__ float rf(float f) {  // f rounded to the dtype, as fp32
  return DT == LAP_DTYPE_F16 ? h2f(f2h(f)) : bf2f(f2bf(f));
}

struct RopeArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* k;
  int64_t k_sb, k_sh;
  const uint16_t* v;
  int64_t v_sb, v_sh;
  const uint16_t* cos;
  const uint16_t* sin;
  int64_t cs_sb;
  int Hq, Hkv, D;
  const int64_t* pos;
  uint16_t* ck;
  int64_t ck_sb, ck_sh, ck_st;
  uint16_t* cv;
  int64_t cv_sb, cv_sh, cv_st;
  int t_cap;
  uint16_t* q_out;
};

// Workgroup (b, r): r < Hq rotates query head r into q_out; r >= Hq rotates
// key head r - Hq into the cache and copies its value row.  Thread i owns
// the rotation pair (i, i + D/2).
template <int DT>
__global__ __launch_bounds__(128) void rope_append_kernel(RopeArgs a) {
  const int b = blockIdx.x / (a.Hq + a.Hkv), r = blockIdx.x % (a.Hq + a.Hkv);
  const int i = threadIdx.x, h2 = a.D / 2;
  if (i >= h2) return;
  const uint16_t* cs = a.cos + (int64_t)b * a.cs_sb;
  const uint16_t* sn = a.sin + (int64_t)b * a.cs_sb;
  const float c0 = ld<DT>(cs, i), c1 = ld<DT>(cs, i + h2);
  const float s0 = ld<DT>(sn, i), s1 = ld<DT>(sn, i + h2);
  const uint16_t* x;
  uint16_t* dst;
  if (r < a.Hq) {
    x = a.q + (int64_t)b * a.q_sb + (int64_t)r * a.q_sh;
    dst = a.q_out + ((int64_t)b * a.Hq + r) * a.D;
  } else {
    const int h = r - a.Hq;
    const int64_t t = a.pos[b];
    if (t < 0 || t >= a.t_cap) return;  // outside the capacity buffer: no write
    x = a.k + (int64_t)b * a.k_sb + (int64_t)h * a.k_sh;
    dst = a.ck + (int64_t)b * a.ck_sb + (int64_t)h * a.ck_sh + t * a.ck_st;
    const uint16_t* vs = a.v + (int64_t)b * a.v_sb + (int64_t)h * a.v_sh;
    uint16_t* vd = a.cv + (int64_t)b * a.cv_sb + (int64_t)h * a.cv_sh + t * a.cv_st;
    vd[i] = vs[i];
    vd[i + h2] = vs[i + h2];
  }
  const float x0 = ld<DT>(x, i), x1 = ld<DT>(x, i + h2);
  dst[i] = rnd<DT>(rf<DT>(x0 * c0) + rf<DT>(-x1 * s0));
  dst[i + h2] = rnd<DT>(rf<DT>(x1 * c1) + rf<DT>(x0 * s1));
}

}  // namespace
}  // namespace lap

using namespace lap;

extern "C" int lap_rope_append(const void* q, int64_t q_sb, int64_t q_sh, const void* k,
                               int64_t k_sb, int64_t k_sh, const void* v, int64_t v_sb,
                               int64_t v_sh, const void* cos, const void* sin, int64_t cs_sb,
                               int dtype, int B, int Hq, int Hkv, int D, const int64_t* pos,
                               void* cache_k, int64_t ck_sb, int64_t ck_sh, int64_t ck_st,
                               void* cache_v, int64_t cv_sb, int64_t cv_sh, int64_t cv_st,
                               int t_cap, void* q_out, lap_stream_t stream) {
  clear_error();
  LAP_CHECK(q && k && v && cos && sin && pos && cache_k && cache_v && q_out,
            "lap_rope_append: null pointer");
  LAP_CHECK(dtype == LAP_DTYPE_F16 || dtype == LAP_DTYPE_BF16,
            "lap_rope_append: dtype must be fp16/bf16");
  LAP_CHECK(B > 0 && Hq > 0 && Hkv > 0 && t_cap > 0, "lap_rope_append: bad sizes");
  LAP_CHECK(D > 0 && D % 2 == 0 && D <= 256, "lap_rope_append: D=%d must be even and <= 256", D);
  LAP_CHECK(q_sh >= D && k_sh >= D && v_sh >= D && cs_sb >= D && ck_st >= D && cv_st >= D,
            "lap_rope_append: strides smaller than D");
  RopeArgs a{static_cast<const uint16_t*>(q), q_sb, q_sh, static_cast<const uint16_t*>(k),
             k_sb, k_sh, static_cast<const uint16_t*>(v), v_sb, v_sh,
             static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin), cs_sb, Hq,
             Hkv, D, pos, static_cast<uint16_t*>(cache_k), ck_sb, ck_sh, ck_st,
             static_cast<uint16_t*>(cache_v), cv_sb, cv_sh, cv_st, t_cap,
             static_cast<uint16_t*>(q_out)};
  const dim3 grid((unsigned)(B * (Hq + Hkv)));
  hipStream_t st = as_stream(stream);
  if (dtype == LAP_DTYPE_F16)
    hipLaunchKernelGGL(rope_append_kernel<LAP_DTYPE_F16>, grid, dim3(128), 0, st, a);
  else
    hipLaunchKernelGGL(rope_append_kernel<LAP_DTYPE_BF16>, grid, dim3(128), 0, st, a);
  LAP_LAUNCH_CHECK("rope_append_kernel");
  return LAP_OK;
}

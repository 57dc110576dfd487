// gather.hip — A4: native-GQA K/V row gather into per-query-head tensors.
//
// Drop-in for gqa_gather_kv / gqa_gather_kv_with_tail
// (aq_kernels/aq_lut_gqa.cu:536-664): out[b,hq,n,:] = K[b, hq/G, t_n, :] with
// t_n = indices[b,hq,n] for n < explicit_N and t_n = tail_start + (n -
// explicit_N) for the implicit tail; rows whose t_n lies outside [0,T) are
// left unwritten.  fp16 and bf16 are both served (bytes are copied).
//
// One workgroup copies a run of rows of one (b, hq); each lane moves 16
// bytes, so a 256-byte row (D = 128) is 16 lanes and a 256-thread workgroup
// moves 16 rows per pass for K and V.
#include "common.h"

namespace lap {
namespace {

template <int VEC>  // bytes per lane: 16, 4 or 2
__global__ __launch_bounds__(256) void gather_kv_kernel(
    const char* __restrict__ keys, const char* __restrict__ vals, int Hkv, int Hq, int T,
    int row_bytes, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t v_sb, int64_t v_sh,
    int64_t v_st, const int64_t* __restrict__ idx, int explicit_N, int tail_start, int N,
    int rows_per_block, char* __restrict__ out_k, char* __restrict__ out_v) {
  const int bh = blockIdx.x;
  const int b = bh / Hq, hq = bh - b * Hq;
  const int G = Hq / Hkv;
  const int hkv = hq / G;
  const int lanes_per_row = row_bytes / VEC;
  const int slot = threadIdx.x / lanes_per_row;
  const int part = threadIdx.x - slot * lanes_per_row;
  if (slot >= rows_per_block) return;
  const int n = blockIdx.y * rows_per_block + slot;
  if (n >= N) return;
  int64_t t;
  if (n < explicit_N) t = idx[(int64_t)bh * explicit_N + n];
  else t = (int64_t)tail_start + (n - explicit_N);
  if (t < 0 || t >= T) return;
  const int64_t ko = (int64_t)b * k_sb + (int64_t)hkv * k_sh + t * k_st + (int64_t)part * VEC;
  const int64_t vo = (int64_t)b * v_sb + (int64_t)hkv * v_sh + t * v_st + (int64_t)part * VEC;
  const int64_t oo = ((int64_t)bh * N + n) * row_bytes + (int64_t)part * VEC;
  if (VEC == 16) {
    *reinterpret_cast<uint4*>(out_k + oo) = *reinterpret_cast<const uint4*>(keys + ko);
    *reinterpret_cast<uint4*>(out_v + oo) = *reinterpret_cast<const uint4*>(vals + vo);
  } else if (VEC == 4) {
    *reinterpret_cast<uint32_t*>(out_k + oo) = *reinterpret_cast<const uint32_t*>(keys + ko);
    *reinterpret_cast<uint32_t*>(out_v + oo) = *reinterpret_cast<const uint32_t*>(vals + vo);
  } else {
    *reinterpret_cast<uint16_t*>(out_k + oo) = *reinterpret_cast<const uint16_t*>(keys + ko);
    *reinterpret_cast<uint16_t*>(out_v + oo) = *reinterpret_cast<const uint16_t*>(vals + vo);
  }
}

bool al(const void* p, int a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace
}  // namespace lap

using namespace lap;

extern "C" int lap_gqa_gather_kv(const void* keys, const void* vals, int dtype, int B, int Hkv,
                                 int T, int D, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                 int64_t v_sb, int64_t v_sh, int64_t v_st,
                                 const int64_t* indices, int Hq, int explicit_N, int tail_start,
                                 int tail_count, void* out_k, void* out_v,
                                 lap_stream_t stream) {
  clear_error();
  LAP_CHECK(keys && vals && out_k && out_v, "lap_gqa_gather_kv: null pointer");
  LAP_CHECK(dtype == LAP_DTYPE_F16 || dtype == LAP_DTYPE_BF16,
            "gqa_gather_kv supports fp16/bf16 K/V");
  LAP_CHECK(B > 0 && Hkv > 0 && Hq > 0 && T >= 0 && D > 0, "lap_gqa_gather_kv: bad sizes");
  LAP_CHECK(Hq % Hkv == 0, "Hq must equal Hkv * G");
  LAP_CHECK(D % 2 == 0, "D must be positive and even");
  LAP_CHECK(explicit_N >= 0 && tail_count >= 0, "lap_gqa_gather_kv: negative counts");
  LAP_CHECK(explicit_N == 0 || indices, "lap_gqa_gather_kv: indices required");
  if (tail_start < 0) LAP_CHECK(tail_count == 0, "lap_gqa_gather_kv: tail_count without tail");
  else LAP_CHECK(tail_start + tail_count <= T, "invalid implicit tail range");
  const int N = explicit_N + tail_count;
  if (N == 0) return LAP_OK;
  const int es = 2;
  const int row_bytes = D * es;
  const char* K = static_cast<const char*>(keys);
  const char* V = static_cast<const char*>(vals);
  char* OK_ = static_cast<char*>(out_k);
  char* OV = static_cast<char*>(out_v);
  auto strides_ok = [&](int64_t a) {
    return (k_sb * es) % a == 0 && (k_sh * es) % a == 0 && (k_st * es) % a == 0 &&
           (v_sb * es) % a == 0 && (v_sh * es) % a == 0 && (v_st * es) % a == 0;
  };
  int vec = 2;
  if (row_bytes % 16 == 0 && strides_ok(16) && al(K, 16) && al(V, 16) && al(OK_, 16) &&
      al(OV, 16) && row_bytes / 16 <= 256)
    vec = 16;
  else if (row_bytes % 4 == 0 && strides_ok(4) && al(K, 4) && al(V, 4) && al(OK_, 4) &&
           al(OV, 4) && row_bytes / 4 <= 256)
    vec = 4;
  LAP_CHECK_CODE(row_bytes / vec <= 256, LAP_ERR_UNSUPPORTED, "lap_gqa_gather_kv: D too large");
  const int lanes = row_bytes / vec;
  const int rows_per_block = 256 / lanes;
  dim3 grid(B * Hq, (N + rows_per_block - 1) / rows_per_block);
  hipStream_t st = as_stream(stream);
#define LAP_GATHER(V_)                                                                      \
  hipLaunchKernelGGL(gather_kv_kernel<V_>, grid, dim3(256), 0, st, K, V, Hkv, Hq, T,        \
                     row_bytes, k_sb * es, k_sh * es, k_st * es, v_sb * es, v_sh * es,      \
                     v_st * es, indices, explicit_N, tail_start, N, rows_per_block, OK_, OV)
  if (vec == 16) LAP_GATHER(16);
  else if (vec == 4) LAP_GATHER(4);
  else LAP_GATHER(2);
#undef LAP_GATHER
  LAP_LAUNCH_CHECK("gather_kv_kernel");
  return LAP_OK;
}

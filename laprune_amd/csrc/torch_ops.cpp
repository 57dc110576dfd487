// torch_ops.cpp — compiled torch binding of the decode path's hot entry
// points: torch custom ops (namespace `laprune`) registered for the GPU
// dispatch key, each a thin call into the C ABI of liblaprune_hip.so.
//
// The reference binds every kernel file as a compiled pybind module and calls
// it eagerly once per layer per token (aq_kernels/aq_lut_gqa.cu:670-691,
// aq_lut.cu:741-745, fused_linear_encode.cu:237-242; called from
// laprune/llm/modifiers/aq_evaluation.py:165-251).  These ops serve that
// eager pattern: sizes and strides come from the tensors, the stream is the
// current torch stream of the tensors' device, and a failing C-ABI call
// raises with lap_last_error()'s message.  Host code only (no kernels here);
// built with hipcc against the torch headers, linked to the HIP library.
#include <torch/library.h>
#include <ATen/core/Tensor.h>
#include <c10/hip/HIPStream.h>

#include <algorithm>
#include <cmath>
#include <optional>

#include "../../include/laprune_hip.h"

namespace {

int dtype_code(const at::Tensor& t) {
  switch (t.scalar_type()) {
    case at::kFloat: return LAP_DTYPE_F32;
    case at::kHalf: return LAP_DTYPE_F16;
    case at::kBFloat16: return LAP_DTYPE_BF16;
    case at::kByte: return LAP_DTYPE_U8;
    case at::kChar: return LAP_DTYPE_I8;
    case at::kInt: return LAP_DTYPE_I32;
    case at::kLong: return LAP_DTYPE_I64;
    default: TORCH_CHECK(false, "laprune: dtype ", t.scalar_type(), " is not served");
  }
  return -1;
}

lap_stream_t stream_of(const at::Tensor& t) {
  return static_cast<lap_stream_t>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check(int status, const char* fn) {
  TORCH_CHECK(status == LAP_OK, fn, ": ", lap_last_error());
}

void* ptr(const at::Tensor& t) { return t.data_ptr(); }
void* ptr(const std::optional<at::Tensor>& t) { return t ? t->data_ptr() : nullptr; }

// Every tensor of a call on the GPU, on one device: the dispatcher routes a
// call with any GPU tensor here, and a host pointer handed to a kernel
// would fault.
void same_gpu(const char* op, std::initializer_list<const at::Tensor*> ts) {
  const at::Tensor* first = nullptr;
  for (const at::Tensor* t : ts) {
    if (!t) continue;
    TORCH_CHECK(t->is_cuda(), op, ": every tensor must be on the GPU");
    if (!first) first = t;
    TORCH_CHECK(t->device() == first->device(), op, ": tensors on different devices");
  }
}
const at::Tensor* opt(const std::optional<at::Tensor>& t) { return t ? &*t : nullptr; }

// q [Hq, D] (row stride free), codebooks [M, K, D] contiguous -> out (fp16
// table, layout LAP_LUT_HMK or LAP_LUT_GMKG).  Replaces the reference's
// torch.matmul LUT (laprune/llm/aq_kv.py:681-682).
void lut_build(const at::Tensor& q, const at::Tensor& cb, int64_t G, int64_t layout,
               const at::Tensor& out) {
  TORCH_CHECK(q.dim() == 2 && cb.dim() == 3 && q.stride(1) == 1 && cb.is_contiguous() &&
                  out.is_contiguous(),
              "laprune::lut_build: q [Hq, D] with unit inner stride, contiguous codebooks and out");
  same_gpu("laprune::lut_build", {&q, &cb, &out});
  check(lap_lut_build(ptr(q), dtype_code(q), q.stride(0), ptr(cb), dtype_code(cb),
                      (int)q.size(0), (int)q.size(1), (int)cb.size(0), (int)cb.size(1), (int)G,
                      (int)layout, ptr(out), stream_of(q)),
        "lap_lut_build");
}

// One decode step after the LUT (lap_decode_step): codes [B, Hkv, >=T, M],
// q [B, Hq, D], keys / vals [B, Hkv, T_kv, D]; uniform scalars, or device
// plans (lap_row_plan [B], int32 x 8) with k_cols / max_sink / max_tail.
void decode_step(const at::Tensor& lut, const std::optional<at::Tensor>& codes, int64_t T,
                 int64_t cand_start, int64_t cand_end, int64_t k, int64_t sink,
                 int64_t tail_start, int64_t tail_count, const std::optional<at::Tensor>& plans,
                 int64_t k_cols, int64_t max_sink, int64_t max_tail, int64_t key_mode,
                 const at::Tensor& q, const at::Tensor& keys, const at::Tensor& vals,
                 double scale, const at::Tensor& idx, const at::Tensor& out,
                 const at::Tensor& ws) {
  TORCH_CHECK(q.dim() == 3 && keys.dim() == 4 && vals.dim() == 4,
              "laprune::decode_step: q [B, Hq, D], keys / vals [B, Hkv, T, D]");
  same_gpu("laprune::decode_step", {&lut, opt(codes), opt(plans), &q, &keys, &vals, &idx, &out, &ws});
  TORCH_CHECK(!codes || codes->scalar_type() == at::kByte, "laprune::decode_step: u8 codes");
  TORCH_CHECK(!plans || plans->scalar_type() == at::kInt, "laprune::decode_step: int32 plans");
  // Sizes the kernels index by, checked here so that a mis-sized tensor is
  // an error and never an out-of-bounds read or write.
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(2), Hkv = keys.size(1);
  TORCH_CHECK(keys.scalar_type() == q.scalar_type() && vals.scalar_type() == q.scalar_type() &&
                  out.scalar_type() == q.scalar_type(),
              "laprune::decode_step: q, keys, vals and out must share one dtype");
  TORCH_CHECK(keys.size(0) == B && vals.size(0) == B && vals.size(1) == Hkv &&
                  vals.size(2) >= keys.size(2) && keys.size(3) == D && vals.size(3) == D,
              "laprune::decode_step: keys / vals must be [B, Hkv, T_kv, D] of q's B and D");
  TORCH_CHECK(out.is_contiguous() && out.numel() >= B * Hq * D,
              "laprune::decode_step: out must be contiguous with at least B * Hq * D elements");
  TORCH_CHECK(Hkv > 0 && Hq % Hkv == 0, "laprune::decode_step: Hq must be a multiple of Hkv");
  TORCH_CHECK(lut.scalar_type() == at::kHalf && lut.is_contiguous() &&
                  lut.numel() >= B * Hq * 32 * 256,
              "laprune::decode_step: lut must be the contiguous fp16 table of B * Hq heads "
              "([B * Hkv, 32, 256, 4] for G = 4, else [B * Hq, 32, 256])");
  const int64_t rows = (key_mode & LAP_SELECT_PER_HEAD) ? Hq : Hkv;
  const int64_t cols = plans ? k_cols : std::max<int64_t>(0, std::min(k, cand_end - cand_start));
  if (cols > 0) {
    TORCH_CHECK(idx.is_contiguous() && idx.numel() >= B * rows * cols &&
                    (idx.scalar_type() == at::kInt || idx.scalar_type() == at::kLong),
                "laprune::decode_step: idx must be contiguous int32/int64 with at least "
                "B * rows * k elements");
    TORCH_CHECK(codes && codes->dim() == 4 && codes->size(0) == B && codes->size(1) == Hkv &&
                    codes->size(2) >= T && codes->size(3) == 32,
                "laprune::decode_step: codes must be [B, Hkv, >=T, 32]");
  }
  TORCH_CHECK(!plans || (plans->is_contiguous() && plans->numel() >= B * 8),
              "laprune::decode_step: plans must hold B lap_row_plan records (B x 8 int32)");
  TORCH_CHECK(ws.is_contiguous(), "laprune::decode_step: contiguous workspace");
  const int64_t cs_b = codes ? codes->stride(0) : 0, cs_h = codes ? codes->stride(1) : 0,
                cs_t = codes ? codes->stride(2) : 0;
  check(lap_decode_step(ptr(lut), codes ? static_cast<const uint8_t*>(codes->data_ptr()) : nullptr,
                        cs_b, cs_h, cs_t, (int)T, (int)cand_start, (int)cand_end, (int)k,
                        (int)sink, (int)tail_start, (int)tail_count,
                        static_cast<const lap_row_plan*>(ptr(plans)), (int)k_cols, (int)max_sink,
                        (int)max_tail, (int)key_mode, ptr(q), q.stride(0), q.stride(1),
                        ptr(keys), ptr(vals), dtype_code(q), (int)q.size(0), (int)q.size(1),
                        (int)keys.size(1), (int)keys.size(2), (int)q.size(2), keys.stride(0),
                        keys.stride(1), keys.stride(2), vals.stride(0), vals.stride(1),
                        vals.stride(2), (float)scale, ptr(idx), dtype_code(idx), ptr(out),
                        ptr(ws), (size_t)ws.numel() * ws.element_size(), stream_of(q)),
        "lap_decode_step");
}

// Dense split-K decode over all T keys (the comparator of record).
void dense_decode(const at::Tensor& q, const at::Tensor& keys, const at::Tensor& vals,
                  double scale, const at::Tensor& out, const at::Tensor& ws) {
  TORCH_CHECK(q.dim() == 3 && keys.dim() == 4 && vals.dim() == 4,
              "laprune::dense_decode: q [B, Hq, D], keys / vals [B, Hkv, T, D]");
  same_gpu("laprune::dense_decode", {&q, &keys, &vals, &out, &ws});
  TORCH_CHECK(keys.scalar_type() == q.scalar_type() && vals.scalar_type() == q.scalar_type() &&
                  out.scalar_type() == q.scalar_type() && out.is_contiguous() &&
                  out.numel() >= q.size(0) * q.size(1) * q.size(2),
              "laprune::dense_decode: keys, vals and a contiguous out of B * Hq * D elements in "
              "q's dtype");
  TORCH_CHECK(keys.size(0) == q.size(0) && vals.size(0) == q.size(0) &&
                  vals.size(1) == keys.size(1) && vals.size(2) >= keys.size(2) &&
                  keys.size(3) == q.size(2) && vals.size(3) == q.size(2),
              "laprune::dense_decode: keys / vals must be [B, Hkv, T, D] of q's B and D");
  check(lap_dense_attn_decode(ptr(q), q.stride(0), q.stride(1), ptr(keys), ptr(vals),
                              dtype_code(q), (int)q.size(0), (int)q.size(1), (int)keys.size(1),
                              (int)keys.size(2), (int)q.size(2), keys.stride(0), keys.stride(1),
                              keys.stride(2), vals.stride(0), vals.stride(1), vals.stride(2),
                              (float)scale, ptr(out), ptr(ws),
                              (size_t)ws.numel() * ws.element_size(), stream_of(q)),
        "lap_dense_attn_decode");
}

// Ragged sparse (or, without indices, dense) decode over device plans.
void attn_decode_ragged(const at::Tensor& q, const at::Tensor& keys, const at::Tensor& vals,
                        const std::optional<at::Tensor>& idx, int64_t H_idx, int64_t k_cols,
                        const at::Tensor& plans, int64_t max_sink, int64_t max_tail,
                        double scale, const at::Tensor& out, const at::Tensor& ws) {
  TORCH_CHECK(q.dim() == 3 && keys.dim() == 4 && vals.dim() == 4,
              "laprune::attn_decode_ragged: q [B, Hq, D], keys / vals [B, Hkv, T, D]");
  same_gpu("laprune::attn_decode_ragged", {&q, &keys, &vals, opt(idx), &plans, &out, &ws});
  TORCH_CHECK(keys.scalar_type() == q.scalar_type() && vals.scalar_type() == q.scalar_type() &&
                  out.scalar_type() == q.scalar_type() && out.is_contiguous() &&
                  out.numel() >= q.size(0) * q.size(1) * q.size(2),
              "laprune::attn_decode_ragged: keys, vals and a contiguous out of B * Hq * D "
              "elements in q's dtype");
  TORCH_CHECK(plans.scalar_type() == at::kInt && plans.is_contiguous() &&
                  plans.numel() >= q.size(0) * 8,
              "laprune::attn_decode_ragged: plans must hold B lap_row_plan records");
  TORCH_CHECK(!idx || (idx->is_contiguous() && idx->numel() >= q.size(0) * H_idx * k_cols),
              "laprune::attn_decode_ragged: idx must hold B * H_idx * k_cols entries");
  check(lap_sparse_attn_decode_ragged(
            ptr(q), q.stride(0), q.stride(1), ptr(keys), ptr(vals), dtype_code(q),
            (int)q.size(0), (int)q.size(1), (int)keys.size(1), (int)keys.size(2),
            (int)q.size(2), keys.stride(0), keys.stride(1), keys.stride(2), vals.stride(0),
            vals.stride(1), vals.stride(2), ptr(idx), idx ? dtype_code(*idx) : LAP_DTYPE_I32,
            (int)H_idx, (int)k_cols, static_cast<const lap_row_plan*>(ptr(plans)),
            (int)max_sink, (int)max_tail, (float)scale, ptr(out), ptr(ws),
            (size_t)ws.numel() * ws.element_size(), stream_of(q)),
        "lap_sparse_attn_decode_ragged");
}

// The step's RoPE + cache append (lap_rope_append): q [B, 1, Hq*D],
// k / v [B, 1, Hkv*D], cos / sin [B, 1, D], pos int64 [B], caches
// [B, Hkv, t_cap, D], q_out [B, Hq, D].
void rope_append(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                 const at::Tensor& cos, const at::Tensor& sin, const at::Tensor& pos,
                 const at::Tensor& cache_k, const at::Tensor& cache_v, int64_t t_cap,
                 const at::Tensor& q_out) {
  TORCH_CHECK(q_out.dim() == 3 && cache_k.dim() == 4 && cache_v.dim() == 4,
              "laprune::rope_append: q_out [B, Hq, D], caches [B, Hkv, T, D]");
  same_gpu("laprune::rope_append", {&q, &k, &v, &cos, &sin, &pos, &cache_k, &cache_v, &q_out});
  TORCH_CHECK(pos.scalar_type() == at::kLong, "laprune::rope_append: int64 positions");
  const int D = (int)cos.size(-1);
  check(lap_rope_append(ptr(q), q.stride(0), D, ptr(k), k.stride(0), D, ptr(v), v.stride(0), D,
                        ptr(cos), ptr(sin), cos.stride(0), dtype_code(q_out),
                        (int)q_out.size(0), (int)q_out.size(1), (int)cache_k.size(1), D,
                        static_cast<const int64_t*>(ptr(pos)), ptr(cache_k), cache_k.stride(0),
                        cache_k.stride(1), cache_k.stride(2), ptr(cache_v), cache_v.stride(0),
                        cache_v.stride(1), cache_v.stride(2), (int)t_cap, ptr(q_out),
                        stream_of(q_out)),
        "lap_rope_append");
}

// Per-sequence flush of the encode buffer (lap_encode_keys_ranges): keys
// [B, Hkv, t_cap, D] cache, ranges int32 [B, 2], codes [B, Hkv, t_cap, M].
void encode_keys_ranges(const at::Tensor& keys, const at::Tensor& ranges, int64_t max_len,
                        int64_t t_cap, const at::Tensor& cb, const at::Tensor& prep,
                        const at::Tensor& codes) {
  TORCH_CHECK(keys.dim() == 4 && codes.dim() == 4 && cb.dim() == 3,
              "laprune::encode_keys_ranges: keys / codes [B, Hkv, T, *], codebooks [M, K, D]");
  TORCH_CHECK(cb.scalar_type() == at::kFloat, "laprune::encode_keys_ranges: fp32 codebooks");
  TORCH_CHECK(ranges.scalar_type() == at::kInt, "laprune::encode_keys_ranges: int32 ranges");
  same_gpu("laprune::encode_keys_ranges", {&keys, &ranges, &cb, &prep, &codes});
  check(lap_encode_keys_ranges(ptr(keys), dtype_code(keys), keys.stride(0), keys.stride(1),
                               keys.stride(2), (int)keys.size(0), (int)keys.size(1),
                               static_cast<const int32_t*>(ptr(ranges)), (int)max_len, (int)t_cap,
                               (int)keys.size(3), static_cast<const float*>(ptr(cb)),
                               (int)cb.size(0), (int)cb.size(1), ptr(prep),
                               (size_t)prep.numel() * prep.element_size(),
                               static_cast<uint8_t*>(ptr(codes)), codes.stride(0),
                               codes.stride(1), codes.stride(2), stream_of(keys)),
        "lap_encode_keys_ranges");
}

// Grouped LUT scoring (the reference's aq_lut_gather_grouped,
// aq_kernels/aq_lut_gqa.cu:460-534): codes [Hkv, T, M], out fp16 [Hkv*G, T].
void score_grouped(const at::Tensor& lut, int64_t layout, const at::Tensor& codes, int64_t G,
                   int64_t M, int64_t K, const at::Tensor& out) {
  TORCH_CHECK(codes.dim() == 3 && codes.scalar_type() == at::kByte,
              "laprune::score_grouped: codes u8 [Hkv, T, M]");
  same_gpu("laprune::score_grouped", {&lut, &codes, &out});
  check(lap_lut_score_grouped(ptr(lut), (int)layout, static_cast<const uint8_t*>(ptr(codes)),
                              codes.stride(0), codes.stride(1), (int)codes.size(0), (int)G,
                              (int)codes.size(1), (int)M, (int)K, ptr(out), stream_of(out)),
        "lap_lut_score_grouped");
}

}  // namespace

TORCH_LIBRARY(laprune, m) {
  m.def("lut_build(Tensor q, Tensor codebooks, int G, int layout, Tensor(a!) out) -> ()");
  m.def("decode_step(Tensor lut, Tensor? codes, int T, int cand_start, int cand_end, int k, "
        "int sink, int tail_start, int tail_count, Tensor? plans, int k_cols, int max_sink, "
        "int max_tail, int key_mode, Tensor q, Tensor keys, Tensor vals, float scale, "
        "Tensor(a!) idx, Tensor(b!) out, Tensor(c!) ws) -> ()");
  m.def("dense_decode(Tensor q, Tensor keys, Tensor vals, float scale, Tensor(a!) out, "
        "Tensor(b!) ws) -> ()");
  m.def("attn_decode_ragged(Tensor q, Tensor keys, Tensor vals, Tensor? idx, int H_idx, "
        "int k_cols, Tensor plans, int max_sink, int max_tail, float scale, Tensor(a!) out, "
        "Tensor(b!) ws) -> ()");
  m.def("rope_append(Tensor q, Tensor k, Tensor v, Tensor cos, Tensor sin, Tensor pos, "
        "Tensor(a!) cache_k, Tensor(b!) cache_v, int t_cap, Tensor(c!) q_out) -> ()");
  m.def("encode_keys_ranges(Tensor keys, Tensor ranges, int max_len, int t_cap, "
        "Tensor codebooks, Tensor prep, Tensor(a!) codes) -> ()");
  m.def("score_grouped(Tensor lut, int layout, Tensor codes, int G, int M, int K, "
        "Tensor(a!) out) -> ()");
}

TORCH_LIBRARY_IMPL(laprune, CUDA, m) {
  m.impl("lut_build", &lut_build);
  m.impl("decode_step", &decode_step);
  m.impl("dense_decode", &dense_decode);
  m.impl("attn_decode_ragged", &attn_decode_ragged);
  m.impl("rope_append", &rope_append);
  m.impl("encode_keys_ranges", &encode_keys_ranges);
  m.impl("score_grouped", &score_grouped);
}

"""The C ABI library loads, exports every symbol include/laprune_hip.h declares,
and rejects invalid arguments with a status and a message — all without a GPU
(argument checks run before any device call)."""
import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "laprune_hip.h"


def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(lap_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    from laprune_amd import _native as N
    return N.lib()


def test_header_declares_the_abi():
    names = declared()
    assert "lap_last_error" in names and "lap_retrieve_topk" in names
    assert len(names) >= 20


def test_every_declared_symbol_is_exported_and_bound(lib):
    from laprune_amd import _native as N
    for name in declared():
        assert hasattr(lib, name), f"{name} not exported"
        if name != "lap_last_error":
            assert name in N.SIGNATURES, f"{name} not bound in _native.SIGNATURES"


def test_abi_version(lib):
    assert lib.lap_abi_version() == 7


def _err(lib):
    return lib.lap_last_error().decode()


def test_invalid_arguments_return_status_and_message(lib):
    from laprune_amd import _native as N
    st = lib.lap_lut_build(None, N.BF16, 128, None, N.F32, 32, 128, 32, 256, 4, N.LUT_GMKG, None, None)
    assert st == N.LAP_ERR_INVALID and "null pointer" in _err(lib)
    al, odd = C.c_void_p(4096), C.c_void_p(4098)  # never dereferenced
    st = lib.lap_lut_build(odd, N.BF16, 128, al, N.F32, 32, 128, 32, 256, 4, N.LUT_GMKG, al, None)
    assert st == N.LAP_ERR_INVALID and "aligned" in _err(lib)
    st = lib.lap_lut_build(al, N.BF16, 130, al, N.F32, 32, 128, 32, 256, 4, N.LUT_GMKG, al, None)
    assert st == N.LAP_ERR_INVALID and "multiple of 4" in _err(lib)
    st = lib.lap_lut_build(al, N.F32, 128, odd, N.F32, 32, 128, 32, 256, 4, N.LUT_GMKG, al, None)
    assert st == N.LAP_ERR_INVALID and "codebooks must be" in _err(lib)
    one = C.c_void_p(16)  # never dereferenced: validation fails first
    st = lib.lap_lut_score_grouped(one, N.LUT_HMK, one, 0, 32, 8, 5, 100, 32, 256, one, None)
    assert st == N.LAP_ERR_INVALID and "G<=4" in _err(lib)
    st = lib.lap_lut_score_mha(one, N.BF16, one, N.U8, 1, 1, 1, 1, one, None)
    assert st == N.LAP_ERR_INVALID and "fp16 or fp32" in _err(lib)
    st = lib.lap_topk_select(one, 10, 1, 1, 10, 5, 20, 3, N.KEY_F16, one, N.I32, None, 0, None)
    assert st == N.LAP_ERR_INVALID and "candidate window" in _err(lib)
    st = lib.lap_gqa_gather_kv(one, one, N.F32, 1, 1, 10, 128, 0, 0, 128, 0, 0, 128, one, 4, 1,
                               -1, 0, one, one, None)
    assert st == N.LAP_ERR_INVALID and "fp16/bf16" in _err(lib)
    st = lib.lap_encode_greedy(one, 128, 4, 128, one, 32, 300, one, 1 << 30, one, 32, None, None)
    assert st == N.LAP_ERR_INVALID and "exceeds 256" in _err(lib)
    st = lib.lap_sparse_attn_decode(one, 0, 128, one, one, N.BF16, 1, 32, 8, 100, 128, 0, 0, 128,
                                    0, 0, 128, one, N.I32, 5, 10, 0, -1, 0, 1.0, one, None, 0, None)
    assert st == N.LAP_ERR_INVALID and "H_idx" in _err(lib)


def test_ragged_entry_points_validate_before_any_device_call(lib):
    from laprune_amd import _native as N
    one = C.c_void_p(256)  # never dereferenced: validation fails first
    st = lib.lap_retrieve_topk_ragged(one, one, 0, 0, 32, 2, 8, 1000, None, 64, N.KEY_F16, None,
                                      one, N.I32, one, 1 << 30, None)
    assert st == N.LAP_ERR_INVALID and "null plans" in _err(lib)
    st = lib.lap_retrieve_topk_ragged(one, one, 0, 0, 32, 2, 8, 1000, one, 64, N.KEY_F16, None,
                                      one, N.F32, one, 1 << 30, None)
    assert st == N.LAP_ERR_INVALID and "int32/int64" in _err(lib)
    st = lib.lap_topk_select_ragged(one, 1000, 10, 1, 4, 1000, one, 64, N.KEY_F16, one, N.I32,
                                    one, 1 << 30, None)
    assert st == N.LAP_ERR_INVALID and "rows_per_plan" in _err(lib)
    st = lib.lap_topk_select_ragged(one, 999, 8, 1, 4, 1000, one, 64, N.KEY_F16, one, N.I32,
                                    one, 1 << 30, None)
    assert st == N.LAP_ERR_INVALID and "row stride" in _err(lib)
    st = lib.lap_sparse_attn_decode_ragged(one, 0, 128, one, one, N.BF16, 2, 32, 8, 100, 128, 0,
                                           0, 128, 0, 0, 128, one, N.I32, 8, 10, None, 4, 64,
                                           1.0, one, None, 0, None)
    assert st == N.LAP_ERR_INVALID and "null plans" in _err(lib)
    st = lib.lap_sparse_attn_decode_ragged(one, 0, 128, one, one, N.BF16, 2, 32, 8, 100, 128, 0,
                                           0, 128, 0, 0, 128, one, N.I32, 8, 10, one, -1, 64,
                                           1.0, one, None, 0, None)
    assert st == N.LAP_ERR_INVALID and "negative" in _err(lib)


def test_workspace_size_queries(lib):
    from laprune_amd import _native as N
    assert N.size_query("lap_topk_workspace_size", 8, 131008) > 8 * 131008 * 2
    assert N.size_query("lap_retrieve_workspace_size", 8, 131072) > 8 * 131072 * 2
    assert N.size_query("lap_attn_decode_workspace_size", 1, 32, 128, 2116) > 0
    assert N.size_query("lap_encode_prep_size", 32, 256, 128) >= 32 * 256 * 128 * 4


def test_aq_kernels_exports_reference_names():
    from laprune_amd import aq_kernels as K
    for name in K.REFERENCE_NAMES:
        assert hasattr(K, name)
    import inspect
    sig = inspect.signature(K._impl.gqa_gather_kv_with_tail)
    assert list(sig.parameters) == ["keys", "vals", "indices", "G", "tail_start", "tail_count",
                                    "threads", "vector_width"]
    assert sig.parameters["threads"].default == 256 and sig.parameters["vector_width"].default == 8
    sig = inspect.signature(K._impl.aq_lut_gather)
    assert list(sig.parameters) == ["lut", "codes", "G", "M_start", "M_end", "indices"]
    sig = inspect.signature(K._impl.fused_linear_encode_forward)
    assert list(sig.parameters) == ["x", "weight_t", "bias", "codebooks", "fp32_residual", "tile_n"]
    sig = inspect.signature(K._impl.aq_lut_gather_grouped)
    assert sig.parameters["grid_y_cap"].default == 48


def test_cpu_tensors_are_rejected_loudly():
    import torch
    from laprune_amd.aq_kernels import _impl
    with pytest.raises(RuntimeError, match="CUDA"):
        _impl.aq_lut_gather_grouped(torch.zeros(4, 32, 256, dtype=torch.float16),
                                    torch.zeros(1, 10, 32, dtype=torch.uint8), 4)
    with pytest.raises(RuntimeError):
        _impl.aq_lut_build(torch.zeros(4, 128), torch.zeros(32, 256, 128))


def test_decode_step_argument_checks(lib):
    """lap_decode_step validates before touching the device: null inputs,
    head counts that do not group, a group size above 8, and a missing
    workspace (also for G = 2, which the kernel chain serves)."""
    from laprune_amd import _native as N
    one = C.c_void_p(4096)  # never dereferenced
    args = dict(lut=one, codes=one, T=1024, cs=4, ce=960, k=64, sink=4, ts=960, tc=64, key=N.KEY_BF16,
                q=one, Hq=32, Hkv=8, ws=None, ws_n=0)

    def call(**kw):
        a = {**args, **kw}
        return lib.lap_decode_step(a["lut"], a["codes"], 8 * 1024 * 32, 1024 * 32, 32, a["T"],
                                   a["cs"], a["ce"], a["k"], a["sink"], a["ts"], a["tc"], None, 0,
                                   0, 0, a["key"], a["q"], 32 * 128, 128, one, one, N.BF16, 1,
                                   a["Hq"], a["Hkv"], 1024, 128, 8 * 1024 * 128, 1024 * 128, 128,
                                   8 * 1024 * 128, 1024 * 128, 128, C.c_float(0.088), one, N.I32,
                                   one, a["ws"], a["ws_n"], None)

    assert call(lut=None) == N.LAP_ERR_INVALID and "null pointer" in _err(lib)
    assert call(Hq=20) == N.LAP_ERR_INVALID and "not a multiple" in _err(lib)
    assert call(Hq=72) == N.LAP_ERR_UNSUPPORTED and "group size 9" in _err(lib)
    assert call(Hq=16) == N.LAP_ERR_WORKSPACE and "workspace of" in _err(lib)
    assert call(ce=2000) == N.LAP_ERR_INVALID and "candidate window" in _err(lib)
    assert call(key=7) == N.LAP_ERR_INVALID and "key mode" in _err(lib)
    assert call() == N.LAP_ERR_WORKSPACE and "workspace of" in _err(lib)
    need = C.c_size_t(0)
    assert lib.lap_decode_step_workspace_size(1, 32, 8, 1024, 128, 132, N.KEY_BF16,
                                              C.byref(need)) == N.LAP_OK
    assert need.value > 0


def test_torch_binding_registers_the_hot_ops():
    """The compiled torch binding loads (no GPU needed) and registers one op
    per hot entry point, each with its schema."""
    from laprune_amd._ops import ops
    o = ops()
    want = {
        "lut_build": "Tensor q, Tensor codebooks, int G, int layout, Tensor(a!) out",
        "decode_step": "Tensor lut, Tensor? codes, int T,",
        "dense_decode": "Tensor q, Tensor keys, Tensor vals, float scale",
        "attn_decode_ragged": "Tensor? idx, int H_idx, int k_cols, Tensor plans",
        "rope_append": "Tensor cos, Tensor sin, Tensor pos",
        "encode_keys_ranges": "Tensor keys, Tensor ranges, int max_len, int t_cap",
        "score_grouped": "Tensor lut, int layout, Tensor codes, int G",
    }
    for name, frag in want.items():
        schema = str(getattr(o, name).default._schema)
        assert schema.startswith(f"laprune::{name}("), schema
        assert frag in schema, (name, schema)


def test_floor_kernels_check_their_arguments(lib):
    """The scorer's measurement kernels reject bad shapes before any launch."""
    from laprune_amd import _native as N
    al = C.c_void_p(4096)  # never dereferenced: validation fails first
    st = lib.lap_floor_stream(al, al, 0, 32, 8, 131072, 2, al, None)
    assert st == N.LAP_ERR_INVALID and "ahead must be 1 or 4" in _err(lib)
    st = lib.lap_floor_stream(al, al, 0, 16, 8, 131072, 1, al, None)
    assert st == N.LAP_ERR_INVALID and "32 bytes apart" in _err(lib)
    st = lib.lap_floor_stream(None, al, 0, 32, 8, 131072, 1, al, None)
    assert st == N.LAP_ERR_INVALID and "null pointer" in _err(lib)
    assert lib.lap_floor_empty(0, 10, None) == N.LAP_ERR_INVALID

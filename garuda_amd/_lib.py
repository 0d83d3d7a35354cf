"""ctypes binding of include/garuda_moe.h (libgaruda_moe.so, built in-tree).

Loading fails loudly: there is no fallback path. If the library is missing,
build it with `python -m garuda_amd.build`.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libgaruda_moe.so"

u32, u64, i32, f32p, u32p = C.c_uint32, C.c_uint64, C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_uint32)
vp = C.c_void_p


class GmoeTensor(C.Structure):
    _fields_ = [("qtype", u32), ("layout", u32), ("data", vp), ("experts", C.POINTER(vp))]


class GmoeLayerDesc(C.Structure):
    _fields_ = [
        ("d_model", u32), ("d_ff", u32), ("n_experts", u32), ("top_k", u32),
        ("gating", u32), ("combine", u32), ("math", u32),
        ("router", f32p),
        ("gate", GmoeTensor), ("up", GmoeTensor), ("down", GmoeTensor),
    ]


class GmoeSlabStats(C.Structure):
    _fields_ = [("hits", u64), ("misses", u64), ("evictions", u64), ("entries", u64),
                ("bytes", u64), ("capacity", u64), ("h2d_bytes", u64)]


class GmoeDenseDesc(C.Structure):
    _fields_ = [("rows", u32), ("cols", u32), ("qtype", u32), ("math", u32), ("data", vp)]


class GmoeGgufHeader(C.Structure):
    _fields_ = [("version", u32), ("n_tensors", u64), ("n_keys", u64), ("data_offset", u64),
                ("file_bytes", u64)]


class GmoeGgufValue(C.Structure):
    _fields_ = [("type", u32), ("elem_type", u32), ("u", u64), ("f", C.c_double),
                ("str", C.POINTER(C.c_char)), ("len", u64), ("node", vp)]


class GmoeGgufTensorInfo(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", u32), ("qtype", u32), ("dims", u64 * 4),
                ("offset", u64), ("n_elements", u64), ("nbytes", u64), ("data", vp)]


class GmoeL2Counts(C.Structure):
    _fields_ = [("l2", u64), ("synthesised", u64), ("written", u64), ("l3", u64), ("promoted", u64)]


class GmoePredictStats(C.Structure):
    _fields_ = [("correct", u64), ("wasted", u64), ("missed", u64)]


# name -> (restype, argtypes)
SIGNATURES = {
    "gmoe_abi_version": (u32, []),
    "gmoe_last_error": (C.c_char_p, []),
    "gmoe_last_invalid_token": (u32, []),
    "gmoe_init": (i32, [i32, u64, C.POINTER(vp)]),
    "gmoe_shutdown": (None, [vp]),
    "gmoe_layer_register": (i32, [vp, C.POINTER(GmoeLayerDesc), u32p]),
    "gmoe_layer_register_fetch": (i32, [vp, C.POINTER(GmoeLayerDesc), vp, vp, u32p]),
    "gmoe_layer_release": (i32, [vp, u32]),
    "gmoe_ffn_forward": (i32, [vp, u32, f32p, u32, f32p, u32p, f32p]),
    "gmoe_ffn_forward_logits": (i32, [vp, u32, f32p, f32p, u32, f32p, u32p, f32p]),
    "gmoe_ffn_forward_async": (i32, [vp, u32, vp, vp, u32, vp, vp, vp, vp]),
    "gmoe_ffn_forward_noalloc": (i32, [vp, u32, vp, vp, u32, vp, vp, vp, vp]),
    "gmoe_expert_prefetch": (i32, [vp, u32, u32]),
    "gmoe_expert_state": (i32, [vp, u32, u32]),
    "gmoe_prefetch_hold": (i32, [vp, i32]),
    "gmoe_prefetch_wait": (i32, [vp]),
    "gmoe_expert_is_resident": (i32, [vp, u32, u32]),
    "gmoe_expert_evict": (i32, [vp, u32, u32]),
    "gmoe_slab_get_stats": (i32, [vp, C.POINTER(GmoeSlabStats)]),
    "gmoe_dequant": (i32, [vp, u32, vp, u64, u64, f32p]),
    "gmoe_matmul": (i32, [vp, u32, u32, vp, u64, u32, u32, f32p, u32, f32p]),
    "gmoe_route": (i32, [vp, u32, f32p, f32p, u32, u32, u32, u32, u32p, f32p, f32p]),
    "gmoe_dispatch": (i32, [vp, u32p, f32p, u32, u32, u32, u32p, u32p, f32p, u32p]),
    "gmoe_expf": (i32, [vp, f32p, u64, f32p]),
    "gmoe_quantize": (i32, [u32, f32p, u64, vp, i32]),
    "gmoe_fill_gaussian": (i32, [u64, C.c_float, C.c_float, u64, f32p, i32]),
    "gmoe_fill_seeded": (i32, [u64, u64, C.c_float, f32p]),
    "gmoe_l2_open": (i32, [C.c_char_p, u32, u32, u32, u32, C.POINTER(vp)]),
    "gmoe_l2_close": (None, [vp]),
    "gmoe_l2_get_counts": (i32, [vp, C.POINTER(GmoeL2Counts)]),
    "gmoe_l2_layer_desc": (i32, [vp, f32p, u32, u32, u32, C.POINTER(GmoeLayerDesc)]),
    "gmoe_tiers_open": (i32, [C.c_char_p, C.c_char_p, u32, u32, u32, u32, C.POINTER(vp)]),
    "gmoe_l2_fetch": (i32, [vp, u32, C.POINTER(vp)]),
    "gmoe_l2_locate": (i32, [vp, u32]),
    "gmoe_l2_layer_register": (i32, [vp, vp, f32p, u32, u32, u32, u32p]),
    "gmoe_dense_register": (i32, [vp, C.POINTER(GmoeDenseDesc), u32p]),
    "gmoe_dense_release": (i32, [vp, u32]),
    "gmoe_dense_forward": (i32, [vp, u32, f32p, u32, f32p]),
    "gmoe_dense_forward_async": (i32, [vp, u32, vp, u32, vp, vp]),
    "gmoe_dense_forward_slices_async": (i32, [vp, u32, vp, u32, vp, u32p, vp]),
    "gmoe_predictor_create": (i32, [u32, C.POINTER(vp)]),
    "gmoe_predictor_destroy": (None, [vp]),
    "gmoe_predictor_observe": (i32, [vp, u32p, u32, u32p, u32]),
    "gmoe_predictor_predict": (i32, [vp, u32p, u32, u32, u32p, u32p]),
    "gmoe_predictor_score": (i32, [vp, u32p, u32, u32p, u32]),
    "gmoe_predictor_stats": (i32, [vp, C.POINTER(GmoePredictStats)]),
    "gmoe_predictor_get_counts": (i32, [vp, u32p, u64]),
    "gmoe_predictor_set_counts": (i32, [vp, u32p, u64]),
    "gmoe_prefetch_step": (i32, [vp, vp, u32, u32, u32p, u32, u32p, u32, u32p, u32, u32, u32p, u32p, u32p, u32p]),
    "gmoe_kv_create": (i32, [vp, vp, C.POINTER(vp)]),
    "gmoe_kv_destroy": (None, [vp]),
    "gmoe_kv_seq_open": (i32, [vp, u32p]),
    "gmoe_kv_seq_close": (i32, [vp, u32]),
    "gmoe_kv_seq_len": (i32, [vp, u32, u32, u32p]),
    "gmoe_kv_free_pages": (i32, [vp, C.POINTER(u64)]),
    "gmoe_kv_fail_reserves": (i32, [vp, u32]),
    "gmoe_attention": (i32, [vp, u32, u32p, u32, f32p, f32p, f32p, f32p]),
    "gmoe_attention_async": (i32, [vp, u32, u32p, u32, vp, vp, vp, vp, vp]),
    "gmoe_gguf_open": (i32, [C.c_char_p, C.POINTER(vp)]),
    "gmoe_gguf_parse": (i32, [vp, u64, C.POINTER(vp)]),
    "gmoe_gguf_close": (None, [vp]),
    "gmoe_gguf_get_header": (i32, [vp, C.POINTER(GmoeGgufHeader)]),
    "gmoe_gguf_key_at": (i32, [vp, u64, C.POINTER(C.c_char_p)]),
    "gmoe_gguf_get_value": (i32, [vp, C.c_char_p, C.POINTER(GmoeGgufValue)]),
    "gmoe_gguf_array_item": (i32, [vp, C.POINTER(GmoeGgufValue), u64, C.POINTER(GmoeGgufValue)]),
    "gmoe_gguf_tensor_at": (i32, [vp, u64, C.POINTER(GmoeGgufTensorInfo)]),
    "gmoe_gguf_find_tensor": (i32, [vp, C.c_char_p, C.POINTER(GmoeGgufTensorInfo)]),
    "gmoe_gguf_layer_desc": (i32, [vp, u32, u32, u32, u32, C.POINTER(GmoeLayerDesc)]),
    "gmoe_gguf_expert_ranges": (i32, [vp, u32, u32, C.POINTER(u64), C.POINTER(u64)]),
    "gmoe_model_create": (i32, [vp, vp, C.POINTER(vp)]),
    "gmoe_model_destroy": (None, [vp]),
    "gmoe_model_decode": (i32, [vp, u32, u32p, u32p, u32p, f32p]),
    "gmoe_model_prefill": (i32, [vp, u32, u32, u32p, u32, u32p, f32p]),
    "gmoe_model_trace_floats": (C.c_size_t, [vp, u32]),
    "gmoe_model_decode_trace": (i32, [vp, u32, u32p, u32p, u32p, f32p, f32p]),
    "gmoe_model_set_graphs": (i32, [vp, C.c_int]),
    "gmoe_model_graph_ready": (C.c_int, [vp, u32]),
    "gmoe_set_kernel_timing": (i32, [vp, i32]),
    "gmoe_kernel_time": (i32, [vp, u32, C.POINTER(C.c_double), C.POINTER(u64)]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded library with typed entry points. Raises if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: the MI355X path has no fallback. "
                "Build it with `python -m garuda_amd.build`."
            )
        h = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib

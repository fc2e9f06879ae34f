"""ctypes binding of libe4b.so (the C ABI declared in include/e4b.h).

The shared library is built in-tree (``e4b-webgpu_amd/libe4b.so``) by
``__graft_entry__.build()``.  There is no fallback: if the library is missing
or fails to load, importing this module raises, so nothing can silently run on
another path.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# E4B_LIBRARY names another build of the same library (libe4b_trace.so, the
# device-side timeline build); by default the in-tree libe4b.so
LIB_PATH = os.path.normpath(os.environ.get("E4B_LIBRARY") or os.path.join(_HERE, "..", "libe4b.so"))

E4B_OK = 0
E4B_EINVAL = -1
E4B_ENOMEM = -2
E4B_EHIP = -3
E4B_ESTATE = -4
E4B_ENOTENSOR = -5
E4B_ERANGE = -6
RECIPE_E4B = 0
RECIPE_A4B = 1

DT_F32 = 0
DT_F16 = 1
DT_F32_HL = 2

GGML_F32 = 0
GGML_F16 = 1
GGML_Q4_0 = 2
GGML_Q6_K = 14


class E4BError(RuntimeError):
    """A libe4b call returned a negative status."""

    def __init__(self, code: int, where: str, msg: str):
        super().__init__(f"{where}: error {code}: {msg}")
        self.code = code


if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"libe4b.so not found at {LIB_PATH}; build it with `python -c 'import __graft_entry__ as g; g.build()'`"
    )

lib = C.CDLL(LIB_PATH)

_vp, _sz, _i64, _u64, _i32, _u32, _f32 = C.c_void_p, C.c_size_t, C.c_int64, C.c_uint64, C.c_int, C.c_uint32, C.c_float
_P = C.POINTER

# (name, restype, argtypes); the order follows include/e4b.h
SIGNATURES = [
    ("e4b_version", C.c_char_p, []),
    ("e4b_last_error", C.c_char_p, []),
    ("e4b_device_count", _i32, [_P(_i32)]),
    ("e4b_set_device", _i32, [_i32]),
    ("e4b_dev_alloc", _vp, [_sz]),
    ("e4b_dev_free", _i32, [_vp]),
    ("e4b_memcpy_h2d", _i32, [_vp, _vp, _sz]),
    ("e4b_memcpy_d2h", _i32, [_vp, _vp, _sz]),
    ("e4b_memset_dev", _i32, [_vp, _i32, _sz]),
    ("e4b_memcpy_d2d", _i32, [_vp, _vp, _sz, _vp]),
    ("e4b_sync", _i32, []),
    ("e4b_stream_sync", _i32, [_vp]),
    ("e4b_event_create", _vp, []),
    ("e4b_event_record", _i32, [_vp, _vp]),
    ("e4b_event_elapsed_ms", _i32, [_vp, _vp, _P(_f32)]),
    ("e4b_event_destroy", _i32, [_vp]),
    ("e4b_split_f32", _i32, [_vp, _i64, _vp, _vp]),
    ("e4b_synth_u64", _u64, [_u64, _u64]),
    ("e4b_synth_normal_f32", _i32, [_u64, _i64, _f32, _f32, _vp]),
    ("e4b_synth_uniform_u32", _i32, [_u64, _i64, _u32, _u32, _vp]),
    ("e4b_synth_q40", _i32, [_u64, _i64, _i64, _f32, _vp]),
    ("e4b_synth_q6k", _i32, [_u64, _i64, _i64, _f32, _vp]),
    ("e4b_q40_packed_bytes", _sz, [_i64, _i64]),
    ("e4b_q40_pack", _i32, [_vp, _i64, _i64, _vp]),
    ("e4b_q6k_packed_bytes", _sz, [_i64, _i64]),
    ("e4b_q6k_pack", _i32, [_vp, _i64, _i64, _vp]),
    ("e4b_k_q40_gemv", _i32, [_vp, _i64, _i64, _vp, _i32, _vp, _vp]),
    ("e4b_k_q40_gemv_geglu", _i32, [_vp, _i64, _i64, _vp, _vp, _vp]),
    ("e4b_k_q40_gemm", _i32, [_vp, _i64, _i64, _vp, _i32, _vp, _vp]),
    ("e4b_k_q40_gemm_geglu", _i32, [_vp, _i64, _i64, _vp, _i32, _vp, _vp]),
    ("e4b_k_q40_geglu_prenorm", _i32, [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _f32, _f32, _vp, _vp, _vp]),
    ("e4b_k_q6k_gemv_argmax", _i32, [_vp, _i64, _i64, _vp, _f32, _vp, _vp, _vp]),
    ("e4b_k_q6k_gemv_argmax_noalloc", _i32, [_vp, _i64, _i64, _vp, _f32, _vp, _vp, _vp]),
    ("e4b_k_q6k_row", _i32, [_vp, _i64, _i64, _i64, _f32, _vp, _vp]),
    ("e4b_k_argmax", _i32, [_vp, _i64, _vp, _vp]),
    ("e4b_rope_inv_freq", _i32, [_f32, _i32, _i32, _vp]),
    ("e4b_k_router_top8", _i32, [_vp, _vp, _vp, _vp, _vp]),
    ("e4b_k_moe_layer", _i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    ("e4b_k_moe_prefill", _i32, [_vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    ("e4b_k_attn_decode", _i32, [_vp, _vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _u32, _f32,
                                 _i32, _vp, _vp]),
    ("e4b_k_attn_prefill", _i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _u32, _vp]),
    ("e4b_create", _vp, [_vp]),
    ("e4b_set_tensor", _i32, [_vp, C.c_char_p, _i32, _P(_i64), _i32, _vp, _sz]),
    ("e4b_finalize", _i32, [_vp]),
    ("e4b_step", _i32, [_vp, _u32, _u32, _vp, _vp]),
    ("e4b_prefill", _i32, [_vp, _vp, _u32, _vp]),
    ("e4b_prefill_steps", _i32, [_vp, _vp, _u32, _vp]),
    ("e4b_profile_step", _i32, [_vp, _u32, _u32, _vp, _i32]),
    ("e4b_profile_prefill", _i32, [_vp, _vp, _u32, _vp, _i32]),
    ("e4b_trace_start", _i32, [_sz]),
    ("e4b_trace_read", _i32, [_vp, _sz, _P(_sz)]),
    ("e4b_trace_stop", _i32, []),
    ("e4b_trace_clock_khz", _i32, [_P(_i32)]),
    ("e4b_decode", _i32, [_vp, _u32, _u32, _vp]),
    ("e4b_argmax", _i32, [_vp, _vp]),
    ("e4b_read_hidden", _i32, [_vp, _vp]),
    ("e4b_read_layer_hidden", _i32, [_vp, _i32, _vp]),
    ("e4b_read_topk", _i32, [_vp, _i32, _vp, _vp]),
    ("e4b_read_logits", _i32, [_vp, _vp]),
    ("e4b_read_kv", _i32, [_vp, _i32, _vp, _vp]),
    ("e4b_kv_slots", _i32, [_vp, _i32]),
    ("e4b_reset", _i32, [_vp]),
    ("e4b_destroy", None, [_vp]),
    ("e4b_time_decode", _i32, [_vp, _u32, _u32, _P(_f32)]),
    ("e4b_kv_count", _i32, [_vp]),
    ("e4b_read_scores", _i32, [_vp, _i32, _vp]),
    ("e4b_kv_compact", _i32, [_vp, _i32, _i32]),
    ("e4b_kv_select", _i64, [_vp, _i32, _i64, _i64, _i32, _i32, _vp]),
    ("e4b_gguf_config", _i32, [C.c_char_p, _vp, _vp, _vp, _i32]),
    ("e4b_load_gguf", _i32, [_vp, C.c_char_p]),
    ("e4b_open_gguf", _vp, [C.c_char_p, _vp]),
]


class ConfigC(C.Structure):
    """struct e4b_config (include/e4b.h)."""

    _fields_ = [
        ("hidden", _i32), ("layers", _i32), ("q_heads", _i32), ("kv_heads", _i32), ("head_dim", _i32),
        ("ffn", _i32), ("ple_dim", _i32), ("vocab", _i32), ("window", _i32), ("ring", _i32), ("max_seq", _i32),
        ("rope_angles", _i32), ("theta_local", _f32), ("theta_global", _f32), ("eps", _f32), ("softcap", _f32),
        ("layer_global", _vp), ("attn_chunk", _i32), ("max_prompt", _i32), ("flags", _u32),
        ("recipe", _i32), ("head_dim_full", _i32), ("rope_angles_full", _i32), ("n_experts", _i32),
        ("expert_ffn", _i32), ("layer_kv_heads", _vp),
    ]


class ProfEntryC(C.Structure):
    """struct e4b_prof_entry (include/e4b.h)."""

    _fields_ = [("name", C.c_char * 40), ("us", _f32), ("n", _i32)]


FLAG_NO_GRAPH = 1
FLAG_STEP_PREFILL = 2
FLAG_KV_SCORE = 4
FLAG_LAYER_HIDDEN = 16


class MoeWeightsC(C.Structure):
    """struct e4b_moe_weights (include/e4b.h); every pointer is a device pointer."""

    _fields_ = [
        ("hidden", _i32), ("n_experts", _i32), ("expert_ffn", _i32), ("dense_ffn", _i32),
        ("eps", _f32), ("layer_scale", _f32),
        ("ffn_norm", _vp), ("router_scale", _vp), ("pre_ffw2", _vp), ("router_w", _vp), ("pes", _vp),
        ("dense_gate_up", _vp), ("exp_gate_up", _vp), ("dense_down", _vp), ("exp_down", _vp),
        ("post_ffw1", _vp), ("post_ffw2", _vp), ("post_ffw", _vp),
    ]

for _name, _res, _args in SIGNATURES:
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def last_error() -> str:
    msg = lib.e4b_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int, where: str) -> int:
    """Raise E4BError for a negative status, else return it."""
    if rc < 0:
        raise E4BError(rc, where, last_error())
    return rc


def exported_symbols() -> list[str]:
    return [n for n, _, _ in SIGNATURES]

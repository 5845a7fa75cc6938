"""ctypes binding of libzeromoe_hip.so (include/zeromoe.h).

The shared library is built in-tree by ``zeromoe_amd.build.build()``.  Loading
fails loudly when it is missing: there is no CPU fallback anywhere in the
product path.
"""
from __future__ import annotations

import ctypes as C
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libzeromoe_hip.so")

P, I, I32, I64, U64, F, SZ = C.c_void_p, C.c_int, C.c_int32, C.c_int64, C.c_uint64, C.c_float, C.c_size_t


class ZmTensor(C.Structure):
    _fields_ = [("type", C.c_int32), ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4), ("data", C.c_void_p)]


class ZmRouterSpec(C.Structure):
    _fields_ = [("gating", I32), ("n_experts", I32), ("topk", I32), ("n_groups", I32), ("n_groups_used", I32),
                ("weights_norm", I32), ("weights_scale", F)]


class ZmMoeLayer(C.Structure):
    _fields_ = [("H", I32), ("F", I32), ("n_slots", I32), ("router", ZmRouterSpec),
                ("type_gate", I32), ("type_up", I32), ("type_down", I32),
                ("w_gate", P), ("w_up", P), ("w_down", P),
                ("router_w", P), ("logit_bias", P), ("sel_bias", P), ("route_map", P), ("route_mask", P),
                ("F_shared", I32), ("type_shared", I32), ("ws_gate", P), ("ws_up", P), ("ws_down", P)]


class ZmExpertScratch(C.Structure):
    _fields_ = [("d_bad", P), ("d_x", P), ("d_gate", P), ("d_up", P), ("d_prod", P), ("d_down", P),
                ("cap_sd", SZ), ("cap_si", SZ), ("device_id", I32)]


class ZmColdLaneDesc(C.Structure):
    _fields_ = [("H", I32), ("F", I32), ("n_experts", I32), ("topk", I32),
                ("type_gate", I32), ("type_up", I32), ("type_down", I32),
                ("w_gate", P), ("w_up", P), ("w_down", P), ("n_slots", I32), ("route_map", P), ("route_mask", P),
                ("max_tokens", I32), ("n_threads", I32), ("scalar", I32)]


class ZmColdLaneStats(C.Structure):
    _fields_ = [("fork_ns", C.c_int64), ("compute_begin_ns", C.c_int64), ("compute_end_ns", C.c_int64),
                ("merge_ns", C.c_int64), ("vectorized", I32)]


_MM = (None, [P, P, P, I, I, I])
_MMS = (None, [P, P, P, I, I, I, P])
_XS = C.POINTER(ZmExpertScratch)

# name -> (restype, argtypes); every function declared in include/zeromoe.h
SIGNATURES = {
    "zm_init": (I, []),
    "zm_last_error": (C.c_char_p, []),
    "zm_version": (C.c_char_p, []),
    "zm_set_iq2xxs_grid": (I, [P]),
    "zm_iq2xxs_builtin_grid": (None, [P]),
    "zm_set_iq4nl_table": (I, [P]),
    "zm_set_iq3xxs_grid": (I, [P]),
    "zm_iq3xxs_builtin_grid": (None, [P]),
    "zm_iq4nl_builtin_table": (None, [P]),
    "zm_mul_mat_id_negative_skip": (I, []),
    "zm_mul_mat_id_negative_skip_batched": (I, []),
    "zm_mul_mat_id": (I, [C.POINTER(ZmTensor)] * 3 + [C.POINTER(ZmTensor), P, I]),
    "zm_mul_mat_id_launches": (U64, []),
    "zm_mul_mat_id_workspace_size": (SZ, [C.POINTER(ZmTensor)] * 4),
    "zm_mul_mat_id_set_workspace": (I, [P, P, SZ]),
    "zm_mul_mat_id_static": (I, [C.POINTER(ZmTensor)] * 3 + [C.POINTER(ZmTensor), P, I]),
    "zm_quantize_q8_K": (I, [P, I64, I64, P, P]),
    "zm_router": (I, [C.POINTER(ZmRouterSpec), P, P, P, P, P, I, P, P, P]),
    "zm_bucket": (I, [P, I, I, I, P, P, P, P, P, P]),
    "zm_block_dots": (I, [I, P, P, I, P, P, P]),
    "zm_moe_workspace_size": (SZ, [C.POINTER(ZmMoeLayer), I]),
    "zm_moe_status": (I, [C.POINTER(ZmMoeLayer), I, P, P]),
    "zm_debug_trace": (I, [P, I]),
    "launch_q2_K_matmul": _MM, "launch_q2_K_matmul_stream": _MMS,
    "launch_q3_K_matmul": _MM, "launch_q3_K_matmul_stream": _MMS,
    "launch_q4_K_matmul": _MM, "launch_q4_K_matmul_stream": _MMS,
    "launch_iq2_xxs_matmul": _MM, "launch_iq2_xxs_matmul_stream": _MMS,
    "zm_f32_matmul": (I, [I, P, P, P, I, I, I, P]),
    "zm_mul_mat_id_f32": (I, [C.POINTER(ZmTensor)] * 3 + [C.POINTER(ZmTensor), P, I]),
    "launch_expert_swiglu": (None, [P, P, P, I, F, I, P, P]),
    "launch_expert_scatter_accum": (None, [P, P, P, P, I, I, I, P]),
    "launch_expert_scatter_add": (None, [P, P, P, I, I, I, P]),
    "launch_q5_K_matmul": (None, [P, P, P, I, I, I]),
    "launch_q5_K_matmul_stream": (None, [P, P, P, I, I, I, P]),
    "launch_q6_K_matmul": (None, [P, P, P, I, I, I]),
    "launch_q6_K_matmul_stream": (None, [P, P, P, I, I, I, P]),
    "launch_iq4_xs_matmul": (None, [P, P, P, I, I, I]),
    "launch_iq3_xxs_matmul": (None, [P, P, P, I, I, I]),
    "launch_iq3_xxs_matmul_stream": (None, [P, P, P, I, I, I, P]),
    "launch_iq4_xs_matmul_stream": (None, [P, P, P, I, I, I, P]),
    "launch_q5_K_matmul_grouped": (C.c_bool, [P, P, P, I, C.c_size_t, I, I]),
    "launch_ggml_moe_unpack": (I, [P, P, P, P, I] + [C.c_size_t] * 7 + [P]),
    "launch_ggml_moe_unpack_scatter": (I, [P, P, P, P, P, I] + [C.c_size_t] * 7 + [P]),
    "launch_glm5next_router_topk": (None, [P, P, P, P, I, I, I, I, I, F, P]),
    "zm_expert_scratch_ensure": (I, [_XS, I, I, I, I]),
    "zm_expert_scratch_release": (None, [_XS]),
    "zm_expert_ffn_issue": (I, [_XS, P, SZ, I, I, P, I, I, I, P, P]),
    "zm_expert_ffn_finish_stage1": (I, [_XS, P, SZ, I, I, I, I, F, I, P]),
    "zm_expert_ffn_finish_stage2": (I, [_XS, P, I, I, P]),
    "zm_expert_bad_counts": (I, [_XS, P, I]),
    "zm_moe_forward": (I, [C.POINTER(ZmMoeLayer), P, P, I, P, P, P, P, SZ, P]),
    "zm_cold_lane_create": (P, [C.POINTER(ZmColdLaneDesc)]),
    "zm_cold_lane_destroy": (None, [P]),
    "zm_cold_lane_fork": (I, [P, P, P, P, I, P]),
    "zm_cold_lane_merge": (I, [P, P, I, P]),
    "zm_cold_lane_compute_host": (I, [P, P, P, P, I, P]),
    "zm_cold_lane_get_stats": (I, [P, C.POINTER(ZmColdLaneStats)]),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc}): {lib().zm_last_error().decode()}")

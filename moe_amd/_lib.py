"""ctypes binding of include/moe_hip.h (libmoe_hip.so, built in-tree).

Loading fails loudly when the library is missing: there is no CPU fallback
anywhere in this package.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmoe_hip.so"

MOE_OK, MOE_EINVAL, MOE_ENOMEM, MOE_EHIP, MOE_EUNSUP = 0, -1, -2, -3, -4
DT_F32, DT_F16, DT_Q4_0, DT_Q5_0, DT_Q8_0, DT_BF16 = 0, 1, 2, 6, 8, 30
GATE_SOFTMAX, GATE_SIGMOID = 0, 1
MODE_AUTO, MODE_EXACT, MODE_GEMV, MODE_MFMA = 0, 1, 2, 3

DT_NAMES = {DT_F32: "F32", DT_F16: "F16", DT_Q4_0: "Q4_0", DT_Q5_0: "Q5_0", DT_Q8_0: "Q8_0", DT_BF16: "BF16"}


class MoeError(RuntimeError):
    """A libmoe_hip call returned a non-zero status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (status {code})")
        self.code = code


class Tensor(C.Structure):
    _fields_ = [("dt", C.c_int32), ("rows", C.c_int32), ("cols", C.c_int32), ("_reserved", C.c_int32),
                ("region", C.c_uint64), ("offset", C.c_uint64)]


def absent() -> Tensor:
    return Tensor(dt=-1)


class LayerDesc(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("n_experts", C.c_int32), ("top_k", C.c_int32), ("gate", C.c_int32),
                ("norm_topk", C.c_int32), ("n_group", C.c_int32), ("topk_group", C.c_int32),
                ("routed_scale", C.c_float), ("router", Tensor), ("e_bias", Tensor),
                ("experts", C.POINTER(Tensor)), ("shared", Tensor * 3), ("shared_gate", Tensor)]


class RoutingC(C.Structure):
    _fields_ = [("disabled", C.POINTER(C.c_int32)), ("n_disabled", C.c_int32),
                ("forced", C.POINTER(C.c_int32)), ("n_forced", C.c_int32),
                ("temp", C.c_float), ("top_k", C.c_int32)]


class RouteC(C.Structure):
    _fields_ = [("expert", C.c_uint32), ("weight", C.c_float)]


class RecC(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dt", C.c_int32), ("_reserved", C.c_int32), ("slabs", C.c_uint64),
                ("rows", C.c_uint64), ("cols", C.c_uint64), ("offset", C.c_uint64), ("bytes", C.c_uint64)]


DT_Q6_REF = -2


# name -> (restype, argtypes); every function include/moe_hip.h declares.
PROTOTYPES = {
    "moe_ctx_create": (C.c_int, [C.c_int, C.POINTER(C.c_void_p)]),
    "moe_ctx_destroy": (None, [C.c_void_p]),
    "moe_upload": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.POINTER(C.c_uint64)]),
    "moe_region_ptr": (C.c_int, [C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p)]),
    "moe_layer_create": (C.c_int, [C.c_void_p, C.POINTER(LayerDesc), C.POINTER(C.c_void_p)]),
    "moe_layer_destroy": (None, [C.c_void_p]),
    "moe_layer_set_routing": (C.c_int, [C.c_void_p, C.POINTER(RoutingC)]),
    "moe_layer_reserve": (C.c_int, [C.c_void_p, C.c_int32]),
    "moe_layer_reserve_stream": (C.c_int, [C.c_void_p, C.c_int32, C.c_void_p]),
    "moe_layer_release_stream": (C.c_int, [C.c_void_p, C.c_void_p]),
    "moe_layer_workspace_size": (C.c_int, [C.c_void_p, C.c_int32, C.POINTER(C.c_uint64)]),
    "moe_layer_forward_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p,
                                            C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "moe_layer_forward_ws": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]),
    "moe_layer_set_mode": (C.c_int, [C.c_void_p, C.c_int]),
    "moe_layer_set_tiled": (C.c_int, [C.c_void_p, C.c_int]),
    "moe_layer_k": (C.c_int, [C.c_void_p]),
    "moe_layer_forward": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "moe_layer_route": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p]),
    "moe_last_error": (C.c_char_p, []),
    "moe_row_bytes": (C.c_uint64, [C.c_int32, C.c_uint64]),
    "moe_quantize_rows": (C.c_int, [C.c_int32, C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p]),
    "moe_dequant_rows": (C.c_int, [C.c_int32, C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p]),
    "moe_synth_normal": (C.c_int, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_double, C.c_double, C.c_void_p]),
    "moe_synth_quantized": (C.c_int, [C.c_uint64, C.c_uint64, C.c_int32, C.c_uint64, C.c_uint64, C.c_double,
                                      C.c_double, C.c_void_p]),
    "moe_debug_expf": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]),
    "moe_debug_decode_kernel": (C.c_int, [C.c_int32]),
    "moe_debug_mfma_kernel": (C.c_int, [C.c_int32]),
    "moe_layer_profile": (C.c_int, [C.c_void_p, C.c_int]),
    "moe_container_open": (C.c_int, [C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p)]),
    "moe_container_close": (None, [C.c_void_p]),
    "moe_container_kind": (C.c_int, [C.c_void_p]),
    "moe_container_count": (C.c_int64, [C.c_void_p]),
    "moe_container_rec": (C.c_int, [C.c_void_p, C.c_int64, C.POINTER(RecC)]),
    "moe_container_find": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(RecC)]),
    "moe_container_config": (C.c_char_p, [C.c_void_p]),
    "moe_gguf_rename": (C.c_int, [C.c_char_p, C.c_char_p, C.c_uint64]),
    "moe_upload_tensors": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.POINTER(C.c_uint64),
                                     C.POINTER(C.c_uint64), C.c_int64, C.POINTER(C.c_uint64),
                                     C.POINTER(C.c_uint64)]),
    "moe_layer_stage_times": (C.c_int, [C.c_void_p, C.POINTER(C.c_double), C.POINTER(C.c_uint64)]),
    "moe_linear_create": (C.c_int, [C.c_void_p, C.POINTER(Tensor), C.POINTER(C.c_void_p)]),
    "moe_linear_destroy": (None, [C.c_void_p]),
    "moe_linear_workspace_size": (C.c_int, [C.c_void_p, C.c_int32, C.POINTER(C.c_uint64)]),
    "moe_linear_forward": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_uint64, C.c_void_p]),
    "moe_embed_rows": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_void_p, C.c_int32, C.c_void_p,
                                 C.c_void_p]),
    "moe_rmsnorm": (C.c_int, [C.c_void_p, C.c_int64, C.c_void_p, C.c_int32, C.c_int32, C.c_float, C.c_void_p,
                              C.c_int64, C.c_void_p]),
    "moe_rope": (C.c_int, [C.c_void_p, C.c_int32, C.c_int64, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_void_p,
                           C.c_void_p, C.c_int32, C.c_void_p]),
    "moe_rope_inv_freqs": (C.c_int, [C.c_int32, C.c_float, C.c_float, C.c_uint64, C.c_float, C.c_float, C.c_float,
                                     C.c_float, C.c_int32, C.c_void_p]),
    "moe_add_bias": (C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p, C.c_int32, C.c_void_p]),
    "moe_scatter_rows": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int64, C.c_void_p, C.c_int64, C.c_void_p,
                                   C.c_void_p]),
    "moe_mla_kv_store": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int64, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                   C.c_int32, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "moe_attention": (C.c_int, [C.c_void_p, C.c_int64, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                C.c_float, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p, C.c_int32,
                                C.c_int32, C.c_void_p, C.c_int64, C.c_void_p]),
    "moe_argmax": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_void_p]),
}

STAGES = ("router", "gating", "dispatch", "expert_up", "expert_down", "combine", "encode")

_lib = None


def lib() -> C.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m moe_amd.build` "
                               "(there is no CPU fallback)")
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


# The bench's measurement probes (moe_amd/diag/moe_diag.h), a library apart
# from the layer's.
DIAG_PATH = LIB_PATH.with_name("libmoe_diag.so")
DIAG_PROTOTYPES = {
    "moe_diag_last_error": (C.c_char_p, []),
    "moe_debug_grid_barrier": (C.c_int, [C.c_int32, C.c_int32, C.c_void_p, C.c_void_p]),
    "moe_debug_mfma_valu": (C.c_int, [C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_void_p,
                                      C.c_void_p]),
    "moe_debug_stream_read": (C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p]),
}
_diag = None


def diag() -> C.CDLL:
    """The probes library (raises if it has not been built)."""
    global _diag
    if _diag is None:
        if not DIAG_PATH.exists():
            raise RuntimeError(f"{DIAG_PATH} is missing: build it with `python -m moe_amd.build`")
        handle = C.CDLL(str(DIAG_PATH))
        for name, (res, args) in DIAG_PROTOTYPES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _diag = handle
    return _diag


def diag_check(code: int, what: str = "") -> None:
    if code != MOE_OK:
        msg = diag().moe_diag_last_error().decode(errors="replace")
        raise MoeError(code, f"{what}: {msg}" if what else msg)


def check(code: int, what: str = "") -> None:
    if code != MOE_OK:
        msg = lib().moe_last_error().decode(errors="replace")
        raise MoeError(code, f"{what}: {msg}" if what else msg)

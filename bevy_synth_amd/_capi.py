"""ctypes binding of the C ABI in include/sparseconv.h (libsparseconv.so).

The library is built in-tree by ``__graft_entry__.build()`` (or
``make -C bevy_synth_amd/csrc``).  There is no fallback: if the shared object
is missing, importing anything that needs it raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsparseconv.so")

SC_OK = 0
SC_DTYPE_F32 = 0
SC_DTYPE_BF16 = 1
SC_DTYPE_I8 = 2
SC_DTYPE_F16 = 3

# Every symbol include/sparseconv.h declares (checked by tests/test_abi.py).
EXPORTED = (
    "sc_abi_version", "sc_status_string", "sc_last_error", "sc_validate_config",
    "sc_kernel_rows", "sc_kernel_offsets", "sc_neighbor_map_workspace_size",
    "sc_neighbor_map_build", "sc_neighbor_map_check", "sc_subm_conv_forward",
    "sc_subm_conv_forward_fused",
    "sc_layer_norm", "sc_add", "sc_subdivision_workspace_size", "sc_subdivision_build",
    "sc_gather_rows", "sc_c2s_skip_add", "sc_convert",
    "sc_conv_plan_size", "sc_conv_plan_build", "sc_conv_plan_order", "sc_conv_plan_tables",
    "sc_subm_conv_forward_planned",
    "sc_conv_weight_pack_size", "sc_conv_weight_pack",
    "sc_subdivision_build_static", "sc_conv_plan_check", "sc_conv_epilogue_workspace_size",
    "sc_subdivision_build_indexed", "sc_linear_skinny", "sc_linear_forward",
    "sc_subdivision_logits_finish", "sc_conv_child_plan_size", "sc_conv_child_plan_build",
    "sc_subm_conv_forward_child_planned", "sc_linear_child_plan_build", "sc_linear_forward_child_planned",
)


class ScConvConfig(ctypes.Structure):
    """sc_conv_config (mirror of SparseSubmConvConfig, crates/burn_flex_gmm/src/lib.rs:5-17)."""

    _fields_ = [
        ("in_channels", ctypes.c_int64),
        ("out_channels", ctypes.c_int64),
        ("kernel_d", ctypes.c_int64),
        ("kernel_h", ctypes.c_int64),
        ("kernel_w", ctypes.c_int64),
        ("in_channels_per_group", ctypes.c_int64),
        ("out_channels_per_group", ctypes.c_int64),
        ("groups", ctypes.c_int64),
        ("axis_order", ctypes.c_int32 * 3),
        ("axis_sign", ctypes.c_int32 * 3),
    ]


class ScConvEpilogue(ctypes.Structure):
    """sc_conv_epilogue: fused + bias -> LayerNorm -> SiLU -> + residual."""

    _fields_ = [
        ("residual", ctypes.c_void_p),
        ("layer_norm", ctypes.c_int),
        ("ln_weight", ctypes.c_void_p),
        ("ln_bias", ctypes.c_void_p),
        ("ln_eps", ctypes.c_float),
        ("silu", ctypes.c_int),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("child_rows", ctypes.c_void_p),
        ("n_child_rows", ctypes.c_int64),
        ("skip_parent", ctypes.c_void_p),
        ("skip_index", ctypes.c_void_p),
        ("skip_parent_rows", ctypes.c_int64),
        ("skip_parent_channels", ctypes.c_int64),
        ("child_count", ctypes.c_void_p),
    ]


class SparseConvError(RuntimeError):
    """A non-zero sc_status; ``status`` is the code, the message is sc_last_error()."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status
        self.message = message


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run __graft_entry__.build() or "
            "make -C bevy_synth_amd/csrc (the HIP library has no fallback)")
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    i64 = ctypes.c_int64
    i32 = ctypes.c_int
    cfgp = ctypes.POINTER(ScConvConfig)
    sizep = ctypes.POINTER(ctypes.c_size_t)
    L.sc_abi_version.restype = i32
    L.sc_status_string.argtypes = [i32]
    L.sc_status_string.restype = ctypes.c_char_p
    L.sc_last_error.restype = ctypes.c_char_p
    L.sc_validate_config.argtypes = [cfgp]
    L.sc_kernel_rows.argtypes = [cfgp, ctypes.POINTER(i64)]
    L.sc_kernel_offsets.argtypes = [cfgp, P, i64]
    L.sc_neighbor_map_workspace_size.argtypes = [i64, sizep]
    L.sc_neighbor_map_build.argtypes = [cfgp, P, i64, i64, P, P, ctypes.c_size_t, P]
    L.sc_neighbor_map_check.argtypes = [P, P]
    L.sc_subm_conv_forward.argtypes = [cfgp, i32, P, i64, P, i64, i32, P, P, P, P, i32, P, P]
    L.sc_subm_conv_forward_fused.argtypes = [cfgp, i32, P, i64, P, i64, i32, P, P, P,
                                             ctypes.POINTER(ScConvEpilogue), i32, P, P]
    L.sc_conv_plan_size.argtypes = [i64, i64, sizep]
    L.sc_conv_plan_build.argtypes = [cfgp, P, i64, P, i64, P, ctypes.c_size_t, P]
    L.sc_conv_plan_order.argtypes = [cfgp, P, i64, i64, P, ctypes.c_size_t, P]
    L.sc_conv_plan_tables.argtypes = [cfgp, P, i64, i64, P, ctypes.c_size_t, P]
    L.sc_subm_conv_forward_planned.argtypes = [cfgp, i32, P, i64, P, i64, i32, P, P, P, P,
                                               ctypes.POINTER(ScConvEpilogue), i32, P, P, P]
    L.sc_conv_plan_check.argtypes = [P, P]
    L.sc_conv_epilogue_workspace_size.argtypes = [cfgp, i32, i64, i32, ctypes.POINTER(ScConvEpilogue), sizep]
    L.sc_conv_weight_pack_size.argtypes = [cfgp, i32, sizep]
    L.sc_conv_weight_pack.argtypes = [cfgp, i32, P, P, P]
    L.sc_layer_norm.argtypes = [i32, P, i64, i64, P, P, ctypes.c_float, i32, i32, P, P]
    L.sc_add.argtypes = [i32, P, P, i64, P, P]
    L.sc_subdivision_workspace_size.argtypes = [i64, sizep]
    L.sc_subdivision_build.argtypes = [P, P, P, P, i64, P, P, P, P, P, ctypes.c_size_t, P]
    L.sc_subdivision_build_indexed.argtypes = [P, P, P, P, i64, P, P, P, P, P, P, ctypes.c_size_t, P]
    L.sc_linear_forward.argtypes = [i32, P, i64, i64, i64, i32, P, P, P, ctypes.POINTER(ScConvEpilogue), i32,
                                    P, P]
    L.sc_linear_skinny.argtypes = [i32, P, i64, i64, P, P, i64, P, P]
    L.sc_subdivision_logits_finish.argtypes = [P, i64, i32, i32, P]
    L.sc_conv_child_plan_size.argtypes = [i64, i64, i64, sizep]
    L.sc_conv_child_plan_build.argtypes = [cfgp, P, P, i64, P, i64, P, ctypes.c_size_t, P]
    L.sc_subm_conv_forward_child_planned.argtypes = [cfgp, i32, P, i64, P, i64, i32, P, P, P, P,
                                                     ctypes.POINTER(ScConvEpilogue), i32, P, P, P]
    L.sc_linear_child_plan_build.argtypes = [i64, P, i64, P, ctypes.c_size_t, P]
    L.sc_linear_forward_child_planned.argtypes = [i32, P, i64, i64, i64, i32, P, P, P,
                                                  ctypes.POINTER(ScConvEpilogue), i32, P, P, P]
    L.sc_subdivision_build_static.argtypes = [P, P, P, P, i64, P, P, P, P, P]
    L.sc_gather_rows.argtypes = [i32, P, i64, i64, i64, P, i64, P, P]
    L.sc_c2s_skip_add.argtypes = [i32, P, i64, i64, i32, P, i64, i64, P, P]
    L.sc_convert.argtypes = [i32, P, i32, P, i64, P]
    for name in EXPORTED:
        fn = getattr(L, name)
        if fn.restype is None or fn.restype is ctypes.c_int:
            if name not in ("sc_status_string", "sc_last_error"):
                fn.restype = i32
    _lib = L
    return L


def check(status: int) -> None:
    if status != SC_OK:
        msg = load().sc_last_error().decode("utf-8", "replace")
        raise SparseConvError(status, msg)

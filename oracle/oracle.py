"""numpy front end to the CPU oracle (oracle/sc_oracle.c -> oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker for the HIP product.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.

Each wrapper names the reference function it restates (the C file carries the
file:line citations).  Integer semantics (maps, child coords, pairs) are exact;
floating-point functions follow the reference's f32 operation order, except
``conv_ref_f64`` which is the fp64 definition used as the tolerance anchor.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

INVALID_NEIGHBOR_ROW = -1  # crates/burn_flex_gmm/src/lib.rs:3


class _Cfg(ctypes.Structure):
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


@dataclass(frozen=True)
class OracleConfig:
    """SparseSubmConvConfig, crates/burn_flex_gmm/src/lib.rs:5-17."""

    in_channels: int
    out_channels: int
    kernel_d: int = 3
    kernel_h: int = 3
    kernel_w: int = 3
    in_channels_per_group: Optional[int] = None
    out_channels_per_group: Optional[int] = None
    groups: int = 1
    axis_order: Sequence[int] = (0, 1, 2)
    axis_sign: Sequence[int] = (1, 1, 1)

    def c(self) -> _Cfg:
        cin_g = self.in_channels_per_group
        cout_g = self.out_channels_per_group
        if cin_g is None:
            cin_g = self.in_channels // self.groups
        if cout_g is None:
            cout_g = self.out_channels // self.groups
        cfg = _Cfg()
        cfg.in_channels = self.in_channels
        cfg.out_channels = self.out_channels
        cfg.kernel_d = self.kernel_d
        cfg.kernel_h = self.kernel_h
        cfg.kernel_w = self.kernel_w
        cfg.in_channels_per_group = cin_g
        cfg.out_channels_per_group = cout_g
        cfg.groups = self.groups
        for j in range(3):
            cfg.axis_order[j] = int(self.axis_order[j])
            cfg.axis_sign[j] = int(self.axis_sign[j])
        return cfg

    @property
    def kernel_rows(self) -> int:
        return self.kernel_d * self.kernel_h * self.kernel_w


def build() -> str:
    """Compile liboracle.so with oracle/Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        cfgp = ctypes.POINTER(_Cfg)
        L.orc_validate_config.argtypes = [cfgp]
        L.orc_kernel_rows.argtypes = [cfgp]
        L.orc_kernel_rows.restype = i64
        L.orc_kernel_layout.argtypes = [cfgp, P]
        L.orc_kernel_layout.restype = i64
        L.orc_build_neighbor_rows.argtypes = [cfgp, P, i64, i64, ctypes.c_int, P]
        L.orc_build_neighbor_rows_scan.argtypes = [cfgp, P, i64, P]
        L.orc_pack_flex_weight.argtypes = [cfgp, P, P]
        L.orc_conv_flex_precomputed.argtypes = [cfgp, P, P, P, i64, P, i64, P, P]
        L.orc_conv_legacy.argtypes = [cfgp, P, P, P, i64, P, P]
        L.orc_conv_ref_f64.argtypes = [cfgp, P, P, P, P, i64, P, i64, P]
        L.orc_bf16_round.argtypes = [P, P, i64]
        L.orc_f16_round.argtypes = [P, P, i64]
        L.orc_set_num_threads.argtypes = [ctypes.c_int]
        L.orc_layer_norm.argtypes = [P, i64, i64, P, P, ctypes.c_float]
        L.orc_silu.argtypes = [P, i64]
        L.orc_subdivision_active.argtypes = [P, i64, P, P]
        L.orc_subdivision_active.restype = i64
        L.orc_subdivide_expand.argtypes = [P, P, i64, P, P]
        L.orc_channel2spatial.argtypes = [P, P, i64, i64, P, P, P]
        L.orc_channel2spatial.restype = i64
        L.orc_repeat_interleave.argtypes = [P, i64, i64, i64, P]
        L.orc_c2s_block.argtypes = [P, P, i64, i64, i64, P, P, P, cfgp, P, P, cfgp, P, P,
                                    ctypes.c_float, P, P]
        L.orc_c2s_block.restype = i64
        L.orc_conv_flex_fast.argtypes = [cfgp, P, P, P, i64, P, i64, P]
        L.orc_fast_set_num_threads.argtypes = [ctypes.c_int]
        L.orc_lcg_fill.argtypes = [ctypes.c_uint64, i64, P]
        L.orc_lcg_fill.restype = ctypes.c_uint64
        _lib = L
    return _lib


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"oracle {what} failed with code {rc}")


def _u32_coords(coords) -> np.ndarray:
    c = np.ascontiguousarray(np.asarray(coords).reshape(-1, 4))
    return np.ascontiguousarray(c.astype(np.uint32))


def kernel_layout(cfg: OracleConfig) -> np.ndarray:
    """kernel_layout, crates/burn_flex_gmm/src/lib.rs:727-752 -> [K,3] i32."""
    out = np.zeros((cfg.kernel_rows, 3), dtype=np.int32)
    k = lib().orc_kernel_layout(ctypes.byref(cfg.c()), _p(out))
    if k < 0:
        raise ValueError("invalid sparse conv config")
    return out


def validate_config(cfg: OracleConfig) -> bool:
    return lib().orc_validate_config(ctypes.byref(cfg.c())) == 0


def build_neighbor_rows(cfg: OracleConfig, coords, query_rows: Optional[int] = None,
                        lowest_row_on_duplicate: bool = True) -> np.ndarray:
    """build_neighbor_rows, crates/burn_flex_gmm/src/lib.rs:69-109 -> [n_q, K] i32.

    lowest_row_on_duplicate=False gives the CPU HashMap semantics (last row
    wins); True gives the device semantics (lowest row), which is what the
    HIP product implements.  Identical for unique coords.
    """
    c = _u32_coords(coords)
    n = c.shape[0]
    q = n if query_rows is None else int(query_rows)
    out = np.full((q, cfg.kernel_rows), -1, dtype=np.int32)
    _check(lib().orc_build_neighbor_rows(ctypes.byref(cfg.c()), _p(c), n, q,
                                         int(lowest_row_on_duplicate), _p(out)),
           "build_neighbor_rows")
    return out


def build_neighbor_rows_scan(cfg: OracleConfig, coords) -> np.ndarray:
    """Brute-force scan, neighbor_rows_from_coords_kernel semantics
    (crates/burn_flex_gmm/src/wgpu/neighbor_kernels.rs:3-46).  O(n^2 K)."""
    c = _u32_coords(coords)
    n = c.shape[0]
    out = np.full((n, cfg.kernel_rows), -1, dtype=np.int32)
    _check(lib().orc_build_neighbor_rows_scan(ctypes.byref(cfg.c()), _p(c), n, _p(out)),
           "scan")
    return out


def pack_flex_weight(cfg: OracleConfig, weight: np.ndarray) -> np.ndarray:
    """pack_flex_weight, crates/burn_flex_gmm/src/lib.rs:377-426."""
    w = np.ascontiguousarray(weight, dtype=np.float32).reshape(-1)
    cc = cfg.c()
    out = np.zeros(cc.groups * cfg.kernel_rows * cc.in_channels_per_group
                   * cc.out_channels_per_group, dtype=np.float32)
    _check(lib().orc_pack_flex_weight(ctypes.byref(cc), _p(w), _p(out)), "pack")
    return out


def set_num_threads(n: int) -> None:
    """Threads of conv_flex_precomputed's gather and sgemm (1 = the reference's
    single-threaded matrixmultiply; more = the all-cores CPU baseline).
    Results do not depend on it."""
    lib().orc_set_num_threads(int(n))


def conv_flex_precomputed(cfg: OracleConfig, weight, bias, inp, nbr,
                          packed: Optional[np.ndarray] = None) -> np.ndarray:
    """sparse_subm_conv_forward_flex_precomputed, crates/burn_flex_gmm/src/lib.rs:242-375."""
    w = np.ascontiguousarray(weight, dtype=np.float32).reshape(-1)
    b = np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
    x = np.ascontiguousarray(inp, dtype=np.float32).reshape(-1, cfg.in_channels)
    m = np.ascontiguousarray(nbr, dtype=np.int32).reshape(-1, cfg.kernel_rows)
    out = np.zeros((m.shape[0], cfg.out_channels), dtype=np.float32)
    pk = None if packed is None else np.ascontiguousarray(packed, dtype=np.float32)
    _check(lib().orc_conv_flex_precomputed(ctypes.byref(cfg.c()), _p(w), _p(b), _p(x),
                                           x.shape[0], _p(m), m.shape[0], _p(pk), _p(out)),
           "conv_flex_precomputed")
    return out


def conv_flex_fast(cfg: OracleConfig, weight, bias, inp, nbr, packed: Optional[np.ndarray] = None,
                   threads: int = 1) -> np.ndarray:
    """Timing only (the CPU baseline): conv_flex_precomputed's gather with a
    packed, register-blocked FMA sgemm of matrixmultiply's kind
    (oracle/sc_fastgemm.c), on `threads` OpenMP threads.  Equal to
    conv_flex_precomputed up to float rounding; never a parity checker."""
    b = np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
    x = np.ascontiguousarray(inp, dtype=np.float32).reshape(-1, cfg.in_channels)
    m = np.ascontiguousarray(nbr, dtype=np.int32).reshape(-1, cfg.kernel_rows)
    pk = pack_flex_weight(cfg, weight) if packed is None else np.ascontiguousarray(packed, dtype=np.float32)
    out = np.zeros((m.shape[0], cfg.out_channels), dtype=np.float32)
    lib().orc_fast_set_num_threads(int(threads))
    _check(lib().orc_conv_flex_fast(ctypes.byref(cfg.c()), _p(pk), _p(b), _p(x), x.shape[0], _p(m), m.shape[0],
                                    _p(out)), "conv_flex_fast")
    return out


def conv_flex(cfg: OracleConfig, weight, bias, coords, inp) -> np.ndarray:
    """sparse_subm_conv_forward_flex, crates/burn_flex_gmm/src/lib.rs:111-131
    (map with the CPU HashMap semantics, then the precomputed path)."""
    nbr = build_neighbor_rows(cfg, coords, lowest_row_on_duplicate=False)
    return conv_flex_precomputed(cfg, weight, bias, inp, nbr)


def conv_legacy(cfg: OracleConfig, weight, bias, coords, inp) -> np.ndarray:
    """sparse_subm_conv_forward_legacy, crates/burn_flex_gmm/src/lib.rs:428-510."""
    c = _u32_coords(coords)
    w = np.ascontiguousarray(weight, dtype=np.float32).reshape(-1)
    b = np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
    x = np.ascontiguousarray(inp, dtype=np.float32).reshape(-1, cfg.in_channels)
    out = np.zeros((c.shape[0], cfg.out_channels), dtype=np.float32)
    _check(lib().orc_conv_legacy(ctypes.byref(cfg.c()), _p(w), _p(b), _p(c), c.shape[0],
                                 _p(x), _p(out)), "conv_legacy")
    return out


def conv_ref_f64(cfg: OracleConfig, weight, bias, inp, nbr,
                 w_scale: Optional[np.ndarray] = None) -> np.ndarray:
    """fp64 sum of the definition (sparse_conv_kernels.rs:5-46) over a map."""
    w = np.ascontiguousarray(weight, dtype=np.float32).reshape(-1)
    b = np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
    x = np.ascontiguousarray(inp, dtype=np.float32).reshape(-1, cfg.in_channels)
    m = np.ascontiguousarray(nbr, dtype=np.int32).reshape(-1, cfg.kernel_rows)
    s = None if w_scale is None else np.ascontiguousarray(w_scale, dtype=np.float32)
    out = np.zeros((m.shape[0], cfg.out_channels), dtype=np.float64)
    _check(lib().orc_conv_ref_f64(ctypes.byref(cfg.c()), _p(w), _p(s), _p(b), _p(x),
                                  x.shape[0], _p(m), m.shape[0], _p(out)), "conv_ref_f64")
    return out


def conv_gemm_f64(cfg: OracleConfig, weight, bias, inp, nbr,
                  w_scale: Optional[np.ndarray] = None, chunk: int = 1024) -> np.ndarray:
    """conv_ref_f64's definition (bias + scale * sum over valid neighbours) as an
    fp64 im2col GEMM in numpy, for the sampled checks at full size (pinned
    equal to conv_ref_f64 in tests/test_oracle.py).  Map entries outside
    [0, rows of inp) are absent."""
    K = cfg.kernel_rows
    g = cfg.groups
    cin_g, cout_g = cfg.in_channels // g, cfg.out_channels // g
    x = np.asarray(inp, dtype=np.float64).reshape(-1, cfg.in_channels)
    n = x.shape[0]
    xz = np.vstack([x, np.zeros((1, cfg.in_channels))])
    m = np.asarray(nbr, dtype=np.int64).reshape(-1, K)
    m = np.where((m >= 0) & (m < n), m, n)
    w = np.asarray(weight, dtype=np.float64).reshape(cfg.out_channels, K * cin_g)
    out = np.zeros((m.shape[0], cfg.out_channels), dtype=np.float64)
    for r0 in range(0, m.shape[0], chunk):
        rows = xz[m[r0:r0 + chunk]]                      # [R, K, Cin]
        for gi in range(g):
            cols = rows[:, :, gi * cin_g:(gi + 1) * cin_g].reshape(rows.shape[0], K * cin_g)
            out[r0:r0 + chunk, gi * cout_g:(gi + 1) * cout_g] = cols @ w[gi * cout_g:(gi + 1) * cout_g].T
    if w_scale is not None:
        out *= np.asarray(w_scale, dtype=np.float64).reshape(1, -1)
    return out + np.asarray(bias, dtype=np.float64).reshape(1, -1)


def bf16_round(x) -> np.ndarray:
    """bf16_round_to_f32, crates/burn_flex_gmm/src/wgpu.rs:57-67."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(a)
    lib().orc_bf16_round(_p(a), _p(out), a.size)
    return out


def f16_round(x) -> np.ndarray:
    """quantize_f16_inplace / quantize_f16_tensor_wgpu (burn_trellis
    sparse_decoder_wgpu_ops.rs:1722-1726, 1082-1088): f32 -> f16 (RNE) -> f32."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(a)
    lib().orc_f16_round(_p(a), _p(out), a.size)
    return out


def layer_norm(x, weight=None, bias=None, eps: float = 1e-6) -> np.ndarray:
    """layer_norm_inplace, burn_trellis sparse_decoder_wgpu_ops.rs:1642-1711."""
    a = np.array(x, dtype=np.float32, copy=True, order="C")
    rows, ch = a.shape
    w = None if weight is None else np.ascontiguousarray(weight, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().orc_layer_norm(_p(a), rows, ch, _p(w), _p(b), ctypes.c_float(eps))
    return a


def silu(x) -> np.ndarray:
    """silu_inplace, burn_trellis sparse_decoder_wgpu_ops.rs:1713-1720."""
    a = np.array(x, dtype=np.float32, copy=True, order="C")
    lib().orc_silu(_p(a), a.size)
    return a


def subdivision_active(logits, thresholds) -> np.ndarray:
    """logits_to_mask + argwhere order (sparse_decoder_wgpu_ops.rs:885-993,1765-1811)
    -> [A,2] i32 (parent, child)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1, 8)
    th = np.ascontiguousarray(thresholds, dtype=np.float32).reshape(8)
    a = lib().orc_subdivision_active(_p(lg), lg.shape[0], _p(th), None)
    out = np.zeros((a, 2), dtype=np.int32)
    lib().orc_subdivision_active(_p(lg), lg.shape[0], _p(th), _p(out))
    return out


def subdivide_expand(parent_coords, pairs):
    """expand_subdivision_coords_and_linear_indices_wgpu
    (sparse_decoder_wgpu_ops.rs:996-1054) -> (child coords [A,4] u32, linear_idx [A] i32)."""
    pc = _u32_coords(parent_coords)
    pr = np.ascontiguousarray(pairs, dtype=np.int32).reshape(-1, 2)
    a = pr.shape[0]
    cc = np.zeros((a, 4), dtype=np.uint32)
    li = np.zeros(a, dtype=np.int32)
    lib().orc_subdivide_expand(_p(pc), _p(pr), a, _p(cc), _p(li))
    return cc, li


def channel2spatial(coords, feats, in_channels: int, mask):
    """channel2spatial, sparse_decoder_wgpu_ops.rs:1999-2054."""
    c = _u32_coords(coords)
    f = np.ascontiguousarray(feats, dtype=np.float32).reshape(-1, in_channels)
    m = np.ascontiguousarray(mask, dtype=np.uint8).reshape(-1, 8)
    a = int(m.sum())
    oc = np.zeros((a, 4), dtype=np.uint32)
    of = np.zeros((a, in_channels // 8), dtype=np.float32)
    got = lib().orc_channel2spatial(_p(c), _p(f), c.shape[0], in_channels, _p(m), _p(oc), _p(of))
    assert got == a
    return oc, of


def repeat_interleave(feats, rep: int) -> np.ndarray:
    """repeat_interleave_channels, sparse_decoder_wgpu_ops.rs:2056-2076."""
    f = np.ascontiguousarray(feats, dtype=np.float32)
    rows, ch = f.shape
    out = np.zeros((rows, ch * rep), dtype=np.float32)
    lib().orc_repeat_interleave(_p(f), rows, ch, rep, _p(out))
    return out


def c2s_block(parent_coords, parent_feats, mask, norm1_w, norm1_b, conv1: OracleConfig, w1, b1,
              conv2: OracleConfig, w2, b2, eps: float = 1e-6):
    """Host C2S upsample block, sparse_decoder_runtime_impl.rs:1236-1343 (fp16 off).
    Returns (child coords [A,4] u32, out [A, Cout] f32)."""
    pc = _u32_coords(parent_coords)
    pf = np.ascontiguousarray(parent_feats, dtype=np.float32)
    p_rows, in_ch = pf.shape
    out_ch = conv2.out_channels
    m = np.ascontiguousarray(mask, dtype=np.uint8).reshape(-1, 8)
    a = int(m.sum())
    cc = np.zeros((a, 4), dtype=np.uint32)
    out = np.zeros((a, out_ch), dtype=np.float32)
    arrs = [np.ascontiguousarray(v, dtype=np.float32) for v in (norm1_w, norm1_b, w1, b1, w2, b2)]
    got = lib().orc_c2s_block(_p(pc), _p(pf), p_rows, in_ch, out_ch, _p(m), _p(arrs[0]),
                              _p(arrs[1]), ctypes.byref(conv1.c()), _p(arrs[2]), _p(arrs[3]),
                              ctypes.byref(conv2.c()), _p(arrs[4]), _p(arrs[5]),
                              ctypes.c_float(eps), _p(cc), _p(out))
    if got < 0:
        raise RuntimeError(f"oracle c2s_block failed with code {-got}")
    return cc, out


class Lcg:
    """The reference tests' LCG, crates/burn_flex_gmm/src/lib.rs:764-778."""

    def __init__(self, seed: int):
        self.state = (int(seed) | 1) & 0xFFFFFFFFFFFFFFFF

    def next_f32(self, n: int) -> np.ndarray:
        out = np.zeros(n, dtype=np.float32)
        self.state = lib().orc_lcg_fill(ctypes.c_uint64(self.state), n, _p(out))
        return out

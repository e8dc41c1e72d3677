"""Device operator API of the sparse-conv path, over the C ABI.

Mirrors burn_flex_gmm's public operator surface (crates/burn_flex_gmm/src/
lib.rs and wgpu.rs:405-427) with torch tensors as the device buffers:

===============================================  ==========================================
reference (Rust)                                  here
===============================================  ==========================================
SparseSubmConvConfig (lib.rs:5-17)                SparseSubmConvConfig
kernel_rows (lib.rs:59-67)                        kernel_rows
kernel_layout / kernel_offsets (lib.rs:727-752)   kernel_offsets
neighbor_rows_tensor_from_coords_tensor           neighbor_rows_tensor_from_coords_tensor
  (wgpu/neighbor.rs:977-1006)
sparse_subm_conv_forward_wgpu[_with_config]       sparse_subm_conv_forward
  (wgpu/sparse_conv.rs:310-367)
layer_norm_affine[_silu]_forward_wgpu             layer_norm
  (wgpu/ops.rs:162-446)
===============================================  ==========================================

Errors: the reference returns ``Result<_, String>``; here a failing call
raises ``SparseConvError`` carrying the status and the same kind of message.
All work is queued on the current torch stream; nothing synchronises except
where documented (the map status check, the subdivision child count).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Optional, Sequence, Tuple

import numpy as np
import torch

from . import _capi
from ._capi import SparseConvError, check

INVALID_NEIGHBOR_ROW = -1

_DTYPES = {
    torch.float32: _capi.SC_DTYPE_F32,
    torch.bfloat16: _capi.SC_DTYPE_BF16,
    torch.int8: _capi.SC_DTYPE_I8,
    torch.float16: _capi.SC_DTYPE_F16,
}


def _dt(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise SparseConvError(3, f"unsupported dtype {t.dtype}") from None


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _require_cuda(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise SparseConvError(2, f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise SparseConvError(2, f"{name} must be contiguous")


@dataclass(frozen=True)
class SparseSubmConvConfig:
    """SparseSubmConvConfig, crates/burn_flex_gmm/src/lib.rs:5-17."""

    in_channels: int
    out_channels: int
    kernel_d: int = 3
    kernel_h: int = 3
    kernel_w: int = 3
    in_channels_per_group: Optional[int] = None
    out_channels_per_group: Optional[int] = None
    groups: int = 1
    axis_order: Sequence[int] = field(default=(0, 1, 2))
    axis_sign: Sequence[int] = field(default=(1, 1, 1))

    def to_c(self) -> _capi.ScConvConfig:
        c = _capi.ScConvConfig()
        c.in_channels = self.in_channels
        c.out_channels = self.out_channels
        c.kernel_d = self.kernel_d
        c.kernel_h = self.kernel_h
        c.kernel_w = self.kernel_w
        c.in_channels_per_group = (self.in_channels // self.groups
                                   if self.in_channels_per_group is None
                                   else self.in_channels_per_group)
        c.out_channels_per_group = (self.out_channels // self.groups
                                    if self.out_channels_per_group is None
                                    else self.out_channels_per_group)
        c.groups = self.groups
        for j in range(3):
            c.axis_order[j] = int(self.axis_order[j])
            c.axis_sign[j] = int(self.axis_sign[j])
        return c


def validate_config(cfg: SparseSubmConvConfig) -> None:
    check(_capi.load().sc_validate_config(ctypes.byref(cfg.to_c())))


def kernel_rows(cfg: SparseSubmConvConfig) -> int:
    out = ctypes.c_int64()
    check(_capi.load().sc_kernel_rows(ctypes.byref(cfg.to_c()), ctypes.byref(out)))
    return out.value


def kernel_offsets(cfg: SparseSubmConvConfig) -> np.ndarray:
    k = kernel_rows(cfg)
    out = np.zeros((k, 3), dtype=np.int32)
    check(_capi.load().sc_kernel_offsets(ctypes.byref(cfg.to_c()),
                                         out.ctypes.data_as(ctypes.c_void_p), k))
    return out


def neighbor_map_workspace_bytes(n_rows: int) -> int:
    out = ctypes.c_size_t()
    check(_capi.load().sc_neighbor_map_workspace_size(int(n_rows), ctypes.byref(out)))
    return out.value


class NeighborMapWorkspace:
    """Caller-owned workspace for the map build, grown on demand (the
    reference caches per-device tensors in a thread-local map,
    crates/burn_flex_gmm/src/wgpu.rs:349-382)."""

    def __init__(self, device=None):
        self.device = torch.device("cuda") if device is None else torch.device(device)
        self.buf = torch.empty(0, dtype=torch.uint8, device=self.device)

    def get(self, n_rows: int) -> torch.Tensor:
        need = neighbor_map_workspace_bytes(n_rows)
        if self.buf.numel() < need:
            self.buf = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self.buf


def neighbor_map_build_into(cfg: SparseSubmConvConfig, coords: torch.Tensor, out: torch.Tensor,
                            workspace: torch.Tensor, query_rows: Optional[int] = None) -> None:
    """Stream-ordered map build into a preallocated ``out`` [query_rows, K]."""
    n = coords.shape[0]
    q = n if query_rows is None else int(query_rows)
    check(_capi.load().sc_neighbor_map_build(
        ctypes.byref(cfg.to_c()), _ptr(coords), n, q, _ptr(out), _ptr(workspace),
        workspace.numel(), _stream()))


NEIGHBOR_TABLE_MODES = {1: "hash32", 2: "hash64", 3: "hash_coords", 4: "dense_grid", 5: "rank_bitmap"}


def neighbor_map_table_mode(workspace: torch.Tensor) -> str:
    """The table the last build into ``workspace`` chose on the device (the
    int32 at byte 40 of the workspace header); syncs the current stream."""
    mode = int(workspace[40:44].view(torch.int32).item())
    return NEIGHBOR_TABLE_MODES.get(mode, "none")


def neighbor_map_rank_levels(workspace: torch.Tensor) -> int:
    """Octree levels of the rank bitmap's key in the last build into
    ``workspace`` (0: rows sorted in (b, x, y, z); L: rows in the order L C2S
    subdivisions below such a set emit them); syncs the current stream."""
    return int(workspace[52:56].view(torch.int32).item())


def neighbor_map_check(workspace: torch.Tensor) -> None:
    """Syncs the current stream and raises on device-detected coord errors."""
    check(_capi.load().sc_neighbor_map_check(_ptr(workspace), _stream()))


def neighbor_rows_tensor_from_coords_tensor(
        cfg: SparseSubmConvConfig, coords: torch.Tensor, query_rows: Optional[int] = None,
        workspace: Optional[NeighborMapWorkspace] = None, check_status: bool = True) -> torch.Tensor:
    """neighbor_rows_tensor_from_coords_tensor (crates/burn_flex_gmm/src/wgpu/neighbor.rs
    :977-1006): coords [N,4] int32 (batch,x,y,z) -> map [N,K] int32, -1 where
    absent, lowest row on duplicated coords.  With check_status (default) the
    call syncs once to read the device status, as the reference reads its
    overflow counter back (neighbor.rs:859-879)."""
    _require_cuda("coords", coords)
    if coords.dtype != torch.int32 or coords.dim() != 2 or coords.shape[1] != 4:
        raise SparseConvError(2, f"coords must be int32 [N,4], got {tuple(coords.shape)} {coords.dtype}")
    n = coords.shape[0]
    q = n if query_rows is None else int(query_rows)
    K = kernel_rows(cfg)
    out = torch.empty((q, K), dtype=torch.int32, device=coords.device)
    ws = (workspace or NeighborMapWorkspace(coords.device)).get(n)
    neighbor_map_build_into(cfg, coords, out, ws, q)
    if check_status:
        neighbor_map_check(ws)
    return out


def conv_plan_bytes(n_q: int, kernel_rows_: int) -> int:
    out = ctypes.c_size_t()
    check(_capi.load().sc_conv_plan_size(int(n_q), int(kernel_rows_), ctypes.byref(out)))
    return out.value


# Plan layout constants of bevy_synth_amd/csrc/sc_plan.hpp.
PLAN_TILE_ROWS = 256
PLAN_HALO_MAX = 960
PLAN_ABSENT = 0xFFFF


def conv_plan_layout(n_q: int, K: int) -> dict:
    """Byte offsets of the plan sections (mirror of plan_layout in sc_plan.hpp;
    tests check the total against sc_conv_plan_size)."""
    def al(x):
        return (x + 255) & ~255
    nt = (n_q + PLAN_TILE_ROWS - 1) // PLAN_TILE_ROWS
    cap = max(2 * n_q, 4096)
    cap = (cap + 1023) // 1024 * 1024
    gcap = max(16 * n_q, 1 << 20)
    gcap = (gcap + 2047) // 2048 * 2048
    L = {"n_tiles": nt}
    o = al(256)
    for name, size in (("order", nt * PLAN_TILE_ROWS * 4), ("tile_u", nt * 4), ("overflow", nt * 4),
                       ("halo", nt * PLAN_HALO_MAX * 4), ("lmap", nt * K * PLAN_TILE_ROWS * 2),
                       ("grid", gcap * 4), ("gsum", gcap // 2048 * 4),
                       ("counts", cap * 4), ("offsets", cap * 4), ("bsum", cap // 1024 * 4)):
        L[name] = o
        o = al(o + size)
    L["total"] = o
    return L


class ConvPlan:
    """Row order + per-tile halo tables of one neighbour map (sc_conv_plan_build).

    Built once per map and passed to every conv on that map, the role the
    reference's neighbour cache plays for its decoder
    (crates/burn_flex_gmm/src/wgpu.rs:349-382).  ``buf`` is the device buffer;
    n_in / n_q / K record the map it was built from."""

    def __init__(self, buf: torch.Tensor, n_in: int, n_q: int, K: int):
        self.buf, self.n_in, self.n_q, self.K = buf, n_in, n_q, K

    def to_host(self) -> dict:
        """Reads the plan back (syncs): header fields and the per-tile tables
        as numpy arrays, for inspection and tests."""
        L = conv_plan_layout(self.n_q, self.K)
        nt = L["n_tiles"]
        b = self.buf.cpu().numpy()

        def sec(name, count, dt):
            return b[L[name]:L[name] + count * np.dtype(dt).itemsize].view(dt)
        hdr = b[:256].view(np.int32)
        n_over = int(hdr[7])
        return {
            "n_tiles": int(hdr[4]), "K": int(hdr[5]), "brick_shift": int(hdr[6]), "n_overflow": n_over,
            "grid_mode": int(hdr[19]), "n_unique": int(hdr[20]), "n_extras": int(hdr[21]),
            "order": sec("order", nt * PLAN_TILE_ROWS, np.int32).reshape(nt, PLAN_TILE_ROWS),
            "tile_u": sec("tile_u", nt, np.int32),
            "overflow": np.sort(sec("overflow", nt, np.int32)[:n_over]),
            "halo": sec("halo", nt * PLAN_HALO_MAX, np.int32).reshape(nt, PLAN_HALO_MAX),
            "lmap": sec("lmap", nt * self.K * PLAN_TILE_ROWS, np.uint16).reshape(nt, self.K, PLAN_TILE_ROWS),
        }


def conv_plan_build_into(cfg: SparseSubmConvConfig, coords: torch.Tensor, neighbor_rows: torch.Tensor,
                         buf: torch.Tensor) -> ConvPlan:
    """Stream-ordered plan build into a preallocated 256-byte aligned uint8 buffer."""
    n_in, n_q, K = coords.shape[0], neighbor_rows.shape[0], kernel_rows(cfg)
    check(_capi.load().sc_conv_plan_build(
        ctypes.byref(cfg.to_c()), _ptr(coords), n_in, _ptr(neighbor_rows), n_q, _ptr(buf),
        buf.numel(), _stream()))
    return ConvPlan(buf, n_in, n_q, K)


def conv_plan_check(plan: "ConvPlan") -> None:
    """Syncs the current stream and raises if a planned conv found ``plan`` or
    its packed weights built for another shape (the conv then wrote nothing)."""
    check(_capi.load().sc_conv_plan_check(_ptr(plan.buf), _stream()))


def conv_plan_order_into(cfg: SparseSubmConvConfig, coords: torch.Tensor, n_q: int,
                         buf: torch.Tensor) -> None:
    """First half of the plan build (sc_conv_plan_order): the row order, from
    the coords alone, so it can run while the map is being built."""
    check(_capi.load().sc_conv_plan_order(
        ctypes.byref(cfg.to_c()), _ptr(coords), coords.shape[0], int(n_q), _ptr(buf), buf.numel(),
        _stream()))


def conv_plan_tables_into(cfg: SparseSubmConvConfig, neighbor_rows: torch.Tensor, n_in: int,
                          buf: torch.Tensor) -> ConvPlan:
    """Second half (sc_conv_plan_tables): the halo tables, from the map; after
    both the order and the map build."""
    n_q, K = neighbor_rows.shape[0], kernel_rows(cfg)
    check(_capi.load().sc_conv_plan_tables(
        ctypes.byref(cfg.to_c()), _ptr(neighbor_rows), int(n_in), n_q, _ptr(buf), buf.numel(),
        _stream()))
    return ConvPlan(buf, int(n_in), n_q, K)


_AUX_STREAMS = {}


def _aux_stream(device: torch.device) -> torch.cuda.Stream:
    """One side stream per device (default priority) for overlapped builds."""
    key = torch.device(device).index if torch.device(device).index is not None else torch.cuda.current_device()
    if key not in _AUX_STREAMS:
        _AUX_STREAMS[key] = torch.cuda.Stream(device=key)
    return _AUX_STREAMS[key]


def count_to_host_async(count: torch.Tensor) -> Tuple[torch.Tensor, "torch.cuda.Event"]:
    """Copies a device int64 count into pinned host memory on the side stream,
    ordered after the current stream's work so far but not after anything
    enqueued on it later: the caller enqueues more GPU work, then waits on
    the returned event and reads the host tensor, so the read-back overlaps
    that work instead of idling the GPU."""
    main = torch.cuda.current_stream(count.device)
    aux = _aux_stream(count.device)
    host = torch.empty(count.shape, dtype=count.dtype, pin_memory=True)
    aux.wait_stream(main)
    with torch.cuda.stream(aux):
        host.copy_(count, non_blocking=True)
        ready = torch.cuda.Event()
        ready.record(aux)
    count.record_stream(aux)
    return host, ready


def map_and_plan_into(cfg: SparseSubmConvConfig, coords: torch.Tensor, neighbor_rows: torch.Tensor,
                      workspace: torch.Tensor, plan_buf: torch.Tensor) -> ConvPlan:
    """The neighbour map and its conv plan, with the plan's row order (which
    reads only the coords) built on a side stream while the map is built on
    the current one; the halo tables follow on the current stream once both
    are done.  Same result as neighbor_map_build_into + conv_plan_build_into."""
    main = torch.cuda.current_stream(coords.device)
    aux = _aux_stream(coords.device)
    n_q = neighbor_rows.shape[0]
    aux.wait_stream(main)
    with torch.cuda.stream(aux):
        conv_plan_order_into(cfg, coords, n_q, plan_buf)
    neighbor_map_build_into(cfg, coords, neighbor_rows, workspace, query_rows=n_q)
    main.wait_stream(aux)
    return conv_plan_tables_into(cfg, neighbor_rows, coords.shape[0], plan_buf)


def build_conv_plan(cfg: SparseSubmConvConfig, coords: torch.Tensor,
                    neighbor_rows: torch.Tensor) -> ConvPlan:
    """Allocates and builds the conv plan of ``neighbor_rows`` (built from ``coords``)."""
    _require_cuda("coords", coords)
    _require_cuda("neighbor_rows", neighbor_rows)
    K = kernel_rows(cfg)
    if neighbor_rows.dtype != torch.int32 or neighbor_rows.dim() != 2 or neighbor_rows.shape[1] != K:
        raise SparseConvError(2, f"conv plan: neighbor rows must be int32 [N_q, {K}]")
    buf = torch.empty(conv_plan_bytes(neighbor_rows.shape[0], K), dtype=torch.uint8,
                      device=coords.device)
    return conv_plan_build_into(cfg, coords, neighbor_rows, buf)


class ChildPlan:
    """A child plan (sc_conv_child_plan_build): per C2S child index, the
    parents whose child is active, in the parent plan's order, in tiles of
    their own, so conv1 of the upsample block computes only active children.
    Built from the parents' ConvPlan, their map and the subdivision's
    child_rows; ``n_children`` is the child count those rows index."""

    def __init__(self, buf: torch.Tensor, n_parents: int, n_children: int, K: int):
        self.buf, self.n_in, self.n_q, self.n_children, self.K = buf, n_parents, n_parents, n_children, K

    def to_host(self) -> dict:
        """Reads the child plan back (syncs): order [tiles, 256], tile_child,
        tile_u, the overflow list, status, the tiles the lists use, the
        splits, and the per-child entry counts and first tiles."""
        n = ctypes.c_size_t()
        check(_capi.load().sc_conv_child_plan_size(self.n_q, self.n_children, self.K, ctypes.byref(n)))
        n_main = (self.n_children + PLAN_TILE_ROWS - 1) // PLAN_TILE_ROWS + 8
        n_extra = n_main // 8 + 16
        nt = n_main + n_extra
        npt = (self.n_q + PLAN_TILE_ROWS - 1) // PLAN_TILE_ROWS
        nch = (npt + 255) // 256
        al = lambda x: (x + 255) & ~255
        o = {"order": 256}
        o["tile_u"] = al(o["order"] + nt * PLAN_TILE_ROWS * 4)
        o["overflow"] = al(o["tile_u"] + nt * 4)
        o["halo"] = al(o["overflow"] + nt * 4)
        o["lmap"] = al(o["halo"] + nt * PLAN_HALO_MAX * 4)
        o["tile_child"] = al(o["lmap"] + nt * self.K * PLAN_TILE_ROWS * 2)
        o["counts"] = al(o["tile_child"] + nt * 4)
        o["chunks"] = al(o["counts"] + npt * 8 * 4)
        o["child_n"] = al(o["chunks"] + nch * 8 * 4)
        o["child_base"] = al(o["child_n"] + 32)
        o["split"] = al(o["child_base"] + 32)
        o["split_n"] = al(o["split"] + n_extra * 8)
        assert al(o["split_n"] + 4) == n.value
        b = self.buf.cpu().numpy()
        sec = lambda name, cnt: b[o[name]:o[name] + 4 * cnt].view(np.int32)
        hdr = b[:256].view(np.int32)
        n_over, n_split = int(hdr[7]), int(hdr[21])
        return {"n_tiles": int(hdr[4]), "n_main": n_main, "status": int(b[:256].view(np.uint32)[18]),
                "n_overflow": n_over, "grid_mode": int(hdr[19]), "n_used": int(hdr[20]), "n_split": n_split,
                "list_tiles": int(hdr[22]),
                "order": sec("order", nt * PLAN_TILE_ROWS).reshape(nt, PLAN_TILE_ROWS),
                "tile_child": sec("tile_child", nt), "tile_u": sec("tile_u", nt),
                "overflow": sec("overflow", nt)[:n_over].copy(),
                "split": sec("split", 2 * n_extra).reshape(n_extra, 2)[:n_split].copy(),
                "child_n": sec("child_n", 8), "child_base": sec("child_base", 8)}


def build_child_plan(cfg: SparseSubmConvConfig, parent_plan: ConvPlan, neighbor_rows: torch.Tensor,
                     child_rows: torch.Tensor, n_children: int) -> ChildPlan:
    """sc_conv_child_plan_build: the child plan of conv1 (``cfg``'s kernel)
    over the parents of ``parent_plan`` / ``neighbor_rows`` [P, K] and the
    subdivision's ``child_rows`` [P, 8] (n_children active)."""
    _require_cuda("neighbor_rows", neighbor_rows)
    _require_cuda("child_rows", child_rows)
    K = kernel_rows(cfg)
    P = neighbor_rows.shape[0]
    if parent_plan.n_q != P or parent_plan.K != K:
        raise SparseConvError(2, f"child plan: parent plan built for n_q={parent_plan.n_q} K={parent_plan.K}, "
                                 f"map has {P} rows and K={K}")
    if child_rows.dtype != torch.int32 or tuple(child_rows.shape) != (P, 8) or not child_rows.is_contiguous():
        raise SparseConvError(2, "child plan: child_rows must be int32 [P, 8]")
    n = ctypes.c_size_t()
    check(_capi.load().sc_conv_child_plan_size(P, int(n_children), K, ctypes.byref(n)))
    buf = torch.empty(n.value, dtype=torch.uint8, device=neighbor_rows.device)
    check(_capi.load().sc_conv_child_plan_build(
        ctypes.byref(cfg.to_c()), _ptr(parent_plan.buf), _ptr(neighbor_rows), P, _ptr(child_rows),
        int(n_children), _ptr(buf), buf.numel(), _stream()))
    return ChildPlan(buf, P, int(n_children), K)


def build_linear_child_plan(child_rows: torch.Tensor, n_children: int) -> ChildPlan:
    """sc_linear_child_plan_build: for the transposed upsample's linear
    (linear_forward with ``child_rows``), per child index the parents whose
    child is active, in row order, in tiles of their own, so that
    linear_forward(..., child_plan=) computes only active children."""
    _require_cuda("child_rows", child_rows)
    if child_rows.dtype != torch.int32 or child_rows.dim() != 2 or child_rows.shape[1] != 8 \
            or not child_rows.is_contiguous():
        raise SparseConvError(2, "child plan: child_rows must be int32 [P, 8]")
    P = child_rows.shape[0]
    n = ctypes.c_size_t()
    check(_capi.load().sc_conv_child_plan_size(P, int(n_children), 1, ctypes.byref(n)))
    buf = torch.empty(n.value, dtype=torch.uint8, device=child_rows.device)
    check(_capi.load().sc_linear_child_plan_build(P, _ptr(child_rows), int(n_children), _ptr(buf), buf.numel(),
                                                  _stream()))
    return ChildPlan(buf, P, int(n_children), 1)


def conv_weight_pack_bytes(cfg: SparseSubmConvConfig, w_dtype: torch.dtype) -> int:
    out = ctypes.c_size_t()
    dt = {torch.bfloat16: _capi.SC_DTYPE_BF16, torch.int8: _capi.SC_DTYPE_I8,
          torch.float16: _capi.SC_DTYPE_F16}.get(w_dtype)
    if dt is None:
        raise SparseConvError(3, "weight packing takes bf16, f16 or int8 weights")
    check(_capi.load().sc_conv_weight_pack_size(ctypes.byref(cfg.to_c()), dt, ctypes.byref(out)))
    return out.value


def pack_conv_weight(cfg: SparseSubmConvConfig, weight: torch.Tensor) -> torch.Tensor:
    """The planned conv's weight layout (sc_conv_weight_pack): bf16 MFMA
    fragments, int8 weights widened exactly (their scales are passed to the
    conv as usual); a one-time per-layer reorder, the role pack_flex_weight
    plays for the reference's CPU path (crates/burn_flex_gmm/src/lib.rs
    :377-426)."""
    _require_cuda("weight", weight)
    buf = torch.empty(conv_weight_pack_bytes(cfg, weight.dtype), dtype=torch.uint8, device=weight.device)
    check(_capi.load().sc_conv_weight_pack(ctypes.byref(cfg.to_c()), _dt(weight), _ptr(weight), _ptr(buf),
                                           _stream()))
    return buf


def sparse_subm_conv_forward(cfg: SparseSubmConvConfig, input: torch.Tensor,
                             neighbor_rows: torch.Tensor, weight: torch.Tensor,
                             bias: Optional[torch.Tensor] = None,
                             w_scale: Optional[torch.Tensor] = None,
                             residual: Optional[torch.Tensor] = None,
                             out_dtype: Optional[torch.dtype] = None,
                             out: Optional[torch.Tensor] = None,
                             layer_norm: bool = False, ln_weight: Optional[torch.Tensor] = None,
                             ln_bias: Optional[torch.Tensor] = None, ln_eps: float = 1e-6,
                             silu: bool = False, plan: Optional[ConvPlan] = None,
                             packed_weight: Optional[torch.Tensor] = None,
                             workspace: Optional[torch.Tensor] = None,
                             child_rows: Optional[torch.Tensor] = None, n_child_rows: Optional[int] = None,
                             skip_parent: Optional[torch.Tensor] = None,
                             skip_index: Optional[torch.Tensor] = None,
                             child_count: Optional[torch.Tensor] = None) -> torch.Tensor:
    """sparse_subm_conv_forward_wgpu (crates/burn_flex_gmm/src/wgpu/sparse_conv.rs:310-367).

    input [N_in, Cin] f32|bf16; neighbor_rows [N_q, K] int32 (N_q <= N_in);
    weight [Cout, KD, KH, KW, Cin_g] (or any view with that element count)
    f32 (f32 input), bf16 or int8 (+ w_scale [Cout] f32) (bf16 input);
    bias [Cout] f32 or None; residual [N_q, Cout] in the output dtype or None.
    Optional fused epilogue: + bias -> LayerNorm over Cout (ln_weight / ln_bias
    [Cout] f32 or None, ln_eps) -> SiLU -> + residual.
    With ``plan`` (a ConvPlan of this map) and ``packed_weight``
    (pack_conv_weight of ``weight``) bf16 convs take the halo-staged kernel
    (same result up to the fixed f32 summation order).
    A LayerNorm that cannot run inside the conv tile (groups > 1 or Cout >
    128) is applied to the f32 conv output by a row kernel; with a bf16
    output that needs an f32 staging buffer (``workspace``, uint8, grown here
    when missing or too small).
    C2S forms (sparse_decoder_runtime_impl.rs:2240-2255, 1054-1133):
    ``child_rows`` [N_q, 8] int32 (subdivision_build_indexed) makes this conv1
    of the upsample block -- query row r's channels [c*C, (c+1)*C), C =
    Cout/8, are child c's features and land in row child_rows[r, c] of an
    [n_child_rows, C] output (LayerNorm then per child); ``child_count`` (the
    subdivision's device int64 count) lets n_child_rows be an upper bound
    such as 8 N_q, so the call needs no host read of the count: a LayerNorm
    staged outside the tile stops at that row.  ``skip_parent`` [P, Cp] with
    ``skip_index`` [N_q] (the children's linear_idx) adds the
    channel-repeated parent skip (conv2).
    Returns [N_q, Cout] in out_dtype (default: the input dtype)."""
    _require_cuda("input", input)
    _require_cuda("neighbor_rows", neighbor_rows)
    _require_cuda("weight", weight)
    if input.dim() != 2 or input.shape[1] != cfg.in_channels:
        raise SparseConvError(2, f"sparse conv input channel mismatch: got {tuple(input.shape)} "
                                 f"expected [*, {cfg.in_channels}]")
    K = kernel_rows(cfg)
    if neighbor_rows.dtype != torch.int32 or neighbor_rows.dim() != 2 or neighbor_rows.shape[1] != K:
        raise SparseConvError(2, f"sparse conv neighbor kernel rows mismatch: got "
                                 f"{tuple(neighbor_rows.shape)} expected [*, {K}]")
    c = cfg.to_c()
    w_elems = cfg.out_channels * K * c.in_channels_per_group
    if weight.numel() != w_elems:
        raise SparseConvError(2, f"sparse conv weight len mismatch: got {weight.numel()} expected {w_elems}")
    if bias is not None:
        _require_cuda("bias", bias)
        if bias.dtype != torch.float32 or bias.numel() != cfg.out_channels:
            raise SparseConvError(2, f"sparse conv bias len mismatch: got {bias.numel()} "
                                     f"expected {cfg.out_channels}")
    if w_scale is not None:
        _require_cuda("w_scale", w_scale)
        if w_scale.dtype != torch.float32 or w_scale.numel() != cfg.out_channels:
            raise SparseConvError(2, "w_scale must be f32 [Cout]")
    n_q = neighbor_rows.shape[0]
    od = input.dtype if out_dtype is None else out_dtype
    out_shape = (n_q, cfg.out_channels)
    if child_rows is not None:
        _require_cuda("child_rows", child_rows)
        if child_rows.dtype != torch.int32 or child_rows.shape != (n_q, 8):
            raise SparseConvError(2, "child_rows must be int32 [N_q, 8]")
        if n_child_rows is None or cfg.out_channels % 8:
            raise SparseConvError(2, "child scatter needs n_child_rows and Cout = 8 * C")
        out_shape = (int(n_child_rows), cfg.out_channels // 8)
    if skip_index is not None:
        _require_cuda("skip_index", skip_index)
        _require_cuda("skip_parent", skip_parent)
        if skip_index.dtype != torch.int32 or skip_index.shape != (n_q,) or skip_parent.dtype != od:
            raise SparseConvError(2, "skip_index must be int32 [N_q] and skip_parent in the output dtype")
    if out is None:
        out = torch.empty(out_shape, dtype=od, device=input.device)
    else:
        _require_cuda("out", out)
        if tuple(out.shape) != out_shape or out.dtype != od:
            raise SparseConvError(2, "out has the wrong shape or dtype")
    if residual is not None:
        _require_cuda("residual", residual)
        if residual.shape != (n_q, cfg.out_channels) or residual.dtype != od:
            raise SparseConvError(2, "residual must be [N_q, Cout] in the output dtype")
    for name, t in (("ln_weight", ln_weight), ("ln_bias", ln_bias)):
        if t is not None:
            _require_cuda(name, t)
            if t.dtype != torch.float32 or t.numel() != cfg.out_channels:
                raise SparseConvError(2, f"{name} must be f32 [Cout]")
    if plan is not None and (plan.n_q != n_q or plan.n_in != input.shape[0] or plan.K != K):
        raise SparseConvError(2, f"conv plan was built for n_in={plan.n_in} n_q={plan.n_q} K={plan.K}, "
                                 f"got n_in={input.shape[0]} n_q={n_q} K={K}")
    if layer_norm or silu or plan is not None or child_rows is not None or skip_index is not None:
        epi = _capi.ScConvEpilogue()
        if child_rows is not None:
            epi.child_rows = child_rows.data_ptr()
            epi.n_child_rows = int(n_child_rows)
            if child_count is not None:
                _require_cuda("child_count", child_count)
                if child_count.dtype != torch.int64 or child_count.numel() != 1:
                    raise SparseConvError(2, "child_count must be a device int64 [1]")
                epi.child_count = child_count.data_ptr()
        if skip_index is not None:
            epi.skip_parent = skip_parent.data_ptr()
            epi.skip_index = skip_index.data_ptr()
            epi.skip_parent_rows = skip_parent.shape[0]
            epi.skip_parent_channels = skip_parent.shape[1]
        epi.residual = None if residual is None else residual.data_ptr()
        epi.layer_norm = int(layer_norm)
        epi.ln_weight = None if ln_weight is None else ln_weight.data_ptr()
        epi.ln_bias = None if ln_bias is None else ln_bias.data_ptr()
        epi.ln_eps = float(ln_eps)
        epi.silu = int(silu)
        need = ctypes.c_size_t()
        check(_capi.load().sc_conv_epilogue_workspace_size(ctypes.byref(c), _dt(input), n_q, _dt(out),
                                                           ctypes.byref(epi), ctypes.byref(need)))
        if need.value:
            if workspace is None or workspace.numel() < need.value:
                workspace = torch.empty(need.value, dtype=torch.uint8, device=input.device)
            epi.workspace = workspace.data_ptr()
            epi.workspace_bytes = workspace.numel()
        if isinstance(plan, ChildPlan):
            if child_rows is None or int(n_child_rows) != plan.n_children:
                raise SparseConvError(2, "a child plan needs the child scatter it was built for "
                                         f"({plan.n_children} children)")
            check(_capi.load().sc_subm_conv_forward_child_planned(
                ctypes.byref(c), _dt(input), _ptr(input), input.shape[0], _ptr(neighbor_rows), n_q,
                _dt(weight), _ptr(weight), _ptr(packed_weight), _ptr(w_scale), _ptr(bias), ctypes.byref(epi),
                _dt(out), _ptr(out), _ptr(plan.buf), _stream()))
            return out
        if plan is not None:
            check(_capi.load().sc_subm_conv_forward_planned(
                ctypes.byref(c), _dt(input), _ptr(input), input.shape[0], _ptr(neighbor_rows), n_q,
                _dt(weight), _ptr(weight), _ptr(packed_weight), _ptr(w_scale), _ptr(bias), ctypes.byref(epi),
                _dt(out), _ptr(out), _ptr(plan.buf), _stream()))
            return out
        check(_capi.load().sc_subm_conv_forward_fused(
            ctypes.byref(c), _dt(input), _ptr(input), input.shape[0], _ptr(neighbor_rows), n_q,
            _dt(weight), _ptr(weight), _ptr(w_scale), _ptr(bias), ctypes.byref(epi), _dt(out),
            _ptr(out), _stream()))
        return out
    check(_capi.load().sc_subm_conv_forward(
        ctypes.byref(c), _dt(input), _ptr(input), input.shape[0], _ptr(neighbor_rows), n_q,
        _dt(weight), _ptr(weight), _ptr(w_scale), _ptr(bias), _ptr(residual), _dt(out),
        _ptr(out), _stream()))
    return out


def linear_forward(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                   w_scale: Optional[torch.Tensor] = None, residual: Optional[torch.Tensor] = None,
                   out_dtype: Optional[torch.dtype] = None, silu: bool = False, layer_norm: bool = False,
                   ln_weight: Optional[torch.Tensor] = None, ln_bias: Optional[torch.Tensor] = None,
                   ln_eps: float = 1e-6, out: Optional[torch.Tensor] = None,
                   workspace: Optional[torch.Tensor] = None, child_rows: Optional[torch.Tensor] = None,
                   n_child_rows: Optional[int] = None, child_plan: Optional["ChildPlan"] = None) -> torch.Tensor:
    """linear_forward_wgpu (burn_trellis sparse_decoder_wgpu_ops.rs:79-160) through
    sc_linear_forward: x [rows, Cin] @ weight[Cout, Cin]^T + bias, with the conv
    epilogue (LayerNorm over the row, SiLU, + residual) fused.  Same dtype rules
    as sparse_subm_conv_forward.
    ``child_rows`` [rows, 8] int32 (subdivision_build_indexed) makes this the
    2x2x2 transposed upsample: row r's channels [c*C, (c+1)*C), C = Cout/8,
    land in row child_rows[r, c] of an [n_child_rows, C] output (LayerNorm
    per child, ln_weight / ln_bias then [C]).  ``child_plan``
    (build_linear_child_plan over the same child_rows) computes only the
    active children (sc_linear_forward_child_planned); the stored values are
    the same."""
    _require_cuda("x", x)
    _require_cuda("weight", weight)
    rows, cin = x.shape
    if weight.dim() != 2 or weight.shape[1] != cin:
        raise SparseConvError(2, f"linear: invalid input channels {cin}, weight {tuple(weight.shape)}")
    cout = weight.shape[0]
    out_shape = (rows, cout)
    if child_rows is not None:
        _require_cuda("child_rows", child_rows)
        if child_rows.dtype != torch.int32 or child_rows.shape != (rows, 8):
            raise SparseConvError(2, "child_rows must be int32 [rows, 8]")
        if n_child_rows is None or cout % 8:
            raise SparseConvError(2, "child scatter needs n_child_rows and Cout = 8 * C")
        if residual is not None:
            raise SparseConvError(2, "linear: the child scatter takes no residual")
        out_shape = (int(n_child_rows), cout // 8)
    for name, t, n in (("bias", bias, cout), ("w_scale", w_scale, cout), ("ln_weight", ln_weight, out_shape[1]),
                       ("ln_bias", ln_bias, out_shape[1])):
        if t is not None:
            _require_cuda(name, t)
            if t.dtype != torch.float32 or t.numel() != n:
                raise SparseConvError(2, f"linear: {name} must be f32 [{n}]")
    od = x.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty(out_shape, dtype=od, device=x.device)
    else:
        _require_cuda("out", out)
        if tuple(out.shape) != out_shape or out.dtype != od:
            raise SparseConvError(2, "linear: out has the wrong shape or dtype")
    if residual is not None:
        _require_cuda("residual", residual)
        if residual.shape != (rows, cout) or residual.dtype != od:
            raise SparseConvError(2, "linear: residual must be [rows, Cout] in the output dtype")
    epi = _capi.ScConvEpilogue()
    if child_rows is not None:
        epi.child_rows = child_rows.data_ptr()
        epi.n_child_rows = int(n_child_rows)
    epi.residual = None if residual is None else residual.data_ptr()
    epi.layer_norm = int(layer_norm)
    epi.ln_weight = None if ln_weight is None else ln_weight.data_ptr()
    epi.ln_bias = None if ln_bias is None else ln_bias.data_ptr()
    epi.ln_eps = float(ln_eps)
    epi.silu = int(silu)
    need = ctypes.c_size_t()
    c = SparseSubmConvConfig(cin, cout, 1, 1, 1).to_c()
    check(_capi.load().sc_conv_epilogue_workspace_size(ctypes.byref(c), _dt(x), rows, _dt(out), ctypes.byref(epi),
                                                       ctypes.byref(need)))
    if need.value:
        if workspace is None or workspace.numel() < need.value:
            workspace = torch.empty(need.value, dtype=torch.uint8, device=x.device)
        epi.workspace = workspace.data_ptr()
        epi.workspace_bytes = workspace.numel()
    if child_plan is not None:
        if child_rows is None:
            raise SparseConvError(2, "linear: a child plan needs child_rows")
        if child_plan.n_q != rows or child_plan.n_children != int(n_child_rows) or child_plan.K != 1:
            raise SparseConvError(2, "linear: the child plan was built for other parents or children")
        check(_capi.load().sc_linear_forward_child_planned(
            _dt(x), _ptr(x), rows, cin, cout, _dt(weight), _ptr(weight), _ptr(w_scale), _ptr(bias),
            ctypes.byref(epi), _dt(out), _ptr(out), _ptr(child_plan.buf), _stream()))
        return out
    check(_capi.load().sc_linear_forward(_dt(x), _ptr(x), rows, cin, cout, _dt(weight), _ptr(weight), _ptr(w_scale),
                                         _ptr(bias), ctypes.byref(epi), _dt(out), _ptr(out), _stream()))
    return out


def layer_norm(x: torch.Tensor, weight: Optional[torch.Tensor] = None,
               bias: Optional[torch.Tensor] = None, eps: float = 1e-6, silu: bool = False,
               out_dtype: Optional[torch.dtype] = None,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """layer_norm_affine[_silu]_forward_wgpu (crates/burn_flex_gmm/src/wgpu/ops.rs:162-446);
    host form layer_norm_inplace + silu_inplace (sparse_decoder_wgpu_ops.rs:1642-1720)."""
    _require_cuda("x", x)
    rows, ch = x.shape
    od = x.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty((rows, ch), dtype=od, device=x.device)
    for name, t in (("weight", weight), ("bias", bias)):
        if t is not None and (t.dtype != torch.float32 or t.numel() != ch):
            raise SparseConvError(2, f"layer_norm_inplace: invalid {name} len {t.numel()}, expected {ch}")
    check(_capi.load().sc_layer_norm(_dt(x), _ptr(x), rows, ch, _ptr(weight), _ptr(bias),
                                     ctypes.c_float(eps), int(silu), _dt(out), _ptr(out),
                                     _stream()))
    return out


def add(a: torch.Tensor, b: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """add_inplace (sparse_decoder_wgpu_ops.rs:1747-1757) as out = a + b."""
    if a.shape != b.shape or a.dtype != b.dtype:
        raise SparseConvError(2, "add: operands differ in shape or dtype")
    if out is None:
        out = torch.empty_like(a)
    check(_capi.load().sc_add(_dt(a), _ptr(a), _ptr(b), a.numel(), _ptr(out), _stream()))
    return out


def convert(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """f32 <-> bf16 with the reference's round-to-nearest-even (wgpu.rs:57-67)."""
    out = torch.empty(x.shape, dtype=dtype, device=x.device)
    check(_capi.load().sc_convert(_dt(x), _ptr(x), _dt(out), _ptr(out), x.numel(), _stream()))
    return out


# ------------------------------------------------------------------ C2S

def subdivision_build(parent_coords: torch.Tensor, logits: Optional[torch.Tensor] = None,
                      mask: Optional[torch.Tensor] = None,
                      thresholds: Optional[Sequence[float]] = None,
                      with_pairs: bool = True
                      ) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """subdivision_active_indices_wgpu + expand_subdivision_coords_and_linear_indices_wgpu
    (sparse_decoder_wgpu_ops.rs:885-1054).  Returns (child_coords [A,4] int32,
    linear_idx [A] int32, pairs [A,2] int32 or None).  Syncs once to read A, as
    the reference's argwhere does."""
    _require_cuda("parent_coords", parent_coords)
    P = parent_coords.shape[0]
    dev = parent_coords.device
    if (logits is None) == (mask is None):
        raise SparseConvError(8, "subdivision needs exactly one of logits or mask")
    if logits is not None:
        if logits.shape != (P, 8) or logits.dtype != torch.float32:
            raise SparseConvError(2, "decoder subdivision logits tensor must be f32 [P, 8]")
        th = (ctypes.c_float * 8)(*([0.0] * 8 if thresholds is None else list(thresholds)))
    else:
        if mask.shape != (P, 8) or mask.dtype not in (torch.uint8, torch.bool):
            raise SparseConvError(2, "subdivision mask must be u8/bool [P, 8]")
        mask = mask.to(torch.uint8).contiguous()
        th = None
    cap = max(8 * P, 1)
    child = torch.empty((cap, 4), dtype=torch.int32, device=dev)
    lin = torch.empty((cap,), dtype=torch.int32, device=dev)
    pairs = torch.empty((cap, 2), dtype=torch.int32, device=dev) if with_pairs else None
    count = torch.empty((1,), dtype=torch.int64, device=dev)
    wsb = ctypes.c_size_t()
    check(_capi.load().sc_subdivision_workspace_size(P, ctypes.byref(wsb)))
    ws = torch.empty(max(wsb.value, 16), dtype=torch.uint8, device=dev)
    check(_capi.load().sc_subdivision_build(
        _ptr(logits), _ptr(mask), th, _ptr(parent_coords), P, _ptr(child), _ptr(lin),
        _ptr(pairs), _ptr(count), _ptr(ws), ws.numel(), _stream()))
    a = int(count.item())
    return child[:a], lin[:a], (pairs[:a] if pairs is not None else None)


class SubdivisionBuffers:
    """Device buffers of one sc_subdivision_build_indexed call over P parents
    (child capacity 8P), reusable across calls of the same P."""

    def __init__(self, P: int, dev):
        cap = max(8 * P, 1)
        self.P = P
        self.child = torch.empty((cap, 4), dtype=torch.int32, device=dev)
        self.lin = torch.empty((cap,), dtype=torch.int32, device=dev)
        self.rows = torch.empty((max(P, 1), 8), dtype=torch.int32, device=dev)
        self.count = torch.empty((1,), dtype=torch.int64, device=dev)
        wsb = ctypes.c_size_t()
        check(_capi.load().sc_subdivision_workspace_size(P, ctypes.byref(wsb)))
        self.ws = torch.empty(max(wsb.value, 16), dtype=torch.uint8, device=dev)


def subdivision_launch(parent_coords: torch.Tensor, logits: Optional[torch.Tensor] = None,
                       mask: Optional[torch.Tensor] = None, thresholds: Optional[Sequence[float]] = None,
                       buffers: Optional[SubdivisionBuffers] = None) -> SubdivisionBuffers:
    """sc_subdivision_build_indexed into `buffers` (new ones when None), on the
    current stream, without waiting: the child count stays on the device
    (buffers.count)."""
    _require_cuda("parent_coords", parent_coords)
    P = parent_coords.shape[0]
    dev = parent_coords.device
    if (logits is None) == (mask is None):
        raise SparseConvError(8, "subdivision needs exactly one of logits or mask")
    if logits is not None:
        if logits.shape != (P, 8) or logits.dtype != torch.float32:
            raise SparseConvError(2, "decoder subdivision logits tensor must be f32 [P, 8]")
        th = (ctypes.c_float * 8)(*([0.0] * 8 if thresholds is None else list(thresholds)))
    else:
        if mask.shape != (P, 8) or mask.dtype not in (torch.uint8, torch.bool):
            raise SparseConvError(2, "subdivision mask must be u8/bool [P, 8]")
        mask = mask.to(torch.uint8).contiguous()
        th = None
    b = buffers if buffers is not None else SubdivisionBuffers(P, dev)
    if b.P != P:
        raise SparseConvError(2, f"subdivision buffers hold {b.P} parents, the call has {P}")
    check(_capi.load().sc_subdivision_build_indexed(
        _ptr(logits), _ptr(mask), th, _ptr(parent_coords), P, _ptr(b.child), _ptr(b.lin), None, _ptr(b.rows),
        _ptr(b.count), _ptr(b.ws), b.ws.numel(), _stream()))
    return b


def subdivision_build_indexed(parent_coords: torch.Tensor, logits: Optional[torch.Tensor] = None,
                              mask: Optional[torch.Tensor] = None,
                              thresholds: Optional[Sequence[float]] = None
                              ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """subdivision_build plus the inverse of linear_idx (sc_subdivision_build_indexed):
    returns (child_coords [A,4], linear_idx [A], child_rows [P,8] int32 with
    child_rows[p, c] = the row of child (p, c) or -1).  Syncs once to read A."""
    b = subdivision_launch(parent_coords, logits, mask, thresholds)
    a = int(b.count.item())
    return b.child[:a], b.lin[:a], b.rows[:b.P]


def linear_skinny(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """linear_skinny_forward_wgpu (crates/burn_flex_gmm/src/wgpu/ops.rs:1390-1410):
    x [rows, Cin] f32|bf16, weight [Cout <= 8, Cin] f32, bias [Cout] f32 ->
    [rows, Cout] f32 (the C2S to_subdiv logits)."""
    _require_cuda("x", x)
    _require_cuda("weight", weight)
    rows, cin = x.shape
    cout = weight.shape[0]
    if weight.dtype != torch.float32 or weight.shape != (cout, cin):
        raise SparseConvError(2, f"skinny linear input/weight mismatch: input_in_channels={cin} "
                                 f"weight {tuple(weight.shape)}")
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != cout):
        raise SparseConvError(2, f"skinny linear bias mismatch: out_channels={cout} bias_len={bias.numel()}")
    out = torch.empty((rows, cout), dtype=torch.float32, device=x.device)
    check(_capi.load().sc_linear_skinny(_dt(x), _ptr(x), rows, cin, _ptr(weight), _ptr(bias), cout, _ptr(out),
                                        _stream()))
    return out


def subdivision_logits_finish(logits: torch.Tensor, round_f16: bool = False, center: bool = False
                              ) -> torch.Tensor:
    """The decoder's to_subdiv logits post-processing, in place on [P, 8] f32:
    f16 rounding under compute_fp16 (sparse_decoder_runtime_impl.rs:871-873),
    then row centering (center_subdivision_logits, sparse_decoder_wgpu_ops.rs
    :1728-1745).  Returns ``logits``."""
    _require_cuda("logits", logits)
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.shape[1] != 8 or not logits.is_contiguous():
        raise SparseConvError(2, "decoder subdivision logits tensor must be f32 [P, 8]")
    check(_capi.load().sc_subdivision_logits_finish(_ptr(logits), logits.shape[0], int(round_f16), int(center),
                                                    _stream()))
    return logits


def gather_rows(src: torch.Tensor, split: int, idx: torch.Tensor) -> torch.Tensor:
    """select(0, idx) on the [rows*split, cols/split] view of src (conv1 child
    selection, sparse_decoder_runtime_impl.rs:2249-2255)."""
    _require_cuda("src", src)
    rows, cols = src.shape
    if cols % split != 0:
        raise SparseConvError(2, "gather_rows: columns not divisible by split")
    width = cols // split
    out = torch.empty((idx.shape[0], width), dtype=src.dtype, device=src.device)
    check(_capi.load().sc_gather_rows(_dt(src), _ptr(src), rows, split, width, _ptr(idx),
                                      idx.shape[0], _ptr(out), _stream()))
    return out


def c2s_skip_add(h: torch.Tensor, parent: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """In place: h += channel-repeated skip of the parent features
    (sparse_decoder_runtime_impl.rs:1054-1076,1123-1133)."""
    n, oc = h.shape
    pr, pc = parent.shape
    check(_capi.load().sc_c2s_skip_add(_dt(h), _ptr(h), n, oc, _dt(parent), _ptr(parent), pr, pc,
                                       _ptr(idx), _stream()))
    return h

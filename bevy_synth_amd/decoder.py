"""Sparse decoder blocks built on the device operators.

* ``ResidualBlock``   : conv3x3x3 -> LayerNorm (no affine) -> SiLU -> conv3x3x3 -> + x
                        (the benchmark residual block; the LN/SiLU ops are the
                        reference's layer_norm_silu_wgpu, sparse_decoder_wgpu_ops.rs
                        :1139-1161, eps 1e-6 from sparse_decoder.rs:43).
* ``C2SUpsampleBlock``: the TRELLIS2 channel-to-spatial upsample block
                        (sparse_decoder_runtime_impl.rs:758-1171, host form
                        :1236-1343): SiLU(LN(parent; norm1)) -> conv1 (Cin ->
                        8*Cout) on parent coords -> select children by
                        linear_idx -> SiLU(LN(children)) -> conv2 on child
                        coords -> + channel-repeated parent skip.
* ``transposed_upsample``: a stride-2 2x2x2 transposed sparse conv, which the
                        reference expresses as C2S with a 1x1x1 conv1 + select.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import torch

from .flex_gmm import (NeighborMapWorkspace, SparseSubmConvConfig, c2s_skip_add, gather_rows,
                       layer_norm, neighbor_rows_tensor_from_coords_tensor,
                       sparse_subm_conv_forward, subdivision_build)

LAYER_NORM32_EPS = 1e-6  # sparse_decoder.rs:43


@dataclass
class ConvLayer:
    """One submanifold conv: weight [Cout, K, Cin_g] (bf16/f32/int8), bias f32,
    optional per-output-channel scale for int8 weights."""

    cfg: SparseSubmConvConfig
    weight: torch.Tensor
    bias: Optional[torch.Tensor] = None
    w_scale: Optional[torch.Tensor] = None

    def __call__(self, x: torch.Tensor, nbr: torch.Tensor, out_dtype=None,
                 residual: Optional[torch.Tensor] = None, layer_norm: bool = False,
                 silu: bool = False, ln_eps: float = LAYER_NORM32_EPS) -> torch.Tensor:
        return sparse_subm_conv_forward(self.cfg, x, nbr, self.weight, self.bias, self.w_scale,
                                        residual=residual, out_dtype=out_dtype,
                                        layer_norm=layer_norm, ln_eps=ln_eps, silu=silu)


@dataclass
class ResidualBlock:
    conv1: ConvLayer
    conv2: ConvLayer
    eps: float = LAYER_NORM32_EPS

    def __call__(self, x: torch.Tensor, nbr: torch.Tensor) -> torch.Tensor:
        # conv1 carries LayerNorm + SiLU in its epilogue; conv2 adds the residual.
        h = self.conv1(x, nbr, out_dtype=x.dtype, layer_norm=True, silu=True, ln_eps=self.eps)
        return self.conv2(h, nbr, out_dtype=x.dtype, residual=x)


@dataclass
class C2SUpsampleBlock:
    in_channels: int
    out_channels: int
    norm1_weight: torch.Tensor
    norm1_bias: torch.Tensor
    conv1: ConvLayer   # Cin -> 8*Cout on parent coords
    conv2: ConvLayer   # Cout -> Cout on child coords
    eps: float = LAYER_NORM32_EPS

    def __call__(self, parent_coords: torch.Tensor, parent_feats: torch.Tensor,
                 logits: Optional[torch.Tensor] = None, mask: Optional[torch.Tensor] = None,
                 thresholds: Optional[Sequence[float]] = None,
                 parent_nbr: Optional[torch.Tensor] = None,
                 workspace: Optional[NeighborMapWorkspace] = None
                 ) -> Tuple[torch.Tensor, torch.Tensor]:
        dt = parent_feats.dtype
        child_coords, linear_idx, _ = subdivision_build(parent_coords, logits=logits, mask=mask,
                                                        thresholds=thresholds, with_pairs=False)
        if parent_nbr is None:
            parent_nbr = neighbor_rows_tensor_from_coords_tensor(self.conv1.cfg, parent_coords,
                                                                 workspace=workspace)
        h = layer_norm(parent_feats, self.norm1_weight, self.norm1_bias, eps=self.eps, silu=True)
        h1 = self.conv1(h, parent_nbr, out_dtype=dt)
        h_up = gather_rows(h1, 8, linear_idx)
        h_up = layer_norm(h_up, eps=self.eps, silu=True, out=h_up)
        child_nbr = neighbor_rows_tensor_from_coords_tensor(self.conv2.cfg, child_coords,
                                                            workspace=workspace)
        out = self.conv2(h_up, child_nbr, out_dtype=dt)
        c2s_skip_add(out, parent_feats, linear_idx)
        return child_coords, out


def transposed_upsample(parent_coords: torch.Tensor, parent_feats: torch.Tensor,
                        conv1x1: ConvLayer, mask: torch.Tensor
                        ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """2x2x2 stride-2 transposed sparse conv as C2S: a 1x1x1 conv Cin -> 8*Cout
    on the parents, then child selection.  Returns (child coords, child feats,
    linear_idx)."""
    K = conv1x1.cfg.kernel_d * conv1x1.cfg.kernel_h * conv1x1.cfg.kernel_w
    if K != 1:
        raise ValueError("transposed_upsample needs a 1x1x1 conv")
    child_coords, linear_idx, _ = subdivision_build(parent_coords, mask=mask, with_pairs=False)
    P = parent_coords.shape[0]
    ident = torch.arange(P, dtype=torch.int32, device=parent_coords.device).reshape(P, 1)
    h1 = conv1x1(parent_feats, ident, out_dtype=parent_feats.dtype)
    return child_coords, gather_rows(h1, 8, linear_idx), linear_idx

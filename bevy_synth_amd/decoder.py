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
* ``Neighborhood``    : one coord set's neighbour map and conv plan, built once
                        per resolution and shared by every 3x3x3 conv there.
* ``DecoderStack``    : config 5's decoder-shaped stack: per stage, residual
                        blocks then a C2S 2x upsample, int8 weights, bf16
                        activations.
* ``TrellisDecoderStage``: one stage of TRELLIS2's sparse structured-latent
                        decoder (sparse_decoder_runtime_impl.rs:522-1171):
                        ConvNeXt blocks, then the C2S upsample whose children
                        the to_subdiv logits choose; loaded from a checkpoint
                        by ``loading.load_decoder_stage``.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple, Union

import torch

from .flex_gmm import (ConvPlan, NeighborMapWorkspace, SparseSubmConvConfig, build_child_plan, build_conv_plan,
                       build_linear_child_plan,
                       c2s_skip_add, gather_rows, kernel_rows, layer_norm, linear_forward, linear_skinny,
                       neighbor_rows_tensor_from_coords_tensor, pack_conv_weight,
                       sparse_subm_conv_forward, subdivision_build, subdivision_build_indexed,
                       subdivision_launch, count_to_host_async,
                       subdivision_logits_finish)

LAYER_NORM32_EPS = 1e-6  # sparse_decoder.rs:43


@dataclass
class Neighborhood:
    """The neighbour map of one coord set and the conv plan built from it, made
    once per resolution and passed to every conv there (the reference decoder
    builds its map once per resolution and reuses it, sparse_decoder.rs
    :1057-1136, through its neighbour cache, crates/burn_flex_gmm/src/
    wgpu.rs:349-382)."""

    coords: torch.Tensor
    nbr: torch.Tensor
    plan: Optional[ConvPlan] = None

    @classmethod
    def build(cls, cfg: SparseSubmConvConfig, coords: torch.Tensor,
              workspace: Optional[NeighborMapWorkspace] = None, with_plan: bool = True,
              check_status: bool = True) -> "Neighborhood":
        """The map (and plan) of ``coords``.  check_status=False skips the
        map's status read-back (a sync), for coords this library derived from
        checked ones (C2S children: 2x + c of non-negative, distinct parents)."""
        nbr = neighbor_rows_tensor_from_coords_tensor(cfg, coords, workspace=workspace, check_status=check_status)
        plan = build_conv_plan(cfg, coords, nbr) if with_plan and kernel_rows(cfg) <= 32 else None
        return cls(coords, nbr, plan)


@dataclass
class ConvLayer:
    """One submanifold conv: weight [Cout, K, Cin_g] (bf16/f32/int8), bias f32,
    optional per-output-channel scale for int8 weights.  Given a Neighborhood
    with a plan, bf16 activations take the halo-staged kernel on weights
    packed once, on first use (the role of the reference's per-layer
    pack_flex_weight, crates/burn_flex_gmm/src/lib.rs:377-426)."""

    cfg: SparseSubmConvConfig
    weight: torch.Tensor
    bias: Optional[torch.Tensor] = None
    w_scale: Optional[torch.Tensor] = None
    packed: Optional[torch.Tensor] = field(default=None, repr=False)

    def packed_weight(self) -> Optional[torch.Tensor]:
        cin_g = self.cfg.to_c().in_channels_per_group
        if (self.packed is None and self.weight.dtype in (torch.bfloat16, torch.float16, torch.int8)
                and cin_g % 32 == 0):
            self.packed = pack_conv_weight(self.cfg, self.weight)
        return self.packed

    def __call__(self, x: torch.Tensor, nbr: Union[torch.Tensor, Neighborhood], out_dtype=None,
                 residual: Optional[torch.Tensor] = None, layer_norm: bool = False,
                 silu: bool = False, ln_eps: float = LAYER_NORM32_EPS, **epi) -> torch.Tensor:
        """``epi``: further epilogue arguments of sparse_subm_conv_forward
        (ln_weight / ln_bias, the C2S forms child_rows / n_child_rows and
        skip_parent / skip_index)."""
        plan, packed = None, None
        if isinstance(nbr, Neighborhood):
            if nbr.plan is not None and x.dtype in (torch.bfloat16, torch.float16):
                packed = self.packed_weight()
                plan = nbr.plan if packed is not None else None
            nbr = nbr.nbr
        return sparse_subm_conv_forward(self.cfg, x, nbr, self.weight, self.bias, self.w_scale,
                                        residual=residual, out_dtype=out_dtype,
                                        layer_norm=layer_norm, ln_eps=ln_eps, silu=silu,
                                        plan=plan, packed_weight=packed, **epi)


@dataclass
class ResidualBlock:
    conv1: ConvLayer
    conv2: ConvLayer
    eps: float = LAYER_NORM32_EPS

    def __call__(self, x: torch.Tensor, nbr: Union[torch.Tensor, Neighborhood]) -> torch.Tensor:
        # conv1 carries LayerNorm + SiLU in its epilogue; conv2 adds the residual.
        h = self.conv1(x, nbr, out_dtype=x.dtype, layer_norm=True, silu=True, ln_eps=self.eps)
        return self.conv2(h, nbr, out_dtype=x.dtype, residual=x)


@dataclass
class LinearLayer:
    """A dense layer, weight [Cout, Cin] (the reference's LinearLayer layout,
    sparse_decoder.rs; bf16 / f16 / f32, or int8 with w_scale), bias [Cout] f32."""

    weight: torch.Tensor
    bias: Optional[torch.Tensor] = None
    w_scale: Optional[torch.Tensor] = None

    def __call__(self, x: torch.Tensor, out_dtype=None, silu: bool = False,
                 residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        return linear_forward(x, self.weight, self.bias, self.w_scale, residual=residual, out_dtype=out_dtype,
                              silu=silu)


@dataclass
class ConvNeXtBlock:
    """TRELLIS2's sparse ConvNeXt block (convnext_blocks_forward_wgpu_tensor,
    sparse_decoder_wgpu_ops.rs:1091-1161; MLP :356-489):
        h = LN(conv3x3x3(x); norm affine) -> mlp_0 -> SiLU -> mlp_2 -> + x.
    The LayerNorm runs in the conv's epilogue (on f32 staging above 128
    channels), SiLU in mlp_0's and the residual in mlp_2's; each stored tensor
    is rounded once to the activation dtype."""

    conv: ConvLayer
    norm_weight: torch.Tensor
    norm_bias: torch.Tensor
    mlp_0: LinearLayer
    mlp_2: LinearLayer
    eps: float = LAYER_NORM32_EPS

    def __call__(self, x: torch.Tensor, nbr: Union[torch.Tensor, "Neighborhood"]) -> torch.Tensor:
        h = self.conv(x, nbr, out_dtype=x.dtype, layer_norm=True, ln_eps=self.eps, ln_weight=self.norm_weight,
                      ln_bias=self.norm_bias)
        return self.forward_tail(h, x)

    def forward_tail(self, h: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        hid = self.mlp_0(h, out_dtype=x.dtype, silu=True)
        return self.mlp_2(hid, out_dtype=x.dtype, residual=x)


@dataclass
class C2SUpsampleBlock:
    in_channels: int
    out_channels: int
    norm1_weight: torch.Tensor
    norm1_bias: torch.Tensor
    conv1: ConvLayer   # Cin -> 8*Cout on parent coords
    conv2: ConvLayer   # Cout -> Cout on child coords
    eps: float = LAYER_NORM32_EPS
    # to_subdiv head (Linear Cin -> 8, f32): the subdivision logits when no
    # mask or logits are given (sparse_decoder_runtime_impl.rs:859-866)
    to_subdiv_weight: Optional[torch.Tensor] = None
    to_subdiv_bias: Optional[torch.Tensor] = None
    # fused: conv1 writes only the active children's slices and normalises
    # them in its epilogue; conv2 adds the parent skip in its epilogue.
    # Unfused: the reference's composition (conv1 [P, 8*Cout] -> select ->
    # LayerNorm -> conv2 -> skip add), kept as the comparison path.
    fused: bool = True
    # the decoder's logits options: f16 rounding of the logits under
    # compute_fp16 (the to_subdiv weights are then f16-rounded too, by the
    # loader), and centering each row (center_subdivision_logits)
    compute_fp16: bool = False
    center_logits: bool = False
    # fused conv1 over the active children only (a child plan of the
    # parents' plan), when the shapes allow it: else all eight children are
    # computed and the inactive ones dropped in the store
    child_plans: bool = True

    def __call__(self, parent_coords: torch.Tensor, parent_feats: torch.Tensor,
                 logits: Optional[torch.Tensor] = None, mask: Optional[torch.Tensor] = None,
                 thresholds: Optional[Sequence[float]] = None,
                 parent_nbr: Optional[torch.Tensor] = None,
                 workspace: Optional[NeighborMapWorkspace] = None
                 ) -> Tuple[torch.Tensor, torch.Tensor]:
        if parent_nbr is None:
            parent_nb = Neighborhood.build(self.conv1.cfg, parent_coords, workspace)
        else:
            parent_nb = Neighborhood(parent_coords, parent_nbr)
        child_nb, out = self.forward(parent_nb, parent_feats, logits=logits, mask=mask,
                                     thresholds=thresholds, workspace=workspace)
        return child_nb.coords, out

    def forward(self, parent_nb: Neighborhood, parent_feats: torch.Tensor,
                logits: Optional[torch.Tensor] = None, mask: Optional[torch.Tensor] = None,
                thresholds: Optional[Sequence[float]] = None,
                workspace: Optional[NeighborMapWorkspace] = None
                ) -> Tuple[Neighborhood, torch.Tensor]:
        """The block on a parent Neighborhood; returns the children's
        Neighborhood (map + plan, for the next stage's convs) and features."""
        dt = parent_feats.dtype
        if logits is None and mask is None:
            if self.to_subdiv_weight is None:
                raise ValueError("C2S upsample needs a mask, logits or a to_subdiv head")
            logits = self.subdivision_logits(parent_feats)
        h = layer_norm(parent_feats, self.norm1_weight, self.norm1_bias, eps=self.eps, silu=True)
        if self.fused:
            # conv1 and its child plan are sized by the bound 8P, so they are
            # enqueued before the child count reaches the host: the count's
            # read-back overlaps conv1 instead of idling the GPU (conv1 writes
            # only the rows child_rows names, all below the count)
            P = parent_nb.coords.shape[0]
            sb = subdivision_launch(parent_nb.coords, logits=logits, mask=mask, thresholds=thresholds)
            host_count, count_ready = count_to_host_async(sb.count)
            child_rows = sb.rows[:P]
            A_max = 8 * P
            nb1 = parent_nb
            if (self.child_plans and parent_nb.plan is not None and A_max > 0
                    and dt in (torch.bfloat16, torch.float16)
                    and (self.conv1.cfg.out_channels == 512 or self.conv1.cfg.out_channels % 1024 == 0)
                    and self.conv1.cfg.groups == 1
                    and self.conv1.packed_weight() is not None):
                cp = build_child_plan(self.conv1.cfg, parent_nb.plan, parent_nb.nbr, child_rows, A_max)
                nb1 = Neighborhood(parent_nb.coords, parent_nb.nbr, cp)
            h_up = self.conv1(h, nb1, out_dtype=dt, layer_norm=True, silu=True, ln_eps=self.eps,
                              child_rows=child_rows, n_child_rows=A_max, child_count=sb.count)
            count_ready.synchronize()
            A = int(host_count[0])
            child_coords, linear_idx, h_up = sb.child[:A], sb.lin[:A], h_up[:A]
        else:
            child_coords, linear_idx, _ = subdivision_build(parent_nb.coords, logits=logits, mask=mask,
                                                            thresholds=thresholds, with_pairs=False)
            h1 = self.conv1(h, parent_nb, out_dtype=dt)
            h_up = gather_rows(h1, 8, linear_idx)
            h_up = layer_norm(h_up, eps=self.eps, silu=True, out=h_up)
        child_nb = Neighborhood.build(self.conv2.cfg, child_coords, workspace,
                                      with_plan=parent_nb.plan is not None, check_status=not self.fused)
        if self.fused:
            out = self.conv2(h_up, child_nb, out_dtype=dt, skip_parent=parent_feats, skip_index=linear_idx)
        else:
            out = self.conv2(h_up, child_nb, out_dtype=dt)
            c2s_skip_add(out, parent_feats, linear_idx)
        return child_nb, out

    def subdivision_logits(self, parent_feats: torch.Tensor) -> torch.Tensor:
        """to_subdiv: [P, 8] f32 logits of the parent features (the skinny
        linear, linear_skinny_forward_wgpu, crates/burn_flex_gmm/src/wgpu/
        ops.rs:1390-1410), then rounded to f16 under compute_fp16 and
        centered per row when asked (sparse_decoder_runtime_impl.rs:859-878)."""
        logits = linear_skinny(parent_feats, self.to_subdiv_weight, self.to_subdiv_bias)
        return subdivision_logits_finish(logits, round_f16=self.compute_fp16, center=self.center_logits)


def transposed_upsample(parent_coords: torch.Tensor, parent_feats: torch.Tensor,
                        conv1x1: ConvLayer, mask: torch.Tensor, active_only: bool = True
                        ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """2x2x2 stride-2 transposed sparse conv as C2S: a 1x1x1 conv Cin -> 8*Cout
    on the parents (parent p's own row: the dense linear, no map) whose
    epilogue writes each active child's Cout slice to the child's row (no
    [P, 8*Cout] tensor).  With ``active_only`` (and 16-bit weights, Cout a
    multiple of 128, Cin of 32) a linear child plan lists, per child index,
    the parents whose child is active, and only those (parent, child) pairs
    are computed; the values are the same.  Returns (child coords, child
    feats, linear_idx)."""
    cfg = conv1x1.cfg
    if cfg.kernel_d * cfg.kernel_h * cfg.kernel_w != 1 or cfg.groups != 1:
        raise ValueError("transposed_upsample needs a 1x1x1 conv with groups == 1")
    child_coords, linear_idx, child_rows = subdivision_build_indexed(parent_coords, mask=mask)
    w = conv1x1.weight.reshape(cfg.out_channels, cfg.in_channels)
    n_children = child_coords.shape[0]
    plan = None
    if (active_only and n_children > 0 and parent_feats.dtype in (torch.bfloat16, torch.float16)
            and w.dtype == parent_feats.dtype and (cfg.out_channels // 8) % 128 == 0
            and cfg.in_channels % 32 == 0):
        plan = build_linear_child_plan(child_rows, n_children)
    h_up = linear_forward(parent_feats, w, conv1x1.bias, conv1x1.w_scale, out_dtype=parent_feats.dtype,
                          child_rows=child_rows, n_child_rows=n_children, child_plan=plan)
    return child_coords, h_up, linear_idx


@dataclass
class DecoderStage:
    blocks: List[ResidualBlock]
    up: C2SUpsampleBlock


@dataclass
class DecoderStack:
    """Config 5's decoder-shaped stack: per stage, residual blocks at the
    stage's resolution, then a C2S 2x upsample (sparse_decoder_runtime_impl.rs
    :758-1171) to the next resolution; one Neighborhood (map + plan) per
    resolution, shared by the stage's convs and the next stage's."""

    stages: List[DecoderStage]

    def __call__(self, coords: torch.Tensor, feats: torch.Tensor, masks: Sequence[torch.Tensor],
                 workspace: Optional[NeighborMapWorkspace] = None, with_plan: bool = True,
                 trace: Optional[list] = None) -> Tuple[Neighborhood, torch.Tensor]:
        """coords [N, 4] i32 and feats [N, C0] at the first resolution; masks[s]
        [P_s, 8] u8 selects stage s's children.  ``trace`` (a list) receives
        (stage, "block", Neighborhood, input, output, block) per residual block
        and (stage, "up", parent Neighborhood, input, output, child
        Neighborhood) per upsample, for tests."""
        st0 = self.stages[0]
        cfg0 = st0.blocks[0].conv1.cfg if st0.blocks else st0.up.conv1.cfg
        nb = Neighborhood.build(cfg0, coords, workspace, with_plan=with_plan)
        x = feats
        for s, st in enumerate(self.stages):
            for blk in st.blocks:
                y = blk(x, nb)
                if trace is not None:
                    trace.append((s, "block", nb, x, y, blk))
                x = y
            child_nb, y = st.up.forward(nb, x, mask=masks[s], workspace=workspace)
            if trace is not None:
                trace.append((s, "up", nb, x, y, child_nb))
            nb, x = child_nb, y
        return nb, x


# decoder_subdivision_child_thresholds (sparse_decoder_wgpu_ops.rs:1813-1822)
# with DecoderRuntimeConfig's defaults (sparse_decoder.rs:182-190): every
# child's threshold is the global 0.0.
DEFAULT_SUBDIVISION_THRESHOLDS = (0.0,) * 8


def subdivision_child_thresholds(threshold: float = 0.0,
                                 child_thresholds: Optional[Sequence[float]] = None) -> Tuple[float, ...]:
    """decoder_subdivision_child_thresholds: the global threshold, replaced
    per child by a finite child threshold."""
    import math
    out = [float(threshold)] * 8
    if child_thresholds is not None:
        for c, t in enumerate(child_thresholds):
            if math.isfinite(t):
                out[c] = float(t)
    return tuple(out)


@dataclass
class TrellisDecoderStage:
    """One stage of TRELLIS2's sparse structured-latent decoder
    (SparseStructuredLatentDecoder, sparse_decoder_runtime_impl.rs:522-1171;
    DecoderStage, sparse_decoder.rs): the stage's ConvNeXt blocks on one
    Neighborhood, then -- every stage but the last -- the C2S upsample, whose
    children the to_subdiv logits select against the thresholds
    (logits_to_mask: logit > threshold, sparse_decoder_wgpu_ops.rs:1759-1811).
    Built from a checkpoint by ``loading.load_decoder_stage``."""

    convnext_blocks: List[ConvNeXtBlock]
    upsample: Optional[C2SUpsampleBlock] = None

    def forward(self, nb: Neighborhood, feats: torch.Tensor,
                thresholds: Sequence[float] = DEFAULT_SUBDIVISION_THRESHOLDS,
                mask: Optional[torch.Tensor] = None, workspace: Optional[NeighborMapWorkspace] = None,
                trace: Optional[list] = None) -> Tuple[Neighborhood, torch.Tensor]:
        """feats [N, C] at ``nb``'s coords -> (the next resolution's
        Neighborhood, its features); the last stage returns ``nb`` itself.
        ``mask`` [P, 8] (the reference's guide subdivisions) replaces the
        logits.  ``trace`` (a list) receives ("convnext", b, input, output),
        ("logits", parent feats, logits) and ("up", parent feats, output)."""
        x = feats
        for b, blk in enumerate(self.convnext_blocks):
            y = blk(x, nb)
            if trace is not None:
                trace.append(("convnext", b, x, y))
            x = y
        if self.upsample is None:
            return nb, x
        logits = None
        if mask is None:
            if self.upsample.to_subdiv_weight is None:
                raise ValueError("decoder stage requires guide_subdivisions but none were provided")
            logits = self.upsample.subdivision_logits(x)
            if trace is not None:
                trace.append(("logits", x, logits))
        child_nb, out = self.upsample.forward(nb, x, logits=logits, mask=mask, thresholds=thresholds,
                                              workspace=workspace)
        if trace is not None:
            trace.append(("up", x, out))
        return child_nb, out

    def __call__(self, coords: torch.Tensor, feats: torch.Tensor, **kw) -> Tuple[torch.Tensor, torch.Tensor]:
        """coords [N, 4] i32 -> (child coords, child features)."""
        cfg = (self.convnext_blocks[0].conv.cfg if self.convnext_blocks
               else self.upsample.conv1.cfg)
        nb = Neighborhood.build(cfg, coords, kw.get("workspace"))
        out_nb, out = self.forward(nb, feats, **kw)
        return out_nb.coords, out


def int8_stack(channels: Sequence[int], blocks_per_stage: int, seed: int,
               device=None) -> DecoderStack:
    """A random-weight stack shaped as config 5 (channels e.g. 512, 256, 128,
    64): per stage ``blocks_per_stage`` residual blocks at channels[s] and a
    C2S upsample channels[s] -> channels[s+1]; every conv 3x3x3 with
    per-output-channel symmetric int8 weights (q ~ U{-127..127}, scale ~
    U(0.5, 1.5)/127, so w = q * scale has std ~1/sqrt(3)); the scales are
    divided by sqrt(27 * Cin) to keep activations O(1).  Zero conv biases;
    norm1 affine ~ N(1, 0.1) / N(0, 0.1)."""
    import numpy as np

    from . import synth

    dev = torch.device("cuda") if device is None else torch.device(device)
    rng = np.random.default_rng(seed)

    def layer(cin: int, cout: int) -> ConvLayer:
        q, scale = synth.int8_weight(rng, cout, 27, cin)
        scale = (scale / np.sqrt(27 * cin / 3.0)).astype(np.float32)
        return ConvLayer(SparseSubmConvConfig(cin, cout), torch.from_numpy(q).to(dev),
                         torch.zeros(cout, dtype=torch.float32, device=dev),
                         torch.from_numpy(scale).to(dev))

    stages = []
    for s in range(len(channels) - 1):
        c, c2 = channels[s], channels[s + 1]
        blocks = [ResidualBlock(layer(c, c), layer(c, c)) for _ in range(blocks_per_stage)]
        n1w = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(c)).astype(np.float32)).to(dev)
        n1b = torch.from_numpy((0.1 * rng.standard_normal(c)).astype(np.float32)).to(dev)
        up = C2SUpsampleBlock(c, c2, n1w, n1b, layer(c, 8 * c2), layer(c2, c2))
        stages.append(DecoderStage(blocks, up))
    return DecoderStack(stages)

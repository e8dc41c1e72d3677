"""GPU parity of the dense linear (sc_linear_forward: the conv tiles with a
1x1x1 kernel and no map) and of TRELLIS2's sparse ConvNeXt block built on it:
conv3x3x3 -> LayerNorm (affine) -> Linear -> SiLU -> Linear -> + x
(convnext_blocks_forward_wgpu_tensor, sparse_decoder_wgpu_ops.rs:1091-1161;
MLP :356-489).

References: the fp64 conv definition (oracle.conv_gemm_f64; a 1x1x1 kernel
with the identity map is the dense layer x W^T + b), the oracle's LayerNorm
and SiLU, bf16 / f16 rounding where the device stores the tensor (f16: the
reference's compute_fp16 fences).  Bars: 1e-4 f32, 1e-2 bf16 / f16."""
import numpy as np
import pytest
import torch

from bevy_synth_amd import decoder as D
from bevy_synth_amd import flex_gmm as F
from bevy_synth_amd import synth
from tests.sampling import sample_rows
from tests.tolerance import TOL_BF16, TOL_F32, assert_close

pytestmark = pytest.mark.gpu

TYPES = {torch.float32: (lambda o, a: np.asarray(a, np.float32), TOL_F32),
         torch.bfloat16: (lambda o, a: o.bf16_round(a), TOL_BF16),
         torch.float16: (lambda o, a: o.f16_round(a), TOL_BF16)}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def to_dev(x, dtype):
    t = dev(np.asarray(x, np.float32))
    return t.to(dtype)  # exact: x already holds dtype-representable values


def host(t):
    return t.float().cpu().numpy()


def dense_f64(oracle, w, b, x):
    cout, cin = w.shape
    ident = np.arange(len(x), dtype=np.int32).reshape(-1, 1)
    return oracle.conv_gemm_f64(oracle.OracleConfig(cin, cout, 1, 1, 1), w.reshape(cout, 1, cin), b, x, ident)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("cin,cout,epi", [(128, 512, "silu"), (512, 128, "residual"), (96, 64, "ln"),
                                          (128, 256, "ln"), (64, 40, "none"),
                                          # 256-channel tiles (129-256 channels): a k-loop of 3 steps
                                          # and a residual through the staged stores, one k-step with
                                          # SiLU, a partial tile, and 196 channels (direct stores)
                                          (96, 200, "residual"), (32, 136, "silu"), (64, 196, "none"),
                                          (1024, 256, "residual")])
def test_linear_forward(oracle, dtype, cin, cout, epi):
    """x W^T + b with each epilogue, on both tile widths (128 and 256 channels), k-loops from 1
    to 32 steps, whole and partial column tiles, and row-contiguous (staged) and direct
    stores; 70,001 rows, so the last row tile is partial."""
    rnd, tol = TYPES[dtype]
    rng = np.random.default_rng(cin + cout)
    rows = 70001
    x = rnd(oracle, synth.normal_f32(rng, (rows, cin)))
    w = rnd(oracle, synth.normal_f32(rng, (cout, cin), 1 / np.sqrt(cin)))
    b = synth.normal_f32(rng, cout, 0.2)
    res = rnd(oracle, synth.normal_f32(rng, (rows, cout))) if epi == "residual" else None
    lw = synth.normal_f32(rng, cout) if epi == "ln" else None
    lb = synth.normal_f32(rng, cout) if epi == "ln" else None
    got = F.linear_forward(to_dev(x, dtype), to_dev(w, dtype), dev(b),
                           residual=None if res is None else to_dev(res, dtype), silu=epi == "silu",
                           layer_norm=epi == "ln", ln_weight=None if lw is None else dev(lw),
                           ln_bias=None if lb is None else dev(lb))
    exp = dense_f64(oracle, w, b, x)
    if epi == "silu":
        exp = oracle.silu(exp.astype(np.float32))
    elif epi == "ln":
        exp = oracle.layer_norm(exp.astype(np.float32), lw, lb, 1e-6)
    elif epi == "residual":
        exp = exp + res
    assert got.shape == (rows, cout) and got.dtype == dtype
    assert_close(host(got), exp, tol, f"linear {cin}->{cout} {epi}")


def _block(rng, C, H, dtype, rnd, oracle):
    def w3(ci, co):
        return rnd(oracle, synth.conv_weight(rng, co, 27, ci, 1 / np.sqrt(27 * ci)))

    def lin(ci, co):
        return rnd(oracle, synth.normal_f32(rng, (co, ci), 1 / np.sqrt(ci)))
    wc, w0, w2 = w3(C, C), lin(C, H), lin(H, C)
    bc, b0, b2 = (synth.normal_f32(rng, n, 0.1) for n in (C, H, C))
    nw, nb = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32), (0.1 * rng.standard_normal(C)).astype(np.float32)
    blk = D.ConvNeXtBlock(D.ConvLayer(F.SparseSubmConvConfig(C, C), to_dev(wc, dtype), dev(bc)), dev(nw), dev(nb),
                          D.LinearLayer(to_dev(w0, dtype), dev(b0)), D.LinearLayer(to_dev(w2, dtype), dev(b2)))
    return blk, (wc, bc, nw, nb, w0, b0, w2, b2)


@pytest.mark.parametrize("dtype,C,H", [(torch.bfloat16, 128, 512), (torch.float16, 128, 512),
                                       (torch.bfloat16, 256, 1024)])
def test_convnext_block(oracle, dtype, C, H):
    """The block on the config-2 shell (113,857 voxels) through the planned
    conv, 2,000 sampled rows against the oracle chain with the device's
    rounding points: conv -> LN(affine) (stored) -> mlp_0 -> SiLU (stored) ->
    mlp_2 + x (stored).  For f16 the chain rounds at each of the reference's
    compute_fp16 fences instead."""
    rnd, _ = TYPES[dtype]
    coords = synth.config2_coords()
    rng = np.random.default_rng(C + H + (dtype == torch.float16))
    blk, (wc, bc, nw, nb, w0, b0, w2, b2) = _block(rng, C, H, dtype, rnd, oracle)
    x = rnd(oracle, synth.normal_f32(rng, (len(coords), C)))
    nbh = D.Neighborhood.build(blk.conv.cfg, dev(coords))
    y = blk(to_dev(x, dtype), nbh)
    assert y.dtype == dtype
    rows = sample_rows(len(coords), rng, 2000, plan=nbh.plan)
    m = nbh.nbr.cpu().numpy()[rows]
    conv = oracle.conv_gemm_f64(oracle.OracleConfig(C, C), wc, bc, x, m).astype(np.float32)
    f16 = dtype == torch.float16
    if f16:
        conv = rnd(oracle, conv)
    h = rnd(oracle, oracle.layer_norm(conv, nw, nb, 1e-6))
    hid = dense_f64(oracle, w0, b0, h).astype(np.float32)
    if f16:
        hid = rnd(oracle, hid)
    hid = rnd(oracle, oracle.silu(hid))
    out = dense_f64(oracle, w2, b2, hid).astype(np.float32)
    if f16:
        out = rnd(oracle, out)
    exp = out + x[rows]
    assert_close(host(y)[rows], exp, TOL_BF16, f"convnext block {dtype} C={C}")

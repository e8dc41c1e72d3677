"""GPU parity of the HIP submanifold conv against the oracle.

f32: within 1e-4 of the oracle's flex path and of its fp64 definition.
bf16 (bf16 operands, f32 accumulate): within 1e-2 of the fp64 definition on
the same bf16-rounded operands.  Metric: max |a-b| / max(|b|, rms(b))."""
import numpy as np
import pytest
import torch

from bevy_synth_amd import flex_gmm as F
from bevy_synth_amd import synth
from tests.tolerance import TOL_BF16, TOL_F32, assert_close

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bf16_dev(x_f32):
    return dev(synth.bf16_bits(x_f32).view(np.int16)).view(torch.bfloat16)


def ocfg(oracle, cfg):
    return oracle.OracleConfig(cfg.in_channels, cfg.out_channels, cfg.kernel_d, cfg.kernel_h,
                               cfg.kernel_w, groups=cfg.groups, axis_order=cfg.axis_order,
                               axis_sign=cfg.axis_sign)


def line_coords(n):
    c = np.zeros((n, 4), np.int32)
    c[:, 1] = np.arange(n)
    return c


def run_f32(cfg, coords, x, w, b, **kw):
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, dev(coords))
    out = F.sparse_subm_conv_forward(cfg, dev(x), nbr, dev(w), dev(b), **kw)
    return out.cpu().numpy(), nbr.cpu().numpy()


def test_kat_conv_uses_neighbor_voxels(kats):
    """sparse_decoder_tests.rs:190-236 -> [201, 12]."""
    g = kats["conv_uses_neighbor_voxels"]
    cfg = F.SparseSubmConvConfig(1, 1, *g["config"]["kernel"])
    out, _ = run_f32(cfg, np.array(g["coords"], np.int32), np.array(g["input"], np.float32),
                     np.array(g["weight"], np.float32), np.array(g["bias"], np.float32))
    assert np.abs(out - np.array(g["expected_output"], np.float32)).max() < g["tolerance"]


@pytest.mark.parametrize("cin,cout,dims,groups,n,seed", [
    (4, 6, (3, 1, 1), 2, 16, 42),      # crates/burn_flex_gmm/src/lib.rs:799-840
    (8, 12, (3, 1, 1), 2, 32, 73),     # lib.rs:864-915
    (4, 6, (3, 1, 1), 2, 32, 123),     # sparse_decoder_tests.rs:295-368
    (64, 128, (3, 3, 3), 1, 4096, 7),  # benches/sparse_subm_conv.rs:37-69 (line coords)
    (64, 128, (3, 3, 3), 1, 192, 9),   # wgpu/tests.rs:1361-1503 (conv vs CPU flex)
])
def test_reference_shapes_f32(oracle, cin, cout, dims, groups, n, seed):
    cfg = F.SparseSubmConvConfig(cin, cout, *dims, groups=groups)
    oc = ocfg(oracle, cfg)
    rng = oracle.Lcg(seed)
    x = rng.next_f32(n * cin).reshape(n, cin)
    w = rng.next_f32(cout * oc.kernel_rows * (cin // groups))
    b = rng.next_f32(cout)
    coords = line_coords(n)
    got, nbr = run_f32(cfg, coords, x, w, b)
    flex = oracle.conv_flex(oc, w, b, coords, x)
    assert np.max(np.abs(got - flex)) <= 1e-4
    assert_close(got, oracle.conv_ref_f64(oc, w, b, x, nbr), TOL_F32, "vs f64")


@pytest.mark.parametrize("axis_order,axis_sign", [((0, 1, 2), (1, 1, 1)), ((2, 1, 0), (-1, 1, 1)),
                                                  ((1, 2, 0), (1, -1, -1))])
def test_checkerboard_axes_groups_f32(oracle, axis_order, axis_sign):
    """lib.rs:917-972 shapes through the device path (scalar kernel: Cin_g = 3)."""
    c = [(0, x, y, z) for x in range(6) for y in range(5) for z in range(4) if (x + y + z) % 2 == 0]
    coords = np.array(c, np.int32)
    rng = oracle.Lcg(991)
    x = rng.next_f32(len(coords) * 6).reshape(-1, 6)
    w = rng.next_f32(8 * 27 * 3)
    b = rng.next_f32(8)
    cfg = F.SparseSubmConvConfig(6, 8, groups=2, axis_order=axis_order, axis_sign=axis_sign)
    got, _ = run_f32(cfg, coords, x, w, b)
    assert np.max(np.abs(got - oracle.conv_legacy(ocfg(oracle, cfg), w, b, coords, x))) <= 1e-4


def test_config1_f32_mfma(oracle):
    """Config 1: 64^3 sphere shell, 14,648 voxels, C=64, f32 (MFMA f32 path)."""
    coords = synth.config1_coords()
    rng = np.random.default_rng(1)
    n = len(coords)
    x = synth.normal_f32(rng, (n, 64))
    w = synth.conv_weight(rng, 64, 27, 64, 1.0 / np.sqrt(27 * 64))
    b = np.zeros(64, np.float32)
    cfg = F.SparseSubmConvConfig(64, 64)
    got, nbr = run_f32(cfg, coords, x, w, b)
    oc = ocfg(oracle, cfg)
    assert_close(got, oracle.conv_ref_f64(oc, w, b, x, nbr), TOL_F32, "config1 vs f64")
    assert_close(got, oracle.conv_flex_precomputed(oc, w, b, x, nbr), TOL_F32, "config1 vs flex")


@pytest.mark.parametrize("cin,cout,groups", [(32, 32, 1), (64, 96, 1), (128, 128, 1),
                                             (256, 64, 1), (64, 64, 2), (96, 200, 1)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_bf16_mfma_shapes(oracle, cin, cout, groups, out_dtype):
    coords = synth.config1_coords()[:6000]
    rng = np.random.default_rng(cin * 7 + cout + groups)
    n = len(coords)
    x = synth.bf16_to_f32(synth.bf16_bits(synth.normal_f32(rng, (n, cin))))
    w = synth.bf16_to_f32(synth.bf16_bits(
        synth.conv_weight(rng, cout, 27, cin // groups, 1.0 / np.sqrt(27 * cin))))
    b = synth.normal_f32(rng, cout, 0.1)
    cfg = F.SparseSubmConvConfig(cin, cout, groups=groups)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, dev(coords))
    out = F.sparse_subm_conv_forward(cfg, bf16_dev(x), nbr, bf16_dev(w), dev(b), out_dtype=out_dtype)
    got = out.float().cpu().numpy()
    exp = oracle.conv_ref_f64(ocfg(oracle, cfg), w, b, x, nbr.cpu().numpy())
    assert_close(got, exp, TOL_BF16 if out_dtype == torch.bfloat16 else 2e-5, "bf16 conv")


def test_int8_weights_w8a16(oracle):
    coords = synth.config1_coords()[:5000]
    rng = np.random.default_rng(5)
    n, cin, cout = len(coords), 128, 64
    x = synth.bf16_to_f32(synth.bf16_bits(synth.normal_f32(rng, (n, cin))))
    q, scale = synth.int8_weight(rng, cout, 27, cin)
    b = synth.normal_f32(rng, cout, 0.1)
    cfg = F.SparseSubmConvConfig(cin, cout)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, dev(coords))
    out = F.sparse_subm_conv_forward(cfg, bf16_dev(x), nbr, dev(q), dev(b), w_scale=dev(scale),
                                     out_dtype=torch.float32)
    exp = oracle.conv_ref_f64(ocfg(oracle, cfg), q.astype(np.float32), b, x, nbr.cpu().numpy(),
                              w_scale=scale)
    assert_close(out.cpu().numpy(), exp, 2e-5, "int8 conv")


def test_k1_is_dense_gemm():
    """K = 1 over the identity map is in @ W^T + b (torch f32 reference)."""
    rng = np.random.default_rng(2)
    n, cin, cout = 3000, 128, 256
    x = synth.bf16_to_f32(synth.bf16_bits(synth.normal_f32(rng, (n, cin))))
    w = synth.bf16_to_f32(synth.bf16_bits(synth.normal_f32(rng, (cout, 1, cin), 0.1)))
    b = synth.normal_f32(rng, cout)
    cfg = F.SparseSubmConvConfig(cin, cout, 1, 1, 1)
    ident = torch.arange(n, dtype=torch.int32, device="cuda").reshape(n, 1)
    out = F.sparse_subm_conv_forward(cfg, bf16_dev(x), ident, bf16_dev(w), dev(b),
                                     out_dtype=torch.float32)
    ref = torch.from_numpy(x).double() @ torch.from_numpy(w[:, 0, :]).double().T + torch.from_numpy(b).double()
    assert_close(out.cpu().numpy(), ref.numpy(), 2e-5, "k1 gemm")


def test_residual_and_query_subset(oracle):
    coords = synth.config1_coords()
    rng = np.random.default_rng(4)
    n, c = len(coords), 64
    x = synth.bf16_to_f32(synth.bf16_bits(synth.normal_f32(rng, (n, c))))
    w = synth.bf16_to_f32(synth.bf16_bits(synth.conv_weight(rng, c, 27, c, 0.03)))
    b = synth.normal_f32(rng, c, 0.1)
    res = synth.normal_f32(rng, (5000, c))
    cfg = F.SparseSubmConvConfig(c, c)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, dev(coords), query_rows=5000)
    out = F.sparse_subm_conv_forward(cfg, bf16_dev(x), nbr, bf16_dev(w), dev(b),
                                     residual=dev(res), out_dtype=torch.float32)
    exp = oracle.conv_ref_f64(ocfg(oracle, cfg), w, b, x, nbr.cpu().numpy()) + res
    assert_close(out.cpu().numpy(), exp, 2e-5, "residual")


def test_isolated_rows_get_bias():
    cfg = F.SparseSubmConvConfig(64, 64)
    coords = np.zeros((300, 4), np.int32)
    coords[:, 1] = np.arange(300) * 3
    rng = np.random.default_rng(0)
    x = synth.normal_f32(rng, (300, 64))
    w = synth.normal_f32(rng, (64, 27, 64))
    w[:, 13, :] = 0
    b = synth.normal_f32(rng, 64)
    got, _ = run_f32(cfg, coords, x, w, b)
    assert np.array_equal(got, np.broadcast_to(b, got.shape))


def test_config3_sampled_rows_and_determinism(oracle):
    """Config 3 size (1.04M voxels, C=128, bf16): sampled rows against the fp64
    definition, and bit-identical output across two runs."""
    coords = synth.config3_coords()
    n, c = len(coords), 128
    rng = np.random.default_rng(3)
    x = synth.bf16_to_f32(synth.bf16_bits(synth.normal_f32(rng, (n, c))))
    w = synth.bf16_to_f32(synth.bf16_bits(synth.conv_weight(rng, c, 27, c, 1.0 / np.sqrt(27 * c))))
    b = np.zeros(c, np.float32)
    cfg = F.SparseSubmConvConfig(c, c)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, dev(coords))
    xd, wd, bd = bf16_dev(x), bf16_dev(w), dev(b)
    out1 = F.sparse_subm_conv_forward(cfg, xd, nbr, wd, bd, out_dtype=torch.bfloat16)
    out2 = F.sparse_subm_conv_forward(cfg, xd, nbr, wd, bd, out_dtype=torch.bfloat16)
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    sample = np.sort(np.random.default_rng(0).choice(n, 3000, replace=False))
    nb = nbr.cpu().numpy()[sample]
    exp = oracle.conv_ref_f64(ocfg(oracle, cfg), w, b, x, nb)
    assert_close(out1.float().cpu().numpy()[sample], exp, TOL_BF16, "config3 sampled")

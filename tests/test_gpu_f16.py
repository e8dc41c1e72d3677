"""GPU parity of the f16 path (SC_DTYPE_F16: f16 activations and weights on
v_mfma_f32_16x16x32_f16, f32 accumulation) -- the decoder's compute_fp16 mode.

The reference computes in f32 on f16-rounded operands and rounds to f16 at
its fences: after each conv, after LayerNorm and after SiLU
(layer_norm_silu_wgpu_with_fp16_fences, sparse_decoder_wgpu_ops.rs:313-334;
quantize_f16_tensor_wgpu, :1082-1088).  The oracle chains below apply exactly
those fences (oracle.f16_round, pinned to numpy's float16); the device rounds
once per stored tensor.  Bar: 1e-2 (tests/tolerance.py), shapes of configs
1-3 at full size (sampled rows where the check is large)."""
import numpy as np
import pytest
import torch

from bevy_synth_amd import flex_gmm as F
from bevy_synth_amd import synth
from tests.sampling import sample_rows
from tests.tolerance import TOL_BF16, assert_close, rel_err

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def f16_dev(x):
    return dev(np.asarray(x, np.float32).astype(np.float16))


def host(t):
    return t.float().cpu().numpy()


def test_convert_f16_matches_reference_rounding(oracle):
    rng = np.random.default_rng(16)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * np.float32(s)
                        for s in (1e-6, 1e-3, 1.0, 300.0, 6e4)] +
                       [np.array([65504, 65519.99, 65520, 2.0 ** -24, 2.0 ** -25, -0.0], np.float32)])
    got = F.convert(dev(x), torch.float16).float().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), oracle.f16_round(x).view(np.uint32))


def _fence(oracle, a):
    return oracle.f16_round(np.asarray(a, np.float32))


@pytest.mark.parametrize("planned", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
def test_config1_conv_f16(oracle, planned, out_dtype):
    """Config 1's shape (64^3 sphere shell, 14,648 voxels, C = 64) in f16, every row."""
    coords = synth.config1_coords()
    rng = np.random.default_rng(161)
    C = 64
    x = _fence(oracle, synth.normal_f32(rng, (len(coords), C)))
    w = _fence(oracle, synth.conv_weight(rng, C, 27, C, 1 / np.sqrt(27 * C)))
    b = synth.normal_f32(rng, C, 0.1)
    cfg = F.SparseSubmConvConfig(C, C)
    cd = dev(coords)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd)
    wd = f16_dev(w)
    kw = {}
    if planned:
        kw = dict(plan=F.build_conv_plan(cfg, cd, nbr), packed_weight=F.pack_conv_weight(cfg, wd))
    got = F.sparse_subm_conv_forward(cfg, f16_dev(x), nbr, wd, dev(b), out_dtype=out_dtype, **kw)
    exp = oracle.conv_gemm_f64(oracle.OracleConfig(C, C), w, b, x, nbr.cpu().numpy())
    e = assert_close(host(got), exp, TOL_BF16, "config 1 f16 conv")
    # f32 accumulation of exact f16 products: well inside one f16 rounding
    assert e <= (1e-3 if out_dtype == torch.float16 else 1e-4), e


@pytest.mark.parametrize("kernel,n", [((3, 3, 1), 14648), ((1, 1, 1), 14648), ((3, 3, 3), 257)])
@pytest.mark.parametrize("cout", [64, 128])
def test_f16_planned_few_offsets_and_rows(oracle, kernel, n, cout):
    """The planned f16 tile on plans over 9 and 1 offsets, and on 257 rows
    (a full tile then a one-row tile), at both tile widths."""
    coords = np.ascontiguousarray(synth.config1_coords()[:n])
    rng = np.random.default_rng(n + cout + sum(kernel))
    cin = 64
    K = kernel[0] * kernel[1] * kernel[2]
    x = _fence(oracle, synth.normal_f32(rng, (n, cin)))
    w = _fence(oracle, synth.conv_weight(rng, cout, K, cin, 1 / np.sqrt(K * cin)))
    b = synth.normal_f32(rng, cout, 0.1)
    cfg = F.SparseSubmConvConfig(cin, cout, *kernel)
    cd = dev(coords)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd)
    wd = f16_dev(w)
    got = F.sparse_subm_conv_forward(cfg, f16_dev(x), nbr, wd, dev(b), out_dtype=torch.float16,
                                     plan=F.build_conv_plan(cfg, cd, nbr),
                                     packed_weight=F.pack_conv_weight(cfg, wd))
    exp = oracle.conv_gemm_f64(oracle.OracleConfig(cin, cout, *kernel), w, b, x, nbr.cpu().numpy())
    assert_close(host(got), exp, TOL_BF16, f"f16 planned conv, kernel {kernel}, {n} rows")


@pytest.mark.parametrize("cout", [64, 128])
def test_f16_planned_overflow_tiles(oracle, cout):
    """The f16 tile with some tiles over the halo budget (cluster centres
    whose 26 neighbours are all distinct): those tiles gather their operands
    from global memory in the same launch; every row against the fp64
    definition, both tile widths."""
    side = 7
    g = np.stack(np.meshgrid(*[np.arange(side)] * 3, indexing="ij"), -1).reshape(-1, 3)[:300]
    centres = 200 + 3 * g
    offs = np.stack(np.meshgrid(*[np.arange(-1, 2)] * 3, indexing="ij"), -1).reshape(-1, 3)
    offs = offs[np.any(offs != 0, axis=1)]
    nb = (centres[:, None, :] + offs[None]).reshape(-1, 3)
    shell = synth.config1_coords()[:3000]
    xyz = np.concatenate([centres, nb])
    cl = np.concatenate([np.zeros((len(xyz), 1), np.int32), xyz.astype(np.int32)], 1)
    coords = np.ascontiguousarray(np.concatenate([shell, cl[:300], cl[300:]]))
    q = 3300
    rng = np.random.default_rng(cout + 5)
    cin = 64
    x = _fence(oracle, synth.normal_f32(rng, (len(coords), cin)))
    w = _fence(oracle, synth.conv_weight(rng, cout, 27, cin, 1 / np.sqrt(27 * cin)))
    b = synth.normal_f32(rng, cout, 0.1)
    cfg = F.SparseSubmConvConfig(cin, cout)
    cd = dev(coords)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd, query_rows=q)
    plan = F.build_conv_plan(cfg, cd, nbr)
    h = plan.to_host()
    assert 0 < h["n_overflow"] < h["n_tiles"]
    wd = f16_dev(w)
    got = F.sparse_subm_conv_forward(cfg, f16_dev(x), nbr, wd, dev(b), out_dtype=torch.float32,
                                     plan=plan, packed_weight=F.pack_conv_weight(cfg, wd))
    exp = oracle.conv_gemm_f64(oracle.OracleConfig(cin, cout), w, b, x, nbr.cpu().numpy())
    assert_close(host(got), exp, 2e-5, f"f16 planned conv with overflow tiles, Cout {cout}")


def test_config2_conv_f16_planned(oracle):
    """Config 2's shape (113,857 voxels, C = 256) in f16 through the planned
    conv, 2,000 sampled rows (first / last / overflow tiles included)."""
    coords = synth.config2_coords()
    rng = np.random.default_rng(162)
    C = 256
    x = _fence(oracle, synth.normal_f32(rng, (len(coords), C)))
    w = _fence(oracle, synth.conv_weight(rng, C, 27, C, 1 / np.sqrt(27 * C)))
    b = np.zeros(C, np.float32)
    cfg = F.SparseSubmConvConfig(C, C)
    cd = dev(coords)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd)
    plan = F.build_conv_plan(cfg, cd, nbr)
    wd = f16_dev(w)
    got = F.sparse_subm_conv_forward(cfg, f16_dev(x), nbr, wd, dev(b), plan=plan,
                                     packed_weight=F.pack_conv_weight(cfg, wd))
    rows = sample_rows(len(coords), rng, 2000, plan=plan)
    n = nbr.cpu().numpy()
    exp = oracle.conv_gemm_f64(oracle.OracleConfig(C, C), w, b, x, n[rows])
    assert_close(host(got)[rows], exp, TOL_BF16, "config 2 f16 planned conv")


def test_config3_residual_block_f16(oracle):
    """Config 3's block (1,040,679 voxels, C = 128) in f16: map + plan + conv ->
    LN -> SiLU (fused) -> conv + x (fused), against the reference's
    compute_fp16 chain (an f16 fence after conv1, LayerNorm, SiLU, conv2 and
    the residual add) at 3,000 sampled rows."""
    coords = synth.config3_coords()
    n = len(coords)
    rng = np.random.default_rng(163)
    C = 128
    x = _fence(oracle, synth.normal_f32(rng, (n, C)))
    std = 1 / np.sqrt(27 * C)
    w1 = _fence(oracle, synth.conv_weight(rng, C, 27, C, std))
    w2 = _fence(oracle, synth.conv_weight(rng, C, 27, C, std))
    b = np.zeros(C, np.float32)
    cfg = F.SparseSubmConvConfig(C, C)
    cd = dev(coords)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd)
    plan = F.build_conv_plan(cfg, cd, nbr)
    xd, w1d, w2d = f16_dev(x), f16_dev(w1), f16_dev(w2)
    h = F.sparse_subm_conv_forward(cfg, xd, nbr, w1d, dev(b), layer_norm=True, silu=True, ln_eps=1e-6,
                                   plan=plan, packed_weight=F.pack_conv_weight(cfg, w1d))
    y = F.sparse_subm_conv_forward(cfg, h, nbr, w2d, dev(b), residual=xd, plan=plan,
                                   packed_weight=F.pack_conv_weight(cfg, w2d))
    assert h.dtype == torch.float16 and y.dtype == torch.float16
    rows = sample_rows(n, rng, 3000, plan=plan)
    m = nbr.cpu().numpy()
    r1 = np.unique(m[rows][m[rows] >= 0])
    oc = oracle.OracleConfig(C, C)
    c1 = _fence(oracle, oracle.conv_gemm_f64(oc, w1, b, x, m[r1]))
    hh = _fence(oracle, oracle.silu(_fence(oracle, oracle.layer_norm(c1, None, None, 1e-6))))
    loc = np.where(m[rows] >= 0, np.searchsorted(r1, np.maximum(m[rows], 0)), -1)
    c2 = _fence(oracle, oracle.conv_gemm_f64(oc, w2, b, hh, loc))
    exp = _fence(oracle, c2 + x[rows])
    assert_close(host(h)[r1], hh, TOL_BF16, "config 3 f16 conv1 -> LN -> SiLU")
    e = assert_close(host(y)[rows], exp, TOL_BF16, "config 3 f16 residual block")
    assert e <= 5e-3, e


@pytest.mark.parametrize("cout", [256, 96])
def test_f16_wide_and_narrow_layer_norm(oracle, cout):
    """conv -> LN -> SiLU with an f16 output: over 256 channels on the f32
    staging (row kernel), over 96 in the tile epilogue."""
    coords = synth.config1_coords()[:6000]
    rng = np.random.default_rng(cout)
    cin = 64
    x = _fence(oracle, synth.normal_f32(rng, (len(coords), cin)))
    w = _fence(oracle, synth.conv_weight(rng, cout, 27, cin, 1 / np.sqrt(27 * cin)))
    b = synth.normal_f32(rng, cout, 2.0)
    cfg = F.SparseSubmConvConfig(cin, cout)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, dev(coords))
    got = F.sparse_subm_conv_forward(cfg, f16_dev(x), nbr, f16_dev(w), dev(b), layer_norm=True, silu=True)
    conv = oracle.conv_gemm_f64(oracle.OracleConfig(cin, cout), w, b, x, nbr.cpu().numpy()).astype(np.float32)
    exp = oracle.silu(oracle.layer_norm(conv, None, None, 1e-6))
    assert_close(host(got), exp, TOL_BF16, f"f16 LN over {cout}")
    assert rel_err(host(got), exp) <= 2e-3


def test_f16_child_scatter_ln(oracle):
    """The C2S conv1 child scatter in f16 (64-channel children: LayerNorm per
    wave half of the tile)."""
    coords = synth.config1_coords()[:5000]
    rng = np.random.default_rng(64)
    mask = (rng.random((len(coords), 8)) < 0.5).astype(np.uint8)
    cin, cc = 64, 64
    x = _fence(oracle, synth.normal_f32(rng, (len(coords), cin)))
    w = _fence(oracle, synth.conv_weight(rng, 8 * cc, 27, cin, 1 / np.sqrt(27 * cin)))
    b = synth.normal_f32(rng, 8 * cc, 0.5)
    cfg = F.SparseSubmConvConfig(cin, 8 * cc)
    cd = dev(coords)
    ccoords, li, rows = F.subdivision_build_indexed(cd, mask=dev(mask))
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd)
    wd = f16_dev(w)
    got = F.sparse_subm_conv_forward(cfg, f16_dev(x), nbr, wd, dev(b), layer_norm=True, silu=True,
                                     child_rows=rows, n_child_rows=ccoords.shape[0],
                                     plan=F.build_conv_plan(cfg, cd, nbr), packed_weight=F.pack_conv_weight(cfg, wd))
    conv = oracle.conv_gemm_f64(oracle.OracleConfig(cin, 8 * cc), w, b, x, nbr.cpu().numpy())
    lin = li.cpu().numpy()
    sl = conv.reshape(len(coords), 8, cc)[lin // 8, lin % 8].astype(np.float32)
    exp = oracle.silu(oracle.layer_norm(sl, None, None, 1e-6))
    assert_close(host(got), exp, TOL_BF16, "f16 child scatter")

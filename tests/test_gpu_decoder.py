"""GPU tests of the decoder-shaped paths at the BASELINE configs' full sizes:
config 5 (the int8 decoder stack: 3 stages of 2 residual blocks + C2S
upsample, 512 -> 64 channels, ~54k -> 3.6M voxels), config 4 (2x2x2
transposed upsample of the config-2 shell at 512 channels, then a 3x3x3
conv at 256^3 and 256 channels) and config 2 (a 3x3x3 conv at 256 channels),
all through the planned (halo-staged) conv.

Parity is checked on sampled output rows against the oracle in fp64
(tests/tolerance.py: bf16 activations 1e-2 relative to max(|b|, rms(b))),
fed the device's own inputs to the block under test and rounding to bf16
where the device stores bf16; coords and child order are checked exactly."""
import numpy as np
import pytest
import torch

from bevy_synth_amd import decoder as D
from bevy_synth_amd import flex_gmm as F
from bevy_synth_amd import synth
from tests.c2s_check import check_up_fused
from tests.sampling import sample_rows
from tests.tolerance import TOL_BF16, assert_close

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host_f32(t):
    return t.float().cpu().numpy()


def conv_rows(oracle, cfg, w, b, x, nbr_rows, w_scale=None):
    """Oracle conv (fp64) at the rows whose map rows are ``nbr_rows`` [R, K],
    reading input rows from ``x`` (a function of row indices -> f32 rows);
    int8 weights as q (f32) with per-output-channel ``w_scale``."""
    need = np.unique(nbr_rows[nbr_rows >= 0])
    local = np.full(nbr_rows.shape, -1, np.int32)
    pos = np.searchsorted(need, nbr_rows[nbr_rows >= 0])
    local[nbr_rows >= 0] = pos
    xin = x(need) if len(need) else np.zeros((0, cfg.in_channels), np.float32)
    oc = oracle.OracleConfig(cfg.in_channels, cfg.out_channels)
    return oracle.conv_gemm_f64(oc, w, b, xin, local, w_scale)


def qw(layer):
    """(q as f32, scales) of an int8 ConvLayer."""
    return layer.weight.cpu().numpy().astype(np.float32), layer.w_scale.cpu().numpy()


def check_block(oracle, blk, nb, x_dev, y_dev, rows):
    """ResidualBlock at sampled rows: conv1 -> LN -> SiLU (bf16) -> conv2 + x."""
    r = oracle.bf16_round
    nbr = nb.nbr
    n1 = nbr[dev(rows.astype(np.int64))].cpu().numpy()
    r1 = np.unique(n1[n1 >= 0])                       # rows whose h conv2 reads
    n2 = nbr[dev(r1.astype(np.int64))].cpu().numpy()
    (q1, s1), (q2, s2) = qw(blk.conv1), qw(blk.conv2)
    b1, b2 = blk.conv1.bias.cpu().numpy(), blk.conv2.bias.cpu().numpy()
    xget = lambda idx: host_f32(x_dev[dev(idx.astype(np.int64))])
    h1 = conv_rows(oracle, blk.conv1.cfg, q1, b1, xget, n2, s1)
    h = r(oracle.silu(oracle.layer_norm(h1.astype(np.float32), None, None, 1e-6)))
    hget = lambda idx: h[np.searchsorted(r1, idx)]
    y = conv_rows(oracle, blk.conv2.cfg, q2, b2, hget, n1, s2) + xget(rows)
    assert_close(host_f32(y_dev[dev(rows.astype(np.int64))]), y, TOL_BF16, "residual block")


@pytest.fixture(scope="module")
def config5_run():
    """Config 5's stack run once: (stack, masks, final Neighborhood, output,
    trace of every residual block and upsample)."""
    coords, masks = synth.config5_stack_inputs()
    rng = np.random.default_rng(55)
    stack = D.int8_stack([512, 256, 128, 64], 2, seed=5)
    x = dev(synth.bf16_bits(synth.normal_f32(rng, (len(coords), 512))).view(np.int16)).view(torch.bfloat16)
    trace = []
    nb, y = stack(dev(coords), x, [dev(m) for m in masks], trace=trace)
    torch.cuda.synchronize()
    return coords, stack, masks, nb, y, trace


def test_config5_int8_decoder_stack(config5_run):
    coords, stack, masks, nb, y, trace = config5_run
    # coords of every stage: the argwhere-order expansion, exactly
    want = coords
    for m in masks:
        want = synth.child_expand(want, m)
    assert np.array_equal(nb.coords.cpu().numpy(), want)
    assert y.shape == (len(want), 64) and bool(torch.isfinite(y.float()).all())
    assert len(trace) == 9 and all(e[2].plan is not None for e in trace), "every resolution got a conv plan"


def test_stack_stage_without_children():
    """A stack whose first upsample activates no child: the next stage's
    residual blocks, map, plan and upsample all run on zero rows and the
    stack returns [0, C] features and [0, 4] coords."""
    coords = np.ascontiguousarray(synth.config1_coords()[:3000])
    rng = np.random.default_rng(77)
    stack = D.int8_stack([64, 64, 32], 1, seed=7)
    x = dev(synth.bf16_bits(synth.normal_f32(rng, (len(coords), 64))).view(np.int16)).view(torch.bfloat16)
    masks = [dev(np.zeros((len(coords), 8), np.uint8)), dev(np.zeros((0, 8), np.uint8))]
    trace = []
    nb, y = stack(dev(coords), x, masks, trace=trace)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (0, 32) and tuple(nb.coords.shape) == (0, 4)
    assert [e[1] for e in trace] == ["block", "up", "block", "up"]
    assert tuple(trace[2][4].shape) == (0, 64)  # the second stage's residual block output


@pytest.mark.parametrize("idx", range(9))
def test_config5_layer_parity(oracle, config5_run, idx):
    """Each residual block and fused upsample of the config-5 stack at 2,000
    sampled output rows (first, last and overflow tiles included) against the
    oracle chain fed the device's own block input."""
    coords, stack, masks, nb, y, trace = config5_run
    s, kind, nb_in, x_in, y_out, extra = trace[idx]
    rng = np.random.default_rng(500 + idx)
    if kind == "block":
        rows = sample_rows(y_out.shape[0], rng, 2000, plan=nb_in.plan)
        check_block(oracle, extra, nb_in, x_in, y_out, rows)
    else:
        pairs = np.argwhere(masks[s])
        rows = sample_rows(y_out.shape[0], rng, 2000, plan=extra.plan)
        check_up_fused(oracle, stack.stages[s].up, nb_in, x_in, y_out, extra, pairs, rows)


def test_config4_transposed_upsample_and_conv(oracle):
    """Config 4: the config-2 shell (512 channels) -> 2x2x2 transposed conv to
    256 channels on the near-surface children -> 3x3x3 conv at 256^3."""
    g = synth.ShellCubeGeometry()
    parents = g.coords()
    mask = synth.subdivision_mask_near_surface(parents, g)
    rng = np.random.default_rng(44)
    cin, cout = 512, 256
    r = oracle.bf16_round
    x = r(synth.normal_f32(rng, (len(parents), cin)))
    wt = r(synth.normal_f32(rng, (8 * cout, 1, cin), 1 / np.sqrt(8 * cin)))
    w2 = r(synth.conv_weight(rng, cout, 27, cout, 1 / np.sqrt(27 * cout)))
    b0 = np.zeros(8 * cout, np.float32)
    b2 = np.zeros(cout, np.float32)
    bf = lambda a: dev(synth.bf16_bits(a).view(np.int16)).view(torch.bfloat16)
    tcfg = F.SparseSubmConvConfig(cin, 8 * cout, 1, 1, 1)
    cc, feats, li = D.transposed_upsample(dev(parents), bf(x), D.ConvLayer(tcfg, bf(wt), dev(b0)),
                                          dev(mask))
    assert np.array_equal(cc.cpu().numpy(), synth.child_expand(parents, mask))
    ccfg = F.SparseSubmConvConfig(cout, cout)
    nb = D.Neighborhood.build(ccfg, cc)
    assert nb.plan is not None
    y = D.ConvLayer(ccfg, bf(w2), dev(b2))(feats, nb)
    torch.cuda.synchronize()
    n = len(cc)
    rows = sample_rows(n, rng, 2000, plan=nb.plan)
    lin = li.cpu().numpy()
    # the transposed conv at sampled children (a 1x1x1 conv of the parent)
    got_t = host_f32(feats[dev(rows.astype(np.int64))])
    par, c = lin[rows] // 8, lin[rows] % 8
    wc = wt[:, 0, :].reshape(8, cout, cin).astype(np.float64)
    exp_t = np.zeros((len(rows), cout))
    for ci in range(8):
        sel = c == ci
        exp_t[sel] = x[par[sel]].astype(np.float64) @ wc[ci].T
    assert_close(got_t, exp_t, TOL_BF16, "config 4 transposed conv")
    # the 3x3x3 conv at sampled children, on the device's bf16 children
    nbr_rows = nb.nbr[dev(rows.astype(np.int64))].cpu().numpy()
    exp = conv_rows(oracle, ccfg, w2, b2, lambda idx: host_f32(feats[dev(idx.astype(np.int64))]), nbr_rows)
    assert_close(host_f32(y[dev(rows.astype(np.int64))]), exp, TOL_BF16, "config 4 conv")


def test_config2_conv_planned(oracle):
    """Config 2: 3x3x3 conv, 256 channels, bf16, on the ~120k-voxel shell+cube."""
    coords = synth.config2_coords()
    rng = np.random.default_rng(22)
    C = 256
    r = oracle.bf16_round
    x = r(synth.normal_f32(rng, (len(coords), C)))
    w = r(synth.conv_weight(rng, C, 27, C, 1 / np.sqrt(27 * C)))
    b = np.zeros(C, np.float32)
    bf = lambda a: dev(synth.bf16_bits(a).view(np.int16)).view(torch.bfloat16)
    cfg = F.SparseSubmConvConfig(C, C)
    nb = D.Neighborhood.build(cfg, dev(coords))
    layer = D.ConvLayer(cfg, bf(w), dev(b))
    y = layer(bf(x), nb)
    y_direct = layer(bf(x), nb.nbr)       # unplanned direct-gather kernel
    torch.cuda.synchronize()
    rows = sample_rows(len(coords), rng, 2000, plan=nb.plan)
    nbr_rows = nb.nbr[dev(rows.astype(np.int64))].cpu().numpy()
    exp = conv_rows(oracle, cfg, w, b, lambda idx: x[idx], nbr_rows)
    assert_close(host_f32(y[dev(rows.astype(np.int64))]), exp, TOL_BF16, "config 2 planned conv")
    a, d = y.float(), y_direct.float()
    assert float((a - d).abs().max()) <= 2 ** -5 * float(d.abs().max())

"""GPU parity of the fused C2S upsample pieces: the indexed subdivision (the
inverse of linear_idx), the to_subdiv skinny linear, conv1's child scatter
with the per-child LayerNorm -> SiLU in its epilogue, conv2's parent skip in
its epilogue, and the whole fused block against the oracle at the config-4
parent set (113,857 parents at 512 channels -> 256-channel children).

References: the fp64 conv definition (oracle.conv_gemm_f64, pinned to
conv_ref_f64), the oracle's LayerNorm / SiLU / repeat-interleave skip, and
numpy's argwhere order.  bf16 tolerance 1e-2 (tests/tolerance.py)."""
import numpy as np
import pytest
import torch

from bevy_synth_amd import decoder as D
from bevy_synth_amd import flex_gmm as F
from bevy_synth_amd import synth
from tests.c2s_check import check_up_fused
from tests.sampling import sample_rows
from tests.tolerance import TOL_BF16, TOL_F32, assert_close

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bf16_dev(x_f32):
    return dev(synth.bf16_bits(x_f32).view(np.int16)).view(torch.bfloat16)


def rbf(x):
    return synth.bf16_to_f32(synth.bf16_bits(np.asarray(x, np.float32)))


def host(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("round_f16,center", [(True, False), (False, True), (True, True), (False, False)])
def test_subdivision_logits_finish(oracle, round_f16, center):
    """The to_subdiv logits' post-processing in place, bit for bit: f16
    rounding (the reference's quantize_f16 under compute_fp16; here against
    the oracle's f16 rounding) and row centering (row_center_logits: the f32
    sum in child order / 8, subtracted)."""
    rng = np.random.default_rng(5 + 2 * round_f16 + center)
    lg = (rng.standard_normal((70001, 8)) * 4).astype(np.float32)
    lg[0] = [70000.0, -70000.0, 1e-8, -1e-8, 0.0, -0.0, 65504.0, 65520.0]  # f16 overflow / underflow edges
    t = dev(lg)
    F.subdivision_logits_finish(t, round_f16=round_f16, center=center)
    exp = oracle.f16_round(lg) if round_f16 else lg.copy()
    if center:
        s = np.zeros(len(exp), np.float32)
        for c in range(8):
            s = (s + exp[:, c]).astype(np.float32)
        exp = (exp - (s / np.float32(8))[:, None]).astype(np.float32)
    got = t.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)) or \
        np.array_equal(np.isnan(got), np.isnan(exp)) and np.array_equal(got[~np.isnan(got)], exp[~np.isnan(exp)])


def test_c2s_f16_logits_pick_children(oracle):
    """compute_fp16: the block's to_subdiv logits are rounded to f16 before
    the threshold test, so a logit that is positive in f32 but below f16's
    smallest subnormal picks no child (the reference rounds, then compares)."""
    P, C = 3000, 64
    rng = np.random.default_rng(31)
    x = synth.normal_f32(rng, (P, C)).astype(np.float16)
    w = np.zeros((8, C), np.float32)
    b = np.array([1e-9, -1e-9, 0.5, -0.5, 1e-3, 70000.0, 2.0 ** -25, 2.0 ** -24], np.float32)
    up = D.C2SUpsampleBlock(C, C, dev(np.ones(C, np.float32)), dev(np.zeros(C, np.float32)), None, None,
                            to_subdiv_weight=dev(w), to_subdiv_bias=dev(b), compute_fp16=True)
    lg = up.subdivision_logits(dev(x)).cpu().numpy()
    exp = np.broadcast_to(oracle.f16_round(b), (P, 8))
    assert np.array_equal(lg.view(np.uint32), exp.view(np.uint32))
    assert np.array_equal(lg[0] > 0, [False, False, True, False, True, True, False, True])


@pytest.mark.parametrize("P", [1, 1023, 1025, 70001])
def test_subdivision_indexed_child_rows(P):
    rng = np.random.default_rng(P)
    parents = np.zeros((P, 4), np.int32)
    parents[:, 1:] = rng.integers(0, 300, (P, 3))
    mask = (rng.random((P, 8)) < 0.4).astype(np.uint8)
    cc, li, rows = F.subdivision_build_indexed(dev(parents), mask=dev(mask))
    cc0, li0, _ = F.subdivision_build(dev(parents), mask=dev(mask))
    assert torch.equal(cc, cc0) and torch.equal(li, li0)
    pairs = np.argwhere(mask)
    exp = np.full((P, 8), -1, np.int32)
    exp[pairs[:, 0], pairs[:, 1]] = np.arange(len(pairs), dtype=np.int32)
    assert np.array_equal(rows.cpu().numpy(), exp)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("cin,cout", [(512, 8), (64, 3), (100, 8)])
def test_linear_skinny(dtype, cin, cout):
    rng = np.random.default_rng(cin * cout)
    rows = 70001
    x = synth.normal_f32(rng, (rows, cin))
    if dtype == torch.bfloat16:
        x = rbf(x)
    w = synth.normal_f32(rng, (cout, cin), 1 / np.sqrt(cin))
    b = synth.normal_f32(rng, cout)
    xd = bf16_dev(x) if dtype == torch.bfloat16 else dev(x)
    got = F.linear_skinny(xd, dev(w), dev(b)).cpu().numpy()
    exp = x.astype(np.float64) @ w.T.astype(np.float64) + b
    assert_close(got, exp, TOL_F32, "skinny linear")


def _parents_and_mask(n=6000, frac=0.45, seed=3):
    coords = synth.config1_coords()[:n]
    rng = np.random.default_rng(seed)
    mask = (rng.random((len(coords), 8)) < frac).astype(np.uint8)
    return coords, mask


@pytest.mark.parametrize("cchild,ln", [(16, True), (64, True), (128, True), (256, True), (64, False),
                                       (24, True), (96, False)])
@pytest.mark.parametrize("planned", [False, True])
def test_conv1_child_scatter(oracle, cchild, ln, planned):
    """conv1 (Cin -> 8*C) on the parents writes child c of parent p to row
    child_rows[p, c], normalised over its C channels: in the tile epilogue
    (C = 64: one wave half; C = 128: the tile) or on f32 staging (C = 16, 24,
    256); C = 24 and 96 take the epilogue's division form (C not a power of
    two)."""
    coords, mask = _parents_and_mask()
    rng = np.random.default_rng(cchild)
    cin, cout = 64, 8 * cchild
    x = rbf(synth.normal_f32(rng, (len(coords), cin)))
    w = rbf(synth.conv_weight(rng, cout, 27, cin, 1 / np.sqrt(27 * cin)))
    b = synth.normal_f32(rng, cout, 0.5)
    cfg = F.SparseSubmConvConfig(cin, cout)
    cd = dev(coords)
    cc, li, rows = F.subdivision_build_indexed(cd, mask=dev(mask))
    A = cc.shape[0]
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd)
    wd = bf16_dev(w)
    kw = {}
    if planned:
        kw = dict(plan=F.build_conv_plan(cfg, cd, nbr), packed_weight=F.pack_conv_weight(cfg, wd))
    got = F.sparse_subm_conv_forward(cfg, bf16_dev(x), nbr, wd, dev(b), layer_norm=ln, silu=ln,
                                     child_rows=rows, n_child_rows=A, **kw)
    assert tuple(got.shape) == (A, cchild)
    conv = oracle.conv_gemm_f64(oracle.OracleConfig(cin, cout), w, b, x, nbr.cpu().numpy())
    lin = li.cpu().numpy()
    sl = conv.reshape(len(coords), 8, cchild)[lin // 8, lin % 8].astype(np.float32)
    exp = oracle.silu(oracle.layer_norm(sl, None, None, 1e-6)) if ln else sl
    assert_close(host(got), exp, TOL_BF16, f"child scatter C={cchild}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("cin,cchild,ln", [(512, 256, False), (64, 64, True), (96, 128, True), (64, 256, True),
                                           (32, 24, False)])
def test_linear_child_scatter(oracle, dtype, cin, cchild, ln):
    """The 2x2x2 transposed upsample's linear form (sc_linear_forward with
    child_rows): row p's slice c of x W^T + b lands in row child_rows[p, c],
    normalised over its C channels with a [C] affine when asked (C = 64 and
    128 in the dense tile's epilogue for bf16 / f16, else on f32 staging)."""
    coords, mask = _parents_and_mask(n=5000, frac=0.45, seed=cin + cchild)
    rng = np.random.default_rng(cin * cchild)
    cout = 8 * cchild
    rnd = {torch.bfloat16: oracle.bf16_round, torch.float16: oracle.f16_round,
           torch.float32: lambda a: np.asarray(a, np.float32)}[dtype]
    x = rnd(synth.normal_f32(rng, (len(coords), cin)))
    w = rnd(synth.normal_f32(rng, (cout, cin), 1 / np.sqrt(cin)))
    b = synth.normal_f32(rng, cout, 0.5)
    lw = synth.normal_f32(rng, cchild) if ln else None
    lb = synth.normal_f32(rng, cchild) if ln else None
    cc, li, rows = F.subdivision_build_indexed(dev(coords), mask=dev(mask))
    A = cc.shape[0]
    got = F.linear_forward(dev(x).to(dtype), dev(w).to(dtype), dev(b), layer_norm=ln,
                           ln_weight=None if lw is None else dev(lw), ln_bias=None if lb is None else dev(lb),
                           child_rows=rows, n_child_rows=A)
    assert tuple(got.shape) == (A, cchild) and got.dtype == dtype
    dense = x.astype(np.float64) @ w.T.astype(np.float64) + b
    lin = li.cpu().numpy()
    sl = dense.reshape(len(coords), 8, cchild)[lin // 8, lin % 8].astype(np.float32)
    exp = oracle.layer_norm(sl, lw, lb, 1e-6) if ln else sl
    tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
    assert_close(host(got), exp, tol, f"linear child scatter {cin}->8x{cchild}")


@pytest.mark.parametrize("cp,cout", [(512, 256), (128, 64), (64, 128), (256, 32), (128, 32), (256, 96)])
def test_conv2_parent_skip(oracle, cp, cout):
    """conv2 on the children + the channel-repeated parent skip in its epilogue
    (S = Cp/8 parent channels per child, each repeated R = Cout/S times):
    R = 4, 4, 16 (one parent load per 4 channels), R = 1, 2 (a load per
    channel) and R = 3 (the division form)."""
    coords, mask = _parents_and_mask(3000, 0.5, seed=cp)
    rng = np.random.default_rng(cp + cout)
    cd = dev(coords)
    cc, li, _ = F.subdivision_build(cd, mask=dev(mask), with_pairs=False)
    A = cc.shape[0]
    cfg = F.SparseSubmConvConfig(cout, cout)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cc)
    h = rbf(synth.normal_f32(rng, (A, cout)))
    w = rbf(synth.conv_weight(rng, cout, 27, cout, 1 / np.sqrt(27 * cout)))
    b = synth.normal_f32(rng, cout, 0.1)
    parent = rbf(synth.normal_f32(rng, (len(coords), cp)))
    wd = bf16_dev(w)
    plan = F.build_conv_plan(cfg, cc, nbr)
    got = F.sparse_subm_conv_forward(cfg, bf16_dev(h), nbr, wd, dev(b), skip_parent=bf16_dev(parent),
                                     skip_index=li, plan=plan, packed_weight=F.pack_conv_weight(cfg, wd))
    lin = li.cpu().numpy()
    S = cp // 8
    skip = parent.reshape(len(coords), 8, S)[lin // 8, lin % 8]
    exp = oracle.conv_gemm_f64(oracle.OracleConfig(cout, cout), w, b, h, nbr.cpu().numpy()) + \
        oracle.repeat_interleave(skip, cout // S)
    assert_close(host(got), exp, TOL_BF16, "conv + parent skip")


def test_linear_child_scatter_no_active_child():
    """The dense linear's child scatter with no active child (a transposed
    upsample whose mask is all zero) returns an empty [0, C] output."""
    coords, _ = _parents_and_mask(n=500, seed=9)
    rng = np.random.default_rng(9)
    cin, cchild = 64, 32
    x = rbf(synth.normal_f32(rng, (len(coords), cin)))
    w = rbf(synth.normal_f32(rng, (8 * cchild, cin), 1 / np.sqrt(cin)))
    cc, _, rows = F.subdivision_build_indexed(dev(coords), mask=dev(np.zeros((len(coords), 8), np.uint8)))
    assert cc.shape[0] == 0
    got = F.linear_forward(bf16_dev(x), bf16_dev(w), dev(synth.normal_f32(rng, 8 * cchild)),
                           child_rows=rows, n_child_rows=0)
    assert tuple(got.shape) == (0, cchild)


@pytest.mark.parametrize("which", ["none", "one", "all"])
@pytest.mark.parametrize("cout", [64, 128])
def test_c2s_block_degenerate_masks(which, cout):
    """The fused block with no active child (the children's map, plan and
    conv2 run on zero rows), one active child, and every child active,
    against the reference's unfused composition within 2^-5."""
    coords, _ = _parents_and_mask(n=700, seed=5)
    rng = np.random.default_rng(cout + len(which))
    P, cin = len(coords), 64
    mask = np.zeros((P, 8), np.uint8)
    if which == "one":
        mask[P // 2, 5] = 1
    elif which == "all":
        mask[:] = 1

    def layer(ci, co):
        w = rbf(synth.conv_weight(rng, co, 27, ci, 1 / np.sqrt(27 * ci)))
        return D.ConvLayer(F.SparseSubmConvConfig(ci, co), bf16_dev(w), dev(synth.normal_f32(rng, co, 0.1)))
    up = D.C2SUpsampleBlock(cin, cout, dev((1 + 0.1 * rng.standard_normal(cin)).astype(np.float32)),
                            dev((0.1 * rng.standard_normal(cin)).astype(np.float32)),
                            layer(cin, 8 * cout), layer(cout, cout))
    pnb = D.Neighborhood.build(up.conv1.cfg, dev(coords))
    x = bf16_dev(synth.normal_f32(rng, (P, cin)))
    md = dev(mask)
    cnb, y = up.forward(pnb, x, mask=md)
    A = int(mask.sum())
    assert tuple(y.shape) == (A, cout) and tuple(cnb.coords.shape) == (A, 4)
    assert np.array_equal(cnb.coords.cpu().numpy(), synth.child_expand(coords, mask).reshape(-1, 4))
    up.fused = False
    _, y_ref = up.forward(pnb, x, mask=md)
    assert tuple(y_ref.shape) == (A, cout)
    if A:
        d = (y.float() - y_ref.float()).abs().max().item()
        assert d <= 2 ** -5 * max(1.0, y_ref.float().abs().max().item()), d


def test_c2s_block_fused_config4_parents(oracle):
    """The fused block on config 4's parent set (the config-2 shell + cube,
    113,857 parents at 512 channels, near-surface children at 256 channels):
    to_subdiv logits, indexed subdivision, conv1 scatter with per-child LN
    (256 channels: f32 staging), conv2 + parent skip; 2,000 sampled children
    (first / last / overflow tiles included) against the oracle chain, the
    child coords against numpy, and the unfused composition within 2^-5."""
    g = synth.ShellCubeGeometry()
    parents = g.coords()
    rng = np.random.default_rng(404)
    cin, cout = 512, 256
    P = len(parents)
    x = bf16_dev(synth.normal_f32(rng, (P, cin)))

    def layer(ci, co):
        w = rbf(synth.conv_weight(rng, co, 27, ci, 1 / np.sqrt(27 * ci)))
        return D.ConvLayer(F.SparseSubmConvConfig(ci, co), bf16_dev(w), dev(synth.normal_f32(rng, co, 0.1)))
    up = D.C2SUpsampleBlock(cin, cout, dev((1 + 0.1 * rng.standard_normal(cin)).astype(np.float32)),
                            dev((0.1 * rng.standard_normal(cin)).astype(np.float32)),
                            layer(cin, 8 * cout), layer(cout, cout),
                            to_subdiv_weight=dev(synth.normal_f32(rng, (8, cin), 1 / np.sqrt(cin))),
                            to_subdiv_bias=dev(np.full(8, 0.3, np.float32)))
    pnb = D.Neighborhood.build(up.conv1.cfg, dev(parents))
    logits = up.subdivision_logits(x)
    cnb, y = up.forward(pnb, x, logits=logits)
    lg = logits.cpu().numpy()
    mask = lg > 0
    pairs = np.argwhere(mask)
    assert 0 < len(pairs) < 8 * P
    assert np.array_equal(cnb.coords.cpu().numpy(), synth.child_expand(parents, mask.astype(np.uint8)))
    rows = sample_rows(len(pairs), rng, 2000, plan=cnb.plan)
    check_up_fused(oracle, up, pnb, x, y, cnb, pairs, rows)
    up.fused = False
    _, y_ref = up.forward(pnb, x, logits=logits)
    d = (y.float() - y_ref.float()).abs().max().item()
    assert d <= 2 ** -5 * max(1.0, y_ref.float().abs().max().item()), d


def _c2s_parents(n=None):
    parents = synth.ShellCubeGeometry().coords()
    return parents if n is None else parents[:n]


@pytest.mark.parametrize("frac", [0.5, 0.0, 1.0])
def test_child_plan_lists(frac):
    """sc_conv_child_plan_build: per child index, the parents whose child is
    active, in the parent plan's order, tiled from child_base[c]; a tile
    whose halo overflowed has its rows 128..255 in a spare tile of the same
    child (the splits listed in tile order); every other slot is -1; the
    overflow list holds exactly the tiles still over the halo budget, in
    tile order."""
    rng = np.random.default_rng(int(frac * 10) + 3)
    parents = _c2s_parents(50000)
    P = len(parents)
    mask = rng.random((P, 8)) < frac
    cfg = F.SparseSubmConvConfig(128, 512)
    pc = dev(parents)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, pc)
    plan = F.build_conv_plan(cfg, pc, nbr)
    cc, _, child_rows = F.subdivision_build_indexed(pc, mask=dev(mask.astype(np.uint8)))
    A = cc.shape[0]
    cp = F.build_child_plan(cfg, plan, nbr, child_rows, A)
    h, ph = cp.to_host(), plan.to_host()
    n_main = (A + 255) // 256 + 8
    assert h["status"] == 0 and h["grid_mode"] == 4 and h["n_tiles"] == n_main + n_main // 8 + 16
    assert h["list_tiles"] == n_main
    porder = ph["order"].ravel()
    porder = porder[porder >= 0]
    order, tc = h["order"], h["tile_child"]
    spare = {int(t): int(u) for t, u in h["split"]}
    assert list(spare) == sorted(spare) and all(n_main <= u < h["n_tiles"] for u in spare.values())
    assert sorted(spare.values()) == list(range(n_main, n_main + len(spare)))
    base, used = 0, set()
    for c in range(8):
        lst = porder[mask[porder, c]]
        nt = (len(lst) + 255) // 256
        assert h["child_n"][c] == len(lst) and h["child_base"][c] == base, c
        seg = []
        for t in range(base, base + nt):
            assert tc[t] == c
            if t in spare:
                u = spare[t]
                assert tc[u] == c and (order[t][128:] == -1).all() and (order[u][128:] == -1).all()
                seg += [order[t][:128], order[u][:128]]
                used.add(u)
            else:
                seg.append(order[t])
            used.add(t)
        seg = np.concatenate(seg) if seg else np.zeros(0, np.int32)
        assert np.array_equal(seg[:len(lst)], lst), c
        assert (seg[len(lst):] == -1).all(), c
        base += nt
    assert h["n_used"] == base
    rest = np.array(sorted(set(range(h["n_tiles"])) - used), np.int64)
    assert (tc[rest] == -1).all() and (order[rest] == -1).all()
    over = [t for t in range(h["n_tiles"]) if tc[t] >= 0 and h["tile_u"][t] > F.PLAN_HALO_MAX]
    assert h["overflow"].tolist() == over
    print(f"children {A}: list tiles {base}, splits {len(spare)}, overflow after splits {len(over)}")
    F.conv_plan_check(cp)


@pytest.mark.parametrize("cin,cchild,ln", [(128, 64, True), (256, 128, True), (128, 256, True),
                                           (128, 64, False)])
def test_conv1_child_plan_matches_parent_plan(cin, cchild, ln):
    """conv1 of the C2S block through the child plan (only active children
    computed) stores exactly what the parent-plan conv1 (all eight children,
    inactive ones dropped) stores -- the same sum in the same order per value,
    whether a tile stages its halo in LDS or, overflowed, gathers from global
    memory -- with 128-channel tiles, with the per-child LayerNorm in the
    tile (128 channels) or
    through the f32 staging (256).  Children of 64 channels take 64-channel
    tiles in the child plan, whose two waves per row half split the stages
    (another order of the same sum): held to the bf16 bar."""
    rng = np.random.default_rng(cin + cchild + ln)
    parents = _c2s_parents()
    P = len(parents)
    mask = rng.random((P, 8)) < 0.5
    cfg = F.SparseSubmConvConfig(cin, 8 * cchild)
    pc = dev(parents)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, pc)
    nb = D.Neighborhood(pc, nbr, F.build_conv_plan(cfg, pc, nbr))
    cc, _, child_rows = F.subdivision_build_indexed(pc, mask=dev(mask.astype(np.uint8)))
    A = cc.shape[0]
    x = bf16_dev(synth.normal_f32(rng, (P, cin)))
    layer = D.ConvLayer(cfg, bf16_dev(synth.conv_weight(rng, 8 * cchild, 27, cin, 1 / np.sqrt(27 * cin))),
                        dev(synth.normal_f32(rng, 8 * cchild, 0.1)))
    kw = dict(out_dtype=torch.bfloat16, layer_norm=ln, silu=ln, child_rows=child_rows, n_child_rows=A)
    ref = layer(x, nb, **kw)
    cp = F.build_child_plan(cfg, nb.plan, nbr, child_rows, A)
    got = layer(x, D.Neighborhood(pc, nbr, cp), **kw)
    F.conv_plan_check(cp)
    assert got.shape == (A, cchild)
    # Every child is bit-equal between the two plans: a tile whose halo
    # overflows gathers its operands from global memory but sums the same
    # stages in the same order as a halo tile.  (64-channel tiles split their
    # stages between two waves by the tile's offset mask, which differs
    # between the plans: the bf16 bar.)
    cr = child_rows.cpu().numpy()
    ph, ch = nb.plan.to_host(), cp.to_host()
    direct = np.zeros(A, bool)
    for t in ph["overflow"]:
        ps = ph["order"][t]
        r = cr[ps[ps >= 0]].ravel()
        direct[r[r >= 0]] = True
    for t in np.nonzero(ch["tile_u"] > F.PLAN_HALO_MAX)[0]:
        ps = ch["order"][t]
        r = cr[ps[ps >= 0], ch["tile_child"][t]]
        direct[r[r >= 0]] = True
    g, r = got.float().cpu().numpy(), ref.float().cpu().numpy()
    print(f"children {A}, through the direct kernel in either plan: {int(direct.sum())}")
    if cchild == 64:
        assert_close(g, r, TOL_BF16, "64-channel children, stage-split tiles")
        return
    assert np.array_equal(g, r)


def test_child_plan_refuses_inconsistent_child_rows():
    """Child rows naming more active children than the plan was sized for
    (every child of every parent at row 0, with one child declared): the
    build flags the plan and leaves it empty, and a conv on it writes
    nothing."""
    rng = np.random.default_rng(8)
    parents = _c2s_parents(20000)
    P = len(parents)
    cfg = F.SparseSubmConvConfig(128, 512)
    pc = dev(parents)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, pc)
    plan = F.build_conv_plan(cfg, pc, nbr)
    child_rows = torch.zeros((P, 8), dtype=torch.int32, device="cuda")
    cp = F.build_child_plan(cfg, plan, nbr, child_rows, 1)
    with pytest.raises(F.SparseConvError) as e:
        F.conv_plan_check(cp)
    assert e.value.status == 2 and "child plan" in e.value.message
    h = cp.to_host()
    assert (h["tile_child"] == -1).all() and (h["order"] == -1).all()
    x = bf16_dev(synth.normal_f32(rng, (P, 128)))
    layer = D.ConvLayer(cfg, bf16_dev(synth.conv_weight(rng, 512, 27, 128, 0.01)), dev(np.zeros(512, np.float32)))
    out = torch.full((1, 64), 7.0, dtype=torch.bfloat16, device="cuda")
    F.sparse_subm_conv_forward(cfg, x, nbr, layer.weight, layer.bias, out=out, plan=cp,
                               packed_weight=layer.packed_weight(), child_rows=child_rows, n_child_rows=1)
    torch.cuda.synchronize()
    assert (out.float() == 7.0).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cin,cchild,ln,frac", [(512, 256, False, 0.74), (128, 128, True, 0.5),
                                                (256, 256, True, 0.3), (64, 128, False, 1.0)])
def test_linear_child_plan_matches_unplanned(dtype, cin, cchild, ln, frac):
    """The transposed upsample's linear over a linear child plan
    (sc_linear_child_plan_build; only active children computed) stores
    exactly what sc_linear_forward stores (all eight children, inactive ones
    dropped): every value the same sum in the same order, with the per-child
    LayerNorm in the tile (128 channels) or on the f32 staging (256).  The
    plan's lists: per child, the parents in row order, tiled from
    child_base[c]; child index 3 is never active; every other slot is -1."""
    rng = np.random.default_rng(cin + cchild + int(frac * 10))
    parents = _c2s_parents(30001)
    P = len(parents)
    mask = rng.random((P, 8)) < frac
    mask[:, 3] = False
    pc = dev(parents)
    cc, _, child_rows = F.subdivision_build_indexed(pc, mask=dev(mask.astype(np.uint8)))
    A = cc.shape[0]
    x = dev(synth.normal_f32(rng, (P, cin))).to(dtype)
    w = dev(synth.normal_f32(rng, (8 * cchild, cin), 1 / np.sqrt(cin))).to(dtype)
    b = dev(synth.normal_f32(rng, 8 * cchild, 0.5))
    kw = dict(layer_norm=ln, child_rows=child_rows, n_child_rows=A)
    if ln:
        kw.update(ln_weight=dev(synth.normal_f32(rng, cchild)), ln_bias=dev(synth.normal_f32(rng, cchild)))
    ref = F.linear_forward(x, w, b, **kw)
    cp = F.build_linear_child_plan(child_rows, A)
    got = F.linear_forward(x, w, b, child_plan=cp, **kw)
    F.conv_plan_check(cp)
    assert got.shape == (A, cchild) and got.dtype == dtype
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    h = cp.to_host()
    tc, order = h["tile_child"], h["order"]
    base = 0
    for c in range(8):
        lst = np.nonzero(mask[:, c])[0]
        nt = (len(lst) + 255) // 256
        assert h["child_n"][c] == len(lst) and h["child_base"][c] == base, c
        seg = order[base:base + nt].ravel()
        assert np.array_equal(seg[:len(lst)], lst) and (seg[len(lst):] == -1).all(), c
        assert (tc[base:base + nt] == c).all(), c
        base += nt
    assert h["n_used"] == base
    assert (tc[base:] == -1).all() and (order[base:] == -1).all()


def test_linear_child_plan_refusals():
    """The linear child plan takes children of a multiple of 128 channels on
    16-bit weights; a plan built for other parents or children is refused on
    the host."""
    rng = np.random.default_rng(12)
    parents = _c2s_parents(3000)
    P = len(parents)
    mask = rng.random((P, 8)) < 0.5
    cc, _, child_rows = F.subdivision_build_indexed(dev(parents), mask=dev(mask.astype(np.uint8)))
    A = cc.shape[0]
    cp = F.build_linear_child_plan(child_rows, A)
    x = bf16_dev(synth.normal_f32(rng, (P, 64)))
    w64 = bf16_dev(synth.normal_f32(rng, (8 * 64, 64), 0.1))
    with pytest.raises(F.SparseConvError) as e:
        F.linear_forward(x, w64, child_rows=child_rows, n_child_rows=A, child_plan=cp)
    assert "multiple of 128" in e.value.message
    w128 = bf16_dev(synth.normal_f32(rng, (8 * 128, 64), 0.1))
    with pytest.raises(F.SparseConvError):
        F.linear_forward(x[:P - 1], w128, child_rows=child_rows[:P - 1].contiguous(), n_child_rows=A,
                         child_plan=cp)

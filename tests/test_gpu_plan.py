"""GPU tests of the conv plan (sc_conv_plan_build), the weight packing
(sc_conv_weight_pack) and the planned, halo-staged conv
(sc_subm_conv_forward_planned).

The plan is checked structurally against the map it was built from (every
(row, offset) entry resolves to the same input row); the planned conv against
the fp64 definition on the same bf16-rounded operands (1e-2, f32 output 2e-5),
including tiles whose halo overflows the LDS budget and take the direct
kernel."""
import numpy as np
import pytest
import torch

from bevy_synth_amd import flex_gmm as F
from bevy_synth_amd import synth
from tests.sampling import sample_rows
from tests.tolerance import TOL_BF16, assert_close

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bf16_dev(x_f32):
    return dev(synth.bf16_bits(x_f32).view(np.int16)).view(torch.bfloat16)


def rbf(a):
    return synth.bf16_to_f32(synth.bf16_bits(np.asarray(a, np.float32)))


def ocfg(oracle, cfg):
    return oracle.OracleConfig(cfg.in_channels, cfg.out_channels, cfg.kernel_d, cfg.kernel_h,
                               cfg.kernel_w, groups=cfg.groups, axis_order=cfg.axis_order,
                               axis_sign=cfg.axis_sign)


def cluster_coords(n_centres, spacing=3):
    """Centres on a lattice of the given spacing, each followed later by its 26
    neighbours: with the centres as query rows, every neighbour is distinct, so
    a 256-row tile touches 27 * 256 input rows (its halo overflows)."""
    side = int(np.ceil(n_centres ** (1 / 3)))
    g = np.stack(np.meshgrid(*[np.arange(side)] * 3, indexing="ij"), -1).reshape(-1, 3)[:n_centres]
    centres = 1 + spacing * g
    offs = np.stack(np.meshgrid(*[np.arange(-1, 2)] * 3, indexing="ij"), -1).reshape(-1, 3)
    offs = offs[np.any(offs != 0, axis=1)]
    nb = (centres[:, None, :] + offs[None]).reshape(-1, 3)
    xyz = np.concatenate([centres, nb])
    out = np.zeros((len(xyz), 4), np.int32)
    out[:, 1:] = xyz
    return out


def check_plan(plan, nbr, n_in):
    h = plan.to_host()
    n_q, K = nbr.shape
    order, tile_u, halo, lmap = h["order"], h["tile_u"], h["halo"], h["lmap"]
    assert h["n_tiles"] == (n_q + 255) // 256 and h["K"] == K
    flat = order.ravel()
    rows = flat[flat >= 0]
    assert len(rows) == n_q and np.array_equal(np.sort(rows), np.arange(n_q)), "order is not a permutation"
    assert np.all(flat[n_q:] == -1), "padding rows are not at the end"
    over = set(np.nonzero(tile_u > F.PLAN_HALO_MAX)[0].tolist())
    assert over == set(h["overflow"].tolist())
    for t in range(h["n_tiles"]):
        if t in over:
            continue
        U = tile_u[t]
        hl = halo[t, :U]
        assert np.all(np.diff(hl) > 0), "halo not strictly increasing"
        r = order[t]
        valid = r >= 0
        m = nbr[r[valid]]                       # [rows, K]
        lm = lmap[t][:, valid].T                # [rows, K]
        present = (m >= 0) & (m < n_in)
        assert np.all((lm == F.PLAN_ABSENT) == ~present)
        assert np.array_equal(hl[lm[present]], m[present])
        assert len(np.unique(m[present])) == U
    return h


def c2s_children(levels, frac=0.5, seed=4):
    """Children of `levels` C2S subdivisions below config 1's sorted shell,
    in the order the subdivision emits them."""
    rng = np.random.default_rng(seed)
    coords = synth.config1_coords()
    for _ in range(levels):
        coords = synth.child_expand(coords, (rng.random((len(coords), 8)) < frac).astype(np.uint8))
    return coords


@pytest.mark.parametrize("which", ["config1", "random_batches", "clusters", "query_subset", "duplicates",
                                   "wide_bbox", "c2s_3_levels", "c2s_2_levels", "slab"])
def test_plan_structure(which):
    rng = np.random.default_rng(11)
    cfg = F.SparseSubmConvConfig(32, 32)
    q = None
    if which == "config1":
        coords = synth.config1_coords()
    elif which == "random_batches":
        c = rng.integers(0, 40, size=(20000, 4)).astype(np.int32)
        c[:, 0] = rng.integers(0, 3, 20000)
        coords = np.unique(c, axis=0)
        coords = coords[rng.permutation(len(coords))]  # unsorted input order
    elif which == "clusters":
        coords = cluster_coords(600)
        q = 600
    elif which == "duplicates":
        # 3,000 extra rows repeating existing coords, in shuffled order: the
        # plan lists every row once, and the rows of duplicated coords come
        # after the distinct ones in increasing row order (deterministic)
        base = synth.config1_coords()
        coords = np.concatenate([base, base[rng.integers(0, len(base), 3000)]])
        coords = coords[rng.permutation(len(coords))]
    elif which == "wide_bbox":
        # a bounding box far beyond the occupancy grid's budget (16 cells per
        # row): the counting-sort order, with duplicated coords in two batches
        c = rng.integers(0, 1000, size=(20000, 4)).astype(np.int32)
        c[:, 0] = rng.integers(0, 2, 20000)
        c[:4000] = c[4000:8000] + np.array([0, 1, 0, 0], np.int32)       # neighbours in x
        c[-300:] = c[:300]                                               # duplicates
        coords = c[rng.permutation(len(c))]
    elif which == "c2s_3_levels":
        # octree order over 3 levels: the rows keep their own order
        coords = c2s_children(3, frac=0.3)
        q = len(coords) - 1000
    elif which == "c2s_2_levels":
        coords = c2s_children(2)
    elif which == "slab":
        # x-planes of 67,600 rows in (b, x, y, z) order: a tile's x-1 and x+1
        # neighbours lie more than the LDS bitmap's 131,072 rows apart, in a
        # few pages (the paged bitmap); some cells empty
        g = np.stack(np.meshgrid(np.arange(4), np.arange(260), np.arange(260), indexing="ij"), -1).reshape(-1, 3)
        g = g[rng.random(len(g)) < 0.9]
        coords = np.concatenate([np.zeros((len(g), 1), np.int32), g.astype(np.int32)], 1)
    else:
        coords = synth.config1_coords()
        q = 9000
    cd = dev(coords)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd, query_rows=q)
    plan = F.build_conv_plan(cfg, cd, nbr)
    h = check_plan(plan, nbr.cpu().numpy(), len(coords))
    # rows sorted and unique in (b, x, y, z): the occupancy bitmap (3); other
    # orders the grid (1); 2 C2S levels over config 1 (234 k rows in a 256^3
    # box) exceed the grid's 16 cells per row: the counting sort (0); 3 levels
    # keep their own order (2)
    qc = coords[:nbr.shape[0]].astype(np.int64)
    key = ((qc[:, 0] * 4096 + qc[:, 1]) * 4096 + qc[:, 2]) * 4096 + qc[:, 3]
    sorted_unique = bool(np.all(np.diff(key) > 0))
    expect = {"wide_bbox": 0, "c2s_2_levels": 0, "c2s_3_levels": 2}.get(which, 3 if sorted_unique else 1)
    assert h["grid_mode"] == expect, (h["grid_mode"], expect)
    assert which not in ("config1", "slab", "query_subset") or expect == 3
    if which == "c2s_3_levels":
        n_q = nbr.shape[0]
        assert np.array_equal(h["order"].ravel()[:n_q], np.arange(n_q))
    if which == "slab":
        spans = [h["halo"][t, h["tile_u"][t] - 1] - h["halo"][t, 0] for t in range(h["n_tiles"])
                 if 0 < h["tile_u"][t] <= F.PLAN_HALO_MAX]
        assert max(spans) > 131072 and h["n_overflow"] == 0
    if which == "clusters":
        assert h["n_overflow"] == h["n_tiles"]
    if which in ("duplicates", "config1"):
        assert h["n_unique"] == len(np.unique(coords, axis=0))
    # deterministic: a second build gives the same tables (entries past a
    # tile's halo count, and the tables of overflowing tiles, are not written)
    h2 = F.build_conv_plan(cfg, cd, nbr).to_host()
    for key in ("order", "tile_u", "overflow"):
        assert np.array_equal(h[key], h2[key]), key
    for t in range(h["n_tiles"]):
        U = h["tile_u"][t]
        if U <= F.PLAN_HALO_MAX:
            assert np.array_equal(h["halo"][t, :U], h2["halo"][t, :U])
            assert np.array_equal(h["lmap"][t], h2["lmap"][t])


def assert_same_plan(h, ref):
    for key in ("order", "tile_u", "overflow"):
        assert np.array_equal(h[key], ref[key]), key
    for t in range(h["n_tiles"]):
        U = h["tile_u"][t]
        if U <= F.PLAN_HALO_MAX:
            assert np.array_equal(h["halo"][t, :U], ref["halo"][t, :U]), t
            assert np.array_equal(h["lmap"][t], ref["lmap"][t]), t


@pytest.mark.parametrize("q", [None, 9000])
def test_overlapped_map_and_plan_matches_separate_builds(q):
    """map_and_plan_into (plan order on a side stream during the map build,
    tables after) == neighbor map build + sc_conv_plan_build on one stream."""
    coords = synth.config1_coords()
    cfg = F.SparseSubmConvConfig(32, 32)
    cd = dev(coords)
    n_q = len(coords) if q is None else q
    ref_nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd, query_rows=n_q)
    ref = F.build_conv_plan(cfg, cd, ref_nbr).to_host()
    nbr = torch.full((n_q, 27), -7, dtype=torch.int32, device="cuda")
    ws = F.NeighborMapWorkspace().get(len(coords))
    buf = torch.empty(F.conv_plan_bytes(n_q, 27), dtype=torch.uint8, device="cuda")
    for _ in range(3):  # repeated builds into the same buffers
        plan = F.map_and_plan_into(cfg, cd, nbr, ws, buf)
        torch.cuda.synchronize()
        assert torch.equal(nbr, ref_nbr)
        assert_same_plan(plan.to_host(), ref)


@pytest.mark.parametrize("cin,cout,groups,wdt", [(64, 128, 1, "bf16"), (96, 200, 1, "bf16"),
                                                  (64, 64, 2, "bf16"), (128, 64, 1, "i8")])
def test_weight_pack_layout(cin, cout, groups, wdt):
    rng = np.random.default_rng(cin + cout)
    cfg = F.SparseSubmConvConfig(cin, cout, groups=groups)
    cin_g, cout_g, K = cin // groups, cout // groups, 27
    if wdt == "bf16":
        w = rbf(synth.normal_f32(rng, (cout, K, cin_g)))
        wd = bf16_dev(w)
        wh = synth.bf16_bits(w).astype(np.int64)
    else:
        q, _ = synth.int8_weight(rng, cout, K, cin_g)
        wd = dev(q)
        wh = q.astype(np.int64)
    packed = F.pack_conv_weight(cfg, wd).cpu().numpy()
    hdr = packed[:256].view(np.int32)
    # header: magic "SCW1", groups, Cout_g, Cin_g, K, source dtype, 128-channel tiles, 0, total bytes
    assert hdr[0] == 0x31574353 and list(hdr[1:8]) == [groups, cout_g, cin_g, K, 1 if wdt == "bf16" else 2,
                                                      (cout_g + 127) // 128, 0]
    assert int(packed[32:40].view(np.int64)[0]) == packed.size
    packed = packed[256:].view(np.uint16).astype(np.int64)  # bf16 fragments for either type
    if wdt != "bf16":
        wh = synth.bf16_bits(wh.astype(np.float32)).astype(np.int64)  # int8 widened exactly
    n_ot, nkc = (cout_g + 127) // 128, cin_g // 32
    exp = np.zeros((groups, n_ot, K, nkc, 8, 64, 8), np.int64)
    for g in range(groups):
        for ot in range(n_ot):
            for jj in range(8):
                for lane in range(64):
                    o = ot * 128 + 16 * jj + (lane & 15)
                    if o >= cout_g:
                        continue
                    for c in range(nkc):
                        i0 = 32 * c + 8 * (lane >> 4)
                        exp[g, ot, :, c, jj, lane, :] = wh[g * cout_g + o, :, i0:i0 + 8]
    assert np.array_equal(packed.reshape(exp.shape), exp)


def planned(cfg, coords, x, w, b, *, wdt="bf16", w_scale=None, q=None, **kw):
    cd = dev(coords)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd, query_rows=q)
    plan = F.build_conv_plan(cfg, cd, nbr)
    wd = bf16_dev(w) if wdt == "bf16" else dev(w)
    pw = F.pack_conv_weight(cfg, wd)
    out = F.sparse_subm_conv_forward(cfg, bf16_dev(x), nbr, wd, dev(b),
                                     w_scale=None if w_scale is None else dev(w_scale),
                                     plan=plan, packed_weight=pw, **kw)
    return out, nbr.cpu().numpy(), plan


@pytest.mark.parametrize("cin,cout,groups", [(32, 32, 1), (64, 96, 1), (128, 128, 1), (256, 64, 1),
                                             (64, 64, 2), (96, 200, 1), (96, 64, 1)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_planned_conv_shapes(oracle, cin, cout, groups, out_dtype):
    coords = synth.config1_coords()
    rng = np.random.default_rng(cin * 7 + cout + groups)
    n = len(coords)
    x = rbf(synth.normal_f32(rng, (n, cin)))
    w = rbf(synth.conv_weight(rng, cout, 27, cin // groups, 1.0 / np.sqrt(27 * cin)))
    b = synth.normal_f32(rng, cout, 0.1)
    cfg = F.SparseSubmConvConfig(cin, cout, groups=groups)
    out, nbr, _ = planned(cfg, coords, x, w, b, out_dtype=out_dtype)
    exp = oracle.conv_ref_f64(ocfg(oracle, cfg), w, b, x, nbr)
    assert_close(out.float().cpu().numpy(), exp, TOL_BF16 if out_dtype == torch.bfloat16 else 2e-5,
                 "planned conv")


@pytest.mark.parametrize("kernel", [(1, 1, 1), (3, 1, 1), (1, 3, 3), (3, 3, 1)])
@pytest.mark.parametrize("cout", [64, 128])
def test_planned_small_kernels(oracle, kernel, cout):
    """Plans over fewer than 27 offsets (K = 1, 3, 9): a tile's used-offset
    mask has a few bits, down to one (K = 1: the halo is the tile's own rows);
    64 output channels take the 64-channel tile, 128 the 128-channel one."""
    coords = synth.config1_coords()
    rng = np.random.default_rng(sum(kernel) * 31 + cout)
    n, cin = len(coords), 64
    K = kernel[0] * kernel[1] * kernel[2]
    x = rbf(synth.normal_f32(rng, (n, cin)))
    w = rbf(synth.conv_weight(rng, cout, K, cin, 1.0 / np.sqrt(K * cin)))
    b = synth.normal_f32(rng, cout, 0.1)
    cfg = F.SparseSubmConvConfig(cin, cout, *kernel)
    out, nbr, _ = planned(cfg, coords, x, w, b, out_dtype=torch.bfloat16)
    assert nbr.shape == (n, K)
    exp = oracle.conv_ref_f64(ocfg(oracle, cfg), w, b, x, nbr)
    assert_close(out.float().cpu().numpy(), exp, TOL_BF16, f"planned conv, kernel {kernel}")


@pytest.mark.parametrize("n", [0, 1, 2, 257])
@pytest.mark.parametrize("cout", [64, 128])
def test_planned_tiny_inputs(oracle, n, cout):
    """Planned convs on 0, 1, 2 and 257 rows: the empty map and plan, a lone
    row whose only neighbour is itself (its tile is 255 padding rows), and a
    full tile followed by a one-row tile."""
    coords = np.ascontiguousarray(synth.config1_coords()[:n])
    rng = np.random.default_rng(n + cout)
    cin = 64
    x = rbf(synth.normal_f32(rng, (n, cin)))
    w = rbf(synth.conv_weight(rng, cout, 27, cin, 1.0 / np.sqrt(27 * cin)))
    b = synth.normal_f32(rng, cout, 0.1)
    cfg = F.SparseSubmConvConfig(cin, cout)
    out, nbr, _ = planned(cfg, coords, x, w, b, out_dtype=torch.bfloat16)
    assert tuple(out.shape) == (n, cout)
    if n == 0:
        return
    exp = oracle.conv_ref_f64(ocfg(oracle, cfg), w, b, x, nbr)
    assert_close(out.float().cpu().numpy(), exp, TOL_BF16, f"planned conv on {n} rows")


def test_planned_int8_weights(oracle):
    coords = synth.config1_coords()
    rng = np.random.default_rng(5)
    n, cin, cout = len(coords), 128, 64
    x = rbf(synth.normal_f32(rng, (n, cin)))
    q, scale = synth.int8_weight(rng, cout, 27, cin)
    b = synth.normal_f32(rng, cout, 0.1)
    cfg = F.SparseSubmConvConfig(cin, cout)
    out, nbr, _ = planned(cfg, coords, x, q, b, wdt="i8", w_scale=scale, out_dtype=torch.float32)
    exp = oracle.conv_ref_f64(ocfg(oracle, cfg), q.astype(np.float32), b, x, nbr, w_scale=scale)
    assert_close(out.cpu().numpy(), exp, 2e-5, "planned int8 conv")


@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize("cin,cout", [(128, 128), (64, 64), (128, 40)])  # 128- and 64-channel tiles
def test_planned_ln_silu_and_residual(oracle, affine, cin, cout):
    coords = synth.config1_coords()
    rng = np.random.default_rng(21)
    n = len(coords)
    x = rbf(synth.normal_f32(rng, (n, cin)))
    w = rbf(synth.conv_weight(rng, cout, 27, cin, 1 / np.sqrt(27 * cin)))
    b = synth.normal_f32(rng, cout, 0.1)
    lw = synth.normal_f32(rng, cout) if affine else None
    lb = synth.normal_f32(rng, cout) if affine else None
    res = rbf(synth.normal_f32(rng, (n, cout)))
    cfg = F.SparseSubmConvConfig(cin, cout)
    ocfg_ = oracle.OracleConfig(cin, cout)
    out, nbr, _ = planned(cfg, coords, x, w, b, residual=bf16_dev(res), layer_norm=True,
                          ln_weight=None if lw is None else dev(lw), ln_bias=None if lb is None else dev(lb),
                          ln_eps=1e-6, silu=True)
    conv = oracle.conv_ref_f64(ocfg_, w, b, x, nbr).astype(np.float32)
    exp = oracle.silu(oracle.layer_norm(conv, lw, lb, 1e-6)) + res
    assert_close(out.float().cpu().numpy(), exp, TOL_BF16, "planned LN/SiLU/residual")
    # conv -> + residual only (the second conv of the residual block)
    out2, _, _ = planned(cfg, coords, x, w, b, residual=dev(res), out_dtype=torch.float32)
    exp2 = oracle.conv_ref_f64(ocfg_, w, b, x, nbr) + res
    assert_close(out2.cpu().numpy(), exp2, 2e-5, "planned residual")


def spread_neighbour_coords(spacing, far=0):
    """One tile of 256 query centres (batch 0, x = 3i), each with two
    neighbours ((3i+1, 0, 0) and (3i, 1, 0)) stored `spacing` rows apart after
    the centres, the second half of them `far` rows further on; every other
    row is a filler of batch 1 (unique coords, no neighbour of a centre).  The
    tile's 768 distinct neighbour rows then span as many rows, and as many
    4,096-row pages, as the spacing makes them."""
    n_c = 256
    nb = np.zeros((2 * n_c, 4), np.int32)
    nb[0::2, 1] = 3 * np.arange(n_c) + 1
    nb[1::2, 1] = 3 * np.arange(n_c)
    nb[1::2, 2] = 1
    rows = n_c + np.arange(2 * n_c, dtype=np.int64) * spacing
    rows[n_c:] += far
    total = int(rows[-1]) + 1
    i = np.arange(total, dtype=np.int64)
    coords = np.stack([np.ones(total, np.int64), i & 1023, (i >> 10) & 1023, i >> 20], 1).astype(np.int32)
    coords[:n_c] = 0
    coords[:n_c, 1] = 3 * np.arange(n_c)
    coords[rows] = nb
    return coords


@pytest.mark.parametrize("spacing,far,conv", [(200, 0, True), (1, 200_000, True), (2000, 0, True),
                                              (1, 4_500_000, False)])
def test_plan_tile_neighbour_spans(oracle, spacing, far, conv):
    """The tile kernel's three ways of numbering a tile's distinct neighbour
    rows, forced by where those rows lie: within the LDS bitmap's 131,072-row
    window (spacing 200), beyond it in two clusters a few pages wide (the
    paged bitmap), spread over ~250 pages (more than the paged bitmap's 32:
    the hash table and sort), and in two clusters more than 4 M rows apart
    (past the page bitmap's range: the hash table).  The plan against the map
    it was built from, and the planned conv against the fp64 definition."""
    coords = spread_neighbour_coords(spacing, far)
    cfg = F.SparseSubmConvConfig(32, 32)
    cd = dev(coords)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd, query_rows=256)
    plan = F.build_conv_plan(cfg, cd, nbr)
    nb = nbr.cpu().numpy()
    assert (nb >= 0).sum() == 3 * 256  # each centre: itself and two neighbours
    h = check_plan(plan, nb, len(coords))
    assert h["n_tiles"] == 1 and h["tile_u"][0] == 768
    if not conv:
        return
    rng = np.random.default_rng(spacing + far)
    x = rbf(synth.normal_f32(rng, (len(coords), 32)))
    w = rbf(synth.conv_weight(rng, 32, 27, 32, 0.05))
    b = synth.normal_f32(rng, 32, 0.1)
    xd, wd = bf16_dev(x), bf16_dev(w)
    out = F.sparse_subm_conv_forward(cfg, xd, nbr, wd, dev(b), plan=plan, packed_weight=F.pack_conv_weight(cfg, wd),
                                     out_dtype=torch.float32)
    exp = oracle.conv_ref_f64(ocfg(oracle, cfg), w, b, x, nb)
    assert_close(out.cpu().numpy(), exp, 2e-5, f"neighbour span {spacing}/{far}")


def test_planned_conv_on_own_order(oracle):
    """The planned conv on rows that keep their own order (3 levels of C2S
    children, 170 k rows) equals the oracle on 2,000 sampled rows and the
    unplanned conv."""
    coords = c2s_children(3, frac=0.45)
    rng = np.random.default_rng(31)
    C = 64
    cfg = F.SparseSubmConvConfig(C, C)
    x = rbf(synth.normal_f32(rng, (len(coords), C)))
    w = rbf(synth.conv_weight(rng, C, 27, C, 1 / np.sqrt(27 * C)))
    b = synth.normal_f32(rng, C, 0.1)
    cd = dev(coords)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd)
    plan = F.build_conv_plan(cfg, cd, nbr)
    assert plan.to_host()["grid_mode"] == 2
    wd = bf16_dev(w)
    got = F.sparse_subm_conv_forward(cfg, bf16_dev(x), nbr, wd, dev(b), plan=plan,
                                     packed_weight=F.pack_conv_weight(cfg, wd)).float().cpu().numpy()
    ref = F.sparse_subm_conv_forward(cfg, bf16_dev(x), nbr, wd, dev(b)).float().cpu().numpy()
    rows = sample_rows(len(coords), rng, 2000, plan=plan)
    exp = oracle.conv_gemm_f64(ocfg(oracle, cfg), w, b, x, nbr.cpu().numpy()[rows])
    assert_close(got[rows], exp, TOL_BF16, "planned conv, own order")
    assert_close(got, ref, TOL_BF16, "planned vs unplanned")


def test_planned_overflow_tiles_and_query_subset(oracle):
    """Cluster centres as query rows: every tile's halo overflows, so every
    tile gathers its operands from global memory."""
    coords = cluster_coords(700)
    rng = np.random.default_rng(8)
    n, c = len(coords), 64
    x = rbf(synth.normal_f32(rng, (n, c)))
    w = rbf(synth.conv_weight(rng, c, 27, c, 0.05))
    b = synth.normal_f32(rng, c, 0.1)
    cfg = F.SparseSubmConvConfig(c, c)
    out, nbr, plan = planned(cfg, coords, x, w, b, q=700, out_dtype=torch.float32)
    h = plan.to_host()
    assert h["n_overflow"] == h["n_tiles"] == 3
    exp = oracle.conv_ref_f64(ocfg(oracle, cfg), w, b, x, nbr)
    assert_close(out.cpu().numpy(), exp, 2e-5, "overflow tiles")


@pytest.mark.parametrize("cin,cout,form", [(32, 32, "plain"), (64, 128, "ln"), (128, 64, "residual"),
                                           (96, 200, "plain")])
def test_planned_mixed_overflow(oracle, cin, cout, form):
    """Some tiles overflow (their operands gathered from global memory),
    others take the LDS halo, in one launch: both tile widths, the stage split
    of 64-channel tiles, LayerNorm -> SiLU in the tile and the residual."""
    a = synth.config1_coords()[:3000]
    cl = cluster_coords(300)
    cl[:, 1:] += 200
    # query rows: the shell, then the cluster centres; the cluster neighbours last
    coords = np.concatenate([a, cl[:300], cl[300:]])
    q = 3300
    rng = np.random.default_rng(9 + cin + cout)
    n = len(coords)
    x = rbf(synth.normal_f32(rng, (n, cin)))
    w = rbf(synth.conv_weight(rng, cout, 27, cin, 0.05))
    b = synth.normal_f32(rng, cout, 0.1)
    res = synth.normal_f32(rng, (q, cout))
    cfg = F.SparseSubmConvConfig(cin, cout)
    kw = {"out_dtype": torch.float32}
    if form == "ln":
        kw.update(layer_norm=True, silu=True, ln_eps=1e-6)
    if form == "residual":
        kw.update(residual=dev(res))
    out, nbr, plan = planned(cfg, coords, x, w, b, q=q, **kw)
    h = plan.to_host()
    assert 0 < h["n_overflow"] < h["n_tiles"]
    exp = oracle.conv_ref_f64(ocfg(oracle, cfg), w, b, x, nbr)
    if form == "ln":
        exp = oracle.silu(oracle.layer_norm(exp.astype(np.float32), None, None, 1e-6))
    if form == "residual":
        exp = exp + res
    assert_close(out.cpu().numpy(), exp, 2e-5 if form != "ln" else 1e-4, f"mixed overflow {form}")


def test_planned_config3_sampled_and_deterministic(oracle):
    """Config 3 (1.04M voxels, C=128, bf16): plan structure, sampled rows
    against the fp64 definition, bit-identical reruns, and agreement with the
    unplanned conv within the bf16 bar."""
    coords = synth.config3_coords()
    n, c = len(coords), 128
    rng = np.random.default_rng(3)
    x = rbf(synth.normal_f32(rng, (n, c)))
    w = rbf(synth.conv_weight(rng, c, 27, c, 1.0 / np.sqrt(27 * c)))
    b = np.zeros(c, np.float32)
    cfg = F.SparseSubmConvConfig(c, c)
    cd = dev(coords)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd)
    plan = F.build_conv_plan(cfg, cd, nbr)
    nb = nbr.cpu().numpy()
    h = check_plan(plan, nb, n)
    assert h["brick_shift"] == 3
    xd, wd, bd = bf16_dev(x), bf16_dev(w), dev(b)
    pw = F.pack_conv_weight(cfg, wd)
    o1 = F.sparse_subm_conv_forward(cfg, xd, nbr, wd, bd, plan=plan, packed_weight=pw)
    o2 = F.sparse_subm_conv_forward(cfg, xd, nbr, wd, bd, plan=plan, packed_weight=pw)
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    sample = np.sort(np.random.default_rng(0).choice(n, 3000, replace=False))
    exp = oracle.conv_ref_f64(ocfg(oracle, cfg), w, b, x, nb[sample])
    assert_close(o1.float().cpu().numpy()[sample], exp, TOL_BF16, "config3 planned sampled")
    unplanned = F.sparse_subm_conv_forward(cfg, xd, nbr, wd, bd)
    d = (o1.float() - unplanned.float()).abs().max().item()
    assert d <= 2.0 ** -5, d  # one bf16 ulp at |y| < 4 at most


def test_plan_argument_errors():
    cfg = F.SparseSubmConvConfig(64, 64)
    coords = dev(synth.config1_coords()[:1000])
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, coords)
    plan = F.build_conv_plan(cfg, coords, nbr)
    x = torch.zeros((1000, 64), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((64, 27, 64), dtype=torch.bfloat16, device="cuda")
    nbr_short = nbr[:500].contiguous()
    with pytest.raises(F.SparseConvError):
        F.sparse_subm_conv_forward(cfg, x, nbr_short, w, plan=plan, packed_weight=F.pack_conv_weight(cfg, w))
    small = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(F.SparseConvError) as e:
        F.conv_plan_build_into(cfg, coords, nbr, small)
    assert e.value.status == 5


def _raw_planned(cfg, x, nbr, w, packed, out, plan_buf, ln_workspace=None):
    """sc_subm_conv_forward_planned straight through the C ABI (no host-side
    shape checks of the plan or the packed weights); with ``ln_workspace``,
    LayerNorm over the row (wider than one tile: the f32 staging path)."""
    import ctypes

    from bevy_synth_amd import _capi

    def p(t):
        return ctypes.c_void_p(t.data_ptr())
    epi = _capi.ScConvEpilogue()
    if ln_workspace is not None:
        epi.layer_norm, epi.ln_eps = 1, 1e-6
        epi.workspace, epi.workspace_bytes = p(ln_workspace), ln_workspace.numel()
    c = cfg.to_c()
    return _capi.load().sc_subm_conv_forward_planned(
        ctypes.byref(c), 1, p(x), x.shape[0], p(nbr), nbr.shape[0], 1, p(w), p(packed), None, None,
        ctypes.byref(epi), 1, p(out), p(plan_buf), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_raw_abi_rejects_plan_and_weights_of_another_shape(oracle):
    """A plan built for another map (here a smaller one: its tables end long
    before the call's layout would put them) or packed weights of another
    config must not be read past their headers: the conv writes nothing and
    sc_conv_plan_check reports it; a rebuilt plan clears the status."""
    coords = synth.config1_coords()
    rng = np.random.default_rng(71)
    n = len(coords)
    cfg = F.SparseSubmConvConfig(64, 64)
    cd_big, cd_small = dev(coords), dev(coords[:3000])
    nbr_big = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd_big)
    nbr_small = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd_small)
    plan_small = F.build_conv_plan(cfg, cd_small, nbr_small)
    plan_big = F.build_conv_plan(cfg, cd_big, nbr_big)
    x = rbf(synth.normal_f32(rng, (n, 64)))
    w = rbf(synth.conv_weight(rng, 64, 27, 64, 1 / np.sqrt(27 * 64)))
    xd, wd = bf16_dev(x), bf16_dev(w)
    pw = F.pack_conv_weight(cfg, wd)
    sentinel = torch.full((n, 64), 7.0, dtype=torch.bfloat16, device="cuda")

    out = sentinel.clone()
    assert _raw_planned(cfg, xd, nbr_big, wd, pw, out, plan_small.buf) == 0
    with pytest.raises(F.SparseConvError) as e:
        F.conv_plan_check(plan_small)
    assert e.value.status == 2 and "another map" in e.value.message
    assert torch.equal(out, sentinel)

    cfg32 = F.SparseSubmConvConfig(64, 32)
    pw32 = F.pack_conv_weight(cfg32, bf16_dev(w[:32]))
    F.conv_plan_check(plan_big)  # clean so far
    out = sentinel.clone()
    assert _raw_planned(cfg, xd, nbr_big, wd, pw32, out, plan_big.buf) == 0
    with pytest.raises(F.SparseConvError) as e:
        F.conv_plan_check(plan_big)
    assert e.value.status == 2 and "packed weights" in e.value.message
    assert torch.equal(out, sentinel)

    # rebuilding clears the status; the matching call then computes the conv
    plan_big = F.build_conv_plan(cfg, cd_big, nbr_big)
    assert _raw_planned(cfg, xd, nbr_big, wd, pw, out, plan_big.buf) == 0
    F.conv_plan_check(plan_big)
    exp = oracle.conv_ref_f64(ocfg(oracle, cfg), w, np.zeros(64, np.float32), x, nbr_big.cpu().numpy())
    assert_close(out.float().cpu().numpy(), exp, TOL_BF16, "planned conv after rebuild")


def test_raw_abi_mismatch_leaves_wide_layer_norm_output_untouched(oracle):
    """Cout = 256 with LayerNorm: the conv stores f32 into the epilogue
    workspace and a row kernel normalises it into d_out.  With packed weights
    of another config the conv writes nothing, and neither does the row
    kernel (it is gated on the plan's status); the flagged plan then keeps a
    matching call from writing too, until it is rebuilt."""
    coords = synth.config1_coords()
    rng = np.random.default_rng(72)
    n = len(coords)
    cfg = F.SparseSubmConvConfig(64, 256)
    cd = dev(coords)
    nbr = F.neighbor_rows_tensor_from_coords_tensor(cfg, cd)
    plan = F.build_conv_plan(cfg, cd, nbr)
    x = rbf(synth.normal_f32(rng, (n, 64)))
    w = rbf(synth.conv_weight(rng, 256, 27, 64, 1 / np.sqrt(27 * 64)))
    xd, wd = bf16_dev(x), bf16_dev(w)
    pw = F.pack_conv_weight(cfg, wd)
    pw128 = F.pack_conv_weight(F.SparseSubmConvConfig(64, 128), bf16_dev(w[:128]))
    ws = torch.zeros(n * 256 * 4, dtype=torch.uint8, device="cuda")
    sentinel = torch.full((n, 256), 7.0, dtype=torch.bfloat16, device="cuda")

    out = sentinel.clone()
    assert _raw_planned(cfg, xd, nbr, wd, pw128, out, plan.buf, ln_workspace=ws) == 0
    with pytest.raises(F.SparseConvError) as e:
        F.conv_plan_check(plan)
    assert e.value.status == 2 and "packed weights" in e.value.message
    assert torch.equal(out, sentinel)
    # the flagged plan: a matching call writes nothing until the rebuild
    assert _raw_planned(cfg, xd, nbr, wd, pw, out, plan.buf, ln_workspace=ws) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, sentinel)
    plan = F.build_conv_plan(cfg, cd, nbr)
    assert _raw_planned(cfg, xd, nbr, wd, pw, out, plan.buf, ln_workspace=ws) == 0
    F.conv_plan_check(plan)
    conv = oracle.conv_ref_f64(ocfg(oracle, cfg), w, np.zeros(256, np.float32), x, nbr.cpu().numpy())
    exp = oracle.layer_norm(conv.astype(np.float32), None, None, 1e-6)
    assert_close(out.float().cpu().numpy(), exp, TOL_BF16, "planned conv + wide LayerNorm after rebuild")

"""Pins the CPU oracle (oracle/sc_oracle.c) before it is trusted as the checker.

Each test names the reference test / fixture it reproduces, or the
independent formulation it is compared with (closed form, brute force,
numpy re-derivation with different primitives).
"""
import numpy as np
import pytest
import torch

from tests.tolerance import rel_err


def line_coords(n):
    c = np.zeros((n, 4), dtype=np.uint32)
    c[:, 1] = np.arange(n)
    return c


def checkerboard(nx, ny, nz):
    """make_sparse_grid_coords, crates/burn_flex_gmm/src/lib.rs:784-797."""
    out = [(0, x, y, z) for x in range(nx) for y in range(ny) for z in range(nz)
           if (x + y + z) % 2 == 0]
    return np.array(out, dtype=np.uint32)


# --------------------------------------------------------------- KATs

def test_kat_conv_uses_neighbor_voxels(oracle, kats):
    """sparse_decoder_tests.rs:190-236: x=0,1; in [1,2]; w [10,1,100] (3x1x1) -> [201, 12]."""
    g = kats["conv_uses_neighbor_voxels"]
    cfg = oracle.OracleConfig(1, 1, *g["config"]["kernel"])
    x = np.array(g["input"], np.float32)
    w = np.array(g["weight"], np.float32)
    b = np.array(g["bias"], np.float32)
    want = np.array(g["expected_output"], np.float32)
    for out in (oracle.conv_flex(cfg, w, b, g["coords"], x), oracle.conv_legacy(cfg, w, b, g["coords"], x)):
        assert np.abs(out - want).max() < g["tolerance"]


def test_kat_query_chunks_keep_global_neighbors(oracle, kats):
    """sparse_decoder_tests.rs:239-292: full map [-1,0,1]; chunk rebuild [-1,0,-1];
    the query-row conv on the full input equals the full conv's row 0."""
    g = kats["query_chunks_keep_global_neighbors"]
    cfg = oracle.OracleConfig(1, 1, *g["config"]["kernel"])
    coords = np.array(g["coords"], np.uint32)
    full = oracle.build_neighbor_rows(cfg, coords)
    chunk = oracle.build_neighbor_rows(cfg, coords[:1])
    assert full.tolist() == g["expected_full_map"]
    assert chunk.tolist() == g["expected_chunk_map_first_row_only"]
    q = oracle.build_neighbor_rows(cfg, coords, query_rows=1)
    assert q.tolist() == g["expected_query_rows_1_map"]
    c = kats["conv_uses_neighbor_voxels"]
    w = np.array(c["weight"], np.float32)
    b = np.array(c["bias"], np.float32)
    x = np.array(c["input"], np.float32)
    fo = oracle.conv_flex_precomputed(cfg, w, b, x, full)
    qo = oracle.conv_flex_precomputed(cfg, w, b, x, full[:1])
    assert np.array_equal(qo, fo[:1])


def test_kat_subdivision_child_expand(oracle, kats):
    """decoder_guide_subdivision_tensor_handoff_parity, sparse_decoder_tests.rs:37-124:
    parents (0,0,0),(1,0,0); active (0,0),(0,3),(1,7) -> child coords
    [0,0,0,0],[0,1,1,0],[0,3,1,1], linear idx [0,3,15]."""
    g = kats["subdivision_child_expand"]
    parents = np.array(g["parent_coords"], np.uint32)
    pairs = np.array(g["active_pairs"], np.int32)
    cc, li = oracle.subdivide_expand(parents, pairs)
    assert cc.tolist() == g["expected_child_coords"]
    assert li.tolist() == g["expected_linear_idx"]


# ------------------------------------------- reference cross-impl tests

def _rand_layer(oracle, rng_seed, cfg, rows):
    rng = oracle.Lcg(rng_seed)
    x = rng.next_f32(rows * cfg.in_channels).reshape(rows, cfg.in_channels)
    cin_g = cfg.in_channels // cfg.groups
    w = rng.next_f32(cfg.out_channels * cfg.kernel_rows * cin_g)
    b = rng.next_f32(cfg.out_channels)
    return x, w, b


def test_flex_matches_legacy_small_kernel(oracle):
    """crates/burn_flex_gmm/src/lib.rs:799-840 (seed 42, 3x1x1, groups 2, 16 line coords)."""
    cfg = oracle.OracleConfig(4, 6, 3, 1, 1, groups=2)
    coords = line_coords(16)
    x, w, b = _rand_layer(oracle, 42, cfg, 16)
    legacy = oracle.conv_legacy(cfg, w, b, coords, x)
    flex = oracle.conv_flex(cfg, w, b, coords, x)
    assert np.max(np.abs(legacy - flex)) <= 1e-5


def test_flex_handles_empty_rows(oracle):
    """crates/burn_flex_gmm/src/lib.rs:842-862."""
    cfg = oracle.OracleConfig(2, 2, 1, 1, 1)
    out = oracle.conv_flex(cfg, np.array([1, 0, 0, 1], np.float32), np.array([0.25, -0.5], np.float32),
                           np.zeros((0, 4), np.uint32), np.zeros((0, 2), np.float32))
    assert out.shape == (0, 2)


@pytest.mark.parametrize("groups", [1, 2])
def test_fast_flex_matches_flex_to_rounding(oracle, groups):
    """The CPU baseline's timing conv (packed FMA sgemm, oracle/sc_fastgemm.c)
    computes the oracle's flex conv: equal to float rounding, on 1 and 3
    threads, with row and column counts off the 6 x 16 register tile."""
    rng = np.random.default_rng(groups)
    cfg = oracle.OracleConfig(48 * groups, 40 * groups, groups=groups)
    c = rng.integers(0, 12, size=(700, 4)).astype(np.int32)
    c[:, 0] = 0
    c = np.unique(c, axis=0)
    x = rng.standard_normal((len(c), cfg.in_channels)).astype(np.float32)
    w = rng.standard_normal((cfg.out_channels, 27, 48)).astype(np.float32)
    b = rng.standard_normal(cfg.out_channels).astype(np.float32)
    nbr = oracle.build_neighbor_rows(cfg, c)
    ref = oracle.conv_flex_precomputed(cfg, w, b, x, nbr)
    for t in (1, 3):
        got = oracle.conv_flex_fast(cfg, w, b, x, nbr, threads=t)
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max(), t


def test_flex_precomputed_matches_default(oracle):
    """crates/burn_flex_gmm/src/lib.rs:864-915 (seed 73, groups 2, 32 line coords)."""
    cfg = oracle.OracleConfig(8, 12, 3, 1, 1, groups=2)
    coords = line_coords(32)
    x, w, b = _rand_layer(oracle, 73, cfg, 32)
    expected = oracle.conv_flex(cfg, w, b, coords, x)
    nbr = oracle.build_neighbor_rows(cfg, coords)
    packed = oracle.pack_flex_weight(cfg, w)
    actual = oracle.conv_flex_precomputed(cfg, w, b, x, nbr, packed)
    assert np.max(np.abs(expected - actual)) <= 1e-5


@pytest.mark.parametrize("axis_order", [(0, 1, 2), (2, 1, 0), (1, 2, 0)])
@pytest.mark.parametrize("axis_sign", [(1, 1, 1), (-1, 1, 1), (1, -1, -1)])
def test_flex_matches_legacy_axis_permutations(oracle, axis_order, axis_sign):
    """crates/burn_flex_gmm/src/lib.rs:917-972 (seed 991, 6x5x4 checkerboard, groups 2)."""
    coords = checkerboard(6, 5, 4)
    rng = oracle.Lcg(991)
    x = rng.next_f32(len(coords) * 6).reshape(-1, 6)
    w = rng.next_f32(8 * 27 * 3)
    b = rng.next_f32(8)
    cfg = oracle.OracleConfig(6, 8, 3, 3, 3, groups=2, axis_order=axis_order, axis_sign=axis_sign)
    legacy = oracle.conv_legacy(cfg, w, b, coords, x)
    flex = oracle.conv_flex(cfg, w, b, coords, x)
    assert np.max(np.abs(legacy - flex)) <= 2e-5


def test_decoder_flex_matches_legacy(oracle):
    """sparse_decoder_tests.rs:295-368 (seed 123, 4->6, 3x1x1, groups 2, 32 coords)."""
    rng = oracle.Lcg(123)
    w = rng.next_f32(6 * 3 * 2)
    b = rng.next_f32(6)
    coords = line_coords(32)
    x = rng.next_f32(32 * 4).reshape(32, 4)
    cfg = oracle.OracleConfig(4, 6, 3, 1, 1, groups=2)
    assert np.max(np.abs(oracle.conv_legacy(cfg, w, b, coords, x)
                         - oracle.conv_flex(cfg, w, b, coords, x))) <= 1e-5


# --------------------------------------------- independent formulations

def test_lcg_matches_bigint_reference(oracle):
    """Lcg of crates/burn_flex_gmm/src/lib.rs:764-778, recomputed with Python ints."""
    got = oracle.Lcg(42).next_f32(64)
    s = 42 | 1
    exp = []
    for _ in range(64):
        s = (s * 6364136223846793005 + 1) % (1 << 64)
        bits = ((s >> 40) & 0xFFFFFFFF) | 1
        exp.append(np.float32(np.float32(bits) / np.float32(4294967295.0)) * np.float32(2.0)
                   - np.float32(1.0))
    assert np.array_equal(got, np.array(exp, np.float32))


def test_kernel_layout_closed_form(oracle):
    """Default axes: k = (dx+1)*9 + (dy+1)*3 + (dz+1), centre k = 13."""
    cfg = oracle.OracleConfig(1, 1)
    off = oracle.kernel_layout(cfg)
    for k in range(27):
        assert tuple(off[k]) == (k // 9 - 1, (k // 3) % 3 - 1, k % 3 - 1)
    # axis_order (2,1,0): kd moves z; sign -1 on axis 0 flips it.
    off2 = oracle.kernel_layout(oracle.OracleConfig(1, 1, axis_order=(2, 1, 0), axis_sign=(-1, 1, 1)))
    for k in range(27):
        assert tuple(off2[k]) == (k % 3 - 1, (k // 3) % 3 - 1, -(k // 9 - 1))


def _random_coords(rng, n, span, dup_frac=0.0, batches=1):
    c = np.zeros((n, 4), np.uint32)
    c[:, 0] = rng.integers(0, batches, n)
    c[:, 1:] = rng.integers(0, span, (n, 3))
    if dup_frac > 0:
        k = int(n * dup_frac)
        src = rng.integers(0, n, k)
        dst = rng.integers(0, n, k)
        c[dst] = c[src]
    return c


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_hash_build_matches_bruteforce_scan(oracle, seed):
    """Lowest-row hash build == the K1 brute-force scan semantics
    (neighbor_kernels.rs:3-46), with duplicates and two batches."""
    rng = np.random.default_rng(seed)
    coords = _random_coords(rng, 300, 6, dup_frac=0.1, batches=2)
    cfg = oracle.OracleConfig(1, 1)
    assert np.array_equal(oracle.build_neighbor_rows(cfg, coords, lowest_row_on_duplicate=True),
                          oracle.build_neighbor_rows_scan(cfg, coords))


def test_duplicate_semantics_cpu_last_device_first(oracle):
    """Duplicated coord: CPU HashMap keeps the last row (lib.rs:83-86), the device
    algorithms the lowest (wgpu/tests.rs:1802-1853 checks hash == scan)."""
    coords = np.concatenate([line_coords(128), np.array([[0, 17, 0, 0], [0, 32, 0, 0],
                                                          [0, 17, 0, 0], [0, 32, 0, 0]], np.uint32)])
    cfg = oracle.OracleConfig(4, 4, 3, 3, 1)
    first = oracle.build_neighbor_rows(cfg, coords, lowest_row_on_duplicate=True)
    last = oracle.build_neighbor_rows(cfg, coords, lowest_row_on_duplicate=False)
    scan = oracle.build_neighbor_rows_scan(cfg, coords)
    assert np.array_equal(first, scan)
    centre = 4  # (0,0,0) offset of 3x3x1
    assert first[16, centre + 3] == 17 and last[16, centre + 3] == 130


def test_dense_grid_equals_numpy_correlation(oracle):
    """On a fully dense 5x4x3 grid the submanifold conv is an ordinary zero-padded
    3-D correlation: out[p] = b + sum_d in[p + d] . W[d].  Recomputed with numpy
    shifts, so an offset sign, axis or operand-order mistake fails."""
    rng = np.random.default_rng(5)
    shape = (5, 4, 3)
    cin, cout = 3, 4
    grid = np.stack(np.meshgrid(*[np.arange(s) for s in shape], indexing="ij"), -1).reshape(-1, 3)
    coords = np.concatenate([np.zeros((len(grid), 1), np.uint32), grid.astype(np.uint32)], 1)
    x = rng.standard_normal((len(grid), cin)).astype(np.float32)
    w = rng.standard_normal((cout, 27, cin)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    cfg = oracle.OracleConfig(cin, cout)
    got = oracle.conv_flex(cfg, w, b, coords, x)
    vol = x.reshape(*shape, cin).astype(np.float64)
    pad = np.pad(vol, ((1, 1), (1, 1), (1, 1), (0, 0)))
    exp = np.broadcast_to(b.astype(np.float64), (*shape, cout)).copy()
    for k in range(27):
        dx, dy, dz = k // 9 - 1, (k // 3) % 3 - 1, k % 3 - 1
        sh = pad[1 + dx:1 + dx + shape[0], 1 + dy:1 + dy + shape[1], 1 + dz:1 + dz + shape[2]]
        exp += sh @ w[:, k, :].T.astype(np.float64)
    assert rel_err(got, exp.reshape(-1, cout)) < 1e-5
    assert rel_err(oracle.conv_ref_f64(cfg, w, b, x, oracle.build_neighbor_rows(cfg, coords)),
                   exp.reshape(-1, cout)) < 1e-12


@pytest.mark.parametrize("groups,int8", [(1, False), (2, False), (1, True)])
def test_conv_gemm_f64_equals_conv_ref_f64(oracle, groups, int8):
    """The numpy im2col form used for the large sampled GPU checks is the same
    definition as conv_ref_f64 (itself pinned by the correlation above): random
    coords, absent neighbours, grouped channels, int8 weights with
    per-channel scales; entries past the input count as absent."""
    rng = np.random.default_rng(17 + groups + int8)
    coords = _random_coords(rng, 400, 12)
    cin, cout = 8 * groups, 6 * groups
    cfg = oracle.OracleConfig(cin, cout, groups=groups)
    x = rng.standard_normal((400, cin)).astype(np.float32)
    if int8:
        w = rng.integers(-127, 128, (cout, 27, cin // groups)).astype(np.float32)
        sc = rng.uniform(0.5, 1.5, cout).astype(np.float32) / 127
    else:
        w = rng.standard_normal((cout, 27, cin // groups)).astype(np.float32)
        sc = None
    b = rng.standard_normal(cout).astype(np.float32)
    nbr = oracle.build_neighbor_rows(cfg, coords)
    nbr[::7, 3] = -1           # absent neighbours mid-row
    exp = oracle.conv_ref_f64(cfg, w, b, x, nbr, sc)
    got = oracle.conv_gemm_f64(cfg, w, b, x, nbr, sc, chunk=64)
    nbr[::5, 4] = 400          # past the input: absent in the GEMM form (the device's rule)
    nbr2 = np.where(nbr >= 400, -1, nbr)
    assert np.array_equal(oracle.conv_gemm_f64(cfg, w, b, x, nbr, sc), oracle.conv_gemm_f64(cfg, w, b, x, nbr2, sc))
    assert np.max(np.abs(got - exp)) <= 1e-12 * max(1.0, float(np.max(np.abs(exp))))


def test_k1_conv_is_dense_gemm_and_isolated_rows_get_bias(oracle):
    rng = np.random.default_rng(9)
    n, cin, cout = 50, 16, 24
    coords = _random_coords(rng, n, 1000)
    x = rng.standard_normal((n, cin)).astype(np.float32)
    w = rng.standard_normal((cout, 1, cin)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    cfg1 = oracle.OracleConfig(cin, cout, 1, 1, 1)
    nbr = oracle.build_neighbor_rows(cfg1, coords)
    assert np.array_equal(nbr[:, 0], np.arange(n))
    got = oracle.conv_flex_precomputed(cfg1, w, b, x, nbr)
    assert rel_err(got, x.astype(np.float64) @ w[:, 0, :].T.astype(np.float64) + b) < 1e-5
    # isolated voxels (spacing 3) only see themselves; with the centre tap zeroed -> bias.
    iso = np.zeros((10, 4), np.uint32)
    iso[:, 1] = np.arange(10) * 3
    cfg3 = oracle.OracleConfig(cin, cout)
    w3 = rng.standard_normal((cout, 27, cin)).astype(np.float32)
    w3[:, 13, :] = 0
    out = oracle.conv_flex(cfg3, w3, b, iso, x[:10])
    assert np.array_equal(out, np.broadcast_to(b, out.shape))


def test_row_permutation_equivariance(oracle):
    """Permuting coord rows permutes outputs (the map relabels consistently)."""
    rng = np.random.default_rng(11)
    coords = checkerboard(6, 6, 6).astype(np.uint32)
    n = len(coords)
    x = rng.standard_normal((n, 5)).astype(np.float32)
    w = rng.standard_normal((7, 27, 5)).astype(np.float32)
    b = rng.standard_normal(7).astype(np.float32)
    cfg = oracle.OracleConfig(5, 7)
    base = oracle.conv_flex(cfg, w, b, coords, x)
    perm = rng.permutation(n)
    permuted = oracle.conv_flex(cfg, w, b, coords[perm], x[perm])
    assert rel_err(permuted, base[perm]) < 1e-5


def test_bf16_round_matches_torch_rne(oracle):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10,
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 0.0, -0.0,
                                  3.0e38, 1e-40], np.float32)])
    got = oracle.bf16_round(x)
    exp = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_layer_norm_silu_closed_form(oracle):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((64, 96)) * 3 + 1).astype(np.float32)
    w = rng.standard_normal(96).astype(np.float32)
    b = rng.standard_normal(96).astype(np.float32)
    got = oracle.silu(oracle.layer_norm(x, w, b, 1e-6))
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    var = ((xd - mu) ** 2).mean(1, keepdims=True)
    y = (xd - mu) / np.sqrt(var + 1e-6) * w + b
    exp = y / (1 + np.exp(-y))
    assert rel_err(got, exp) < 1e-5


def test_subdivision_active_matches_argwhere(oracle):
    rng = np.random.default_rng(6)
    logits = rng.standard_normal((200, 8)).astype(np.float32)
    thr = rng.standard_normal(8).astype(np.float32) * 0.3
    pairs = oracle.subdivision_active(logits, thr)
    assert np.array_equal(pairs, np.argwhere(logits > thr[None, :]).astype(np.int32))


def test_channel2spatial_host_equals_device_form(oracle):
    """Host channel2spatial + repeat_interleave skip (sparse_decoder_wgpu_ops.rs
    :1999-2076) == the device form: reshape [P*8, C/8] + select(linear_idx) and a
    grouped broadcast add (sparse_decoder_runtime_impl.rs:1054-1133)."""
    rng = np.random.default_rng(7)
    P, cin, cout = 40, 64, 16
    parents = _random_coords(rng, P, 50)
    feats = rng.standard_normal((P, cin)).astype(np.float32)
    mask = (rng.random((P, 8)) < 0.4).astype(np.uint8)
    cc, cf = oracle.channel2spatial(parents, feats, cin, mask)
    pairs = np.argwhere(mask).astype(np.int32)
    cc2, li = oracle.subdivide_expand(parents, pairs)
    assert np.array_equal(cc, cc2)
    assert np.array_equal(cf, feats.reshape(P * 8, cin // 8)[li])
    h = rng.standard_normal((len(li), cout)).astype(np.float32)
    rep = cout // (cin // 8)
    host = h + oracle.repeat_interleave(cf, rep)
    dev = (h.reshape(len(li), cin // 8, rep) + cf[:, :, None]).reshape(len(li), cout)
    assert np.array_equal(host, dev)
    assert np.array_equal(oracle.repeat_interleave(cf, rep), np.repeat(cf, rep, axis=1))


def test_c2s_block_matches_numpy_composition(oracle):
    """oracle.c2s_block (host loops) == a numpy composition of the device-form
    steps (LN+SiLU closed form, conv_ref_f64, reshape/select, broadcast skip)."""
    rng = np.random.default_rng(8)
    g = np.stack(np.meshgrid(np.arange(4), np.arange(4), np.arange(3), indexing="ij"), -1).reshape(-1, 3)
    parents = np.concatenate([np.zeros((len(g), 1), np.uint32), g.astype(np.uint32)], 1)
    P, cin, cout = len(parents), 16, 8
    feats = rng.standard_normal((P, cin)).astype(np.float32)
    mask = (rng.random((P, 8)) < 0.5).astype(np.uint8)
    n1w = rng.standard_normal(cin).astype(np.float32)
    n1b = rng.standard_normal(cin).astype(np.float32)
    c1 = oracle.OracleConfig(cin, 8 * cout)
    c2 = oracle.OracleConfig(cout, cout)
    w1 = (rng.standard_normal((8 * cout, 27, cin)) * 0.1).astype(np.float32)
    b1 = rng.standard_normal(8 * cout).astype(np.float32)
    w2 = (rng.standard_normal((cout, 27, cout)) * 0.1).astype(np.float32)
    b2 = rng.standard_normal(cout).astype(np.float32)
    cc, out = oracle.c2s_block(parents, feats, mask, n1w, n1b, c1, w1, b1, c2, w2, b2)

    def ln_silu(x, w=None, b=None):
        x = x.astype(np.float64)
        mu = x.mean(1, keepdims=True)
        y = (x - mu) / np.sqrt(((x - mu) ** 2).mean(1, keepdims=True) + 1e-6)
        if w is not None:
            y = y * w + b
        return y / (1 + np.exp(-y))

    h = ln_silu(feats, n1w, n1b)
    h1 = oracle.conv_ref_f64(c1, w1, b1, h.astype(np.float32), oracle.build_neighbor_rows(c1, parents))
    pairs = np.argwhere(mask).astype(np.int32)
    cc2, li = oracle.subdivide_expand(parents, pairs)
    assert np.array_equal(cc, cc2)
    hup = ln_silu(h1.reshape(P * 8, cout)[li])
    h2 = oracle.conv_ref_f64(c2, w2, b2, hup.astype(np.float32), oracle.build_neighbor_rows(c2, cc2))
    skip = feats.reshape(P * 8, cin // 8)[li]
    exp = (h2.reshape(len(li), cin // 8, -1) + skip[:, :, None]).reshape(len(li), cout)
    assert rel_err(out, exp) < 1e-4


def test_f16_round_matches_numpy_float16(oracle):
    """f16_round (quantize_f16_inplace: f32 -> binary16 RNE -> f32) bit for bit
    against numpy's float16 cast: normals at every scale, subnormals, the
    overflow boundary (65504 / 65520), exact ties between f16 neighbours
    (round to even), signed zeros and infinities."""
    rng = np.random.default_rng(0)
    parts = [rng.standard_normal(50000).astype(np.float32) * np.float32(s)
             for s in (1e-7, 1e-5, 1e-3, 1.0, 100.0, 3e4, 7e4)]
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, -65520.0, np.inf, -np.inf,
                     2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001, 2.0 ** -14, 2.0 ** -14 * (1 - 2.0 ** -11)],
                    np.float32)
    h = rng.integers(0x0001, 0x7bff, 20000).astype(np.uint16).view(np.float16).astype(np.float32)
    ties = (h.view(np.uint32) + (1 << 12)).view(np.float32)      # exactly half an f16 ulp above (normals)
    x = np.concatenate(parts + [edge, ties, -ties])
    with np.errstate(over="ignore"):
        exp = x.astype(np.float16).astype(np.float32)
    got = oracle.f16_round(x)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))

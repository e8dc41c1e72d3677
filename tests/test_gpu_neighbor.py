"""GPU parity: the HIP neighbour map is bit-exact against the oracle (device
semantics: lowest row on duplicated coords), on the reference's own test
shapes and on the benchmark geometries."""
import numpy as np
import pytest
import torch

from bevy_synth_amd import flex_gmm as F
from bevy_synth_amd import synth
from bevy_synth_amd._capi import SparseConvError

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def gpu_map(cfg, coords, query_rows=None):
    out = F.neighbor_rows_tensor_from_coords_tensor(cfg, dev(coords.astype(np.int32)), query_rows)
    return out.cpu().numpy()


def ocfg(oracle, cfg):
    return oracle.OracleConfig(cfg.in_channels, cfg.out_channels, cfg.kernel_d, cfg.kernel_h,
                               cfg.kernel_w, groups=cfg.groups, axis_order=cfg.axis_order,
                               axis_sign=cfg.axis_sign)


def line_coords(n):
    c = np.zeros((n, 4), np.int32)
    c[:, 1] = np.arange(n)
    return c


def test_kat_query_chunks(oracle, kats):
    """sparse_decoder_tests.rs:239-292."""
    g = kats["query_chunks_keep_global_neighbors"]
    cfg = F.SparseSubmConvConfig(1, 1, *g["config"]["kernel"])
    coords = np.array(g["coords"], np.int32)
    assert gpu_map(cfg, coords).tolist() == g["expected_full_map"]
    assert gpu_map(cfg, coords[:1]).tolist() == g["expected_chunk_map_first_row_only"]
    assert gpu_map(cfg, coords, query_rows=1).tolist() == g["expected_query_rows_1_map"]


@pytest.mark.parametrize("dims,n", [((3, 3, 1), 192), ((9, 9, 9), 256), ((9, 9, 9), 512),
                                    ((3, 3, 3), 5000), ((1, 1, 1), 100)])
def test_line_coords_match_scan(oracle, dims, n):
    """wgpu/tests.rs:1752-1986 (hash / sorted / bucket == scan on line coords)."""
    cfg = F.SparseSubmConvConfig(4, 4, *dims)
    coords = line_coords(n)
    exp = oracle.build_neighbor_rows(ocfg(oracle, cfg), coords)
    if n <= 600:
        assert np.array_equal(exp, oracle.build_neighbor_rows_scan(ocfg(oracle, cfg), coords))
    assert np.array_equal(gpu_map(cfg, coords), exp)


def test_duplicate_coords_lowest_row(oracle):
    """wgpu/tests.rs:1802-1853: 128 line coords + duplicates of x=17 and x=32."""
    cfg = F.SparseSubmConvConfig(4, 4, 3, 3, 1)
    coords = np.concatenate([line_coords(128), np.array([[0, 17, 0, 0], [0, 32, 0, 0],
                                                         [0, 17, 0, 0], [0, 32, 0, 0]], np.int32)])
    got = gpu_map(cfg, coords)
    assert np.array_equal(got, oracle.build_neighbor_rows_scan(ocfg(oracle, cfg), coords))


@pytest.mark.parametrize("axis_order", [(0, 1, 2), (2, 1, 0), (1, 2, 0)])
@pytest.mark.parametrize("axis_sign", [(1, 1, 1), (-1, 1, 1), (1, -1, -1)])
def test_axis_permutations_checkerboard(oracle, axis_order, axis_sign):
    cfg = F.SparseSubmConvConfig(6, 8, groups=2, axis_order=axis_order, axis_sign=axis_sign)
    c = [(0, x, y, z) for x in range(6) for y in range(5) for z in range(4) if (x + y + z) % 2 == 0]
    coords = np.array(c, np.int32)
    assert np.array_equal(gpu_map(cfg, coords), oracle.build_neighbor_rows(ocfg(oracle, cfg), coords))


@pytest.mark.parametrize("seed", [0, 1])
def test_random_coords_batches_duplicates(oracle, seed):
    rng = np.random.default_rng(seed)
    n = 20000
    c = np.zeros((n, 4), np.int32)
    c[:, 0] = rng.integers(0, 3, n)
    c[:, 1:] = rng.integers(0, 40, (n, 3))
    cfg = F.SparseSubmConvConfig(1, 1)
    assert np.array_equal(gpu_map(cfg, c), oracle.build_neighbor_rows(ocfg(oracle, cfg), c))


def _wide_coords(rng, n, scale_axes):
    base = rng.integers(0, 3000, (n, 3)).astype(np.int64)
    for ax in scale_axes:
        base[: n // 2, ax] *= 4000  # spread half of them wide
    c = np.zeros((n, 4), np.int32)
    c[:, 0] = rng.integers(0, 2, n)
    c[:, 1:] = base.astype(np.int32)
    # plant neighbours (x + 1, same batch) and a few duplicates
    c[n // 2: n // 2 + 100, 1:] = c[n // 2 + 100: n // 2 + 200, 1:] + np.array([1, 0, 0])
    c[n // 2: n // 2 + 100, 0] = c[n // 2 + 100: n // 2 + 200, 0]
    c[n - 20:] = c[n - 40: n - 20]
    return c


@pytest.mark.parametrize("scale_axes,lo,hi", [((0,), 2.0 ** 32, 2.0 ** 64),
                                              ((0, 1, 2), 2.0 ** 64, np.inf)])
def test_wide_coordinates(oracle, scale_axes, lo, hi):
    """Bboxes of more than 2^32 cells use 64-bit keys; beyond 2^64 cells the
    row-only table compares coords directly."""
    c = _wide_coords(np.random.default_rng(3), 4000, scale_axes)
    span = [float(c[:, j].max() - c[:, j].min() + 1) for j in range(4)]
    cells = float(np.prod(np.array(span, dtype=np.float64)))
    assert lo < cells < hi
    cfg = F.SparseSubmConvConfig(1, 1)
    exp = oracle.build_neighbor_rows(ocfg(oracle, cfg), c)
    assert (exp >= 0).sum() > len(c)
    assert np.array_equal(gpu_map(cfg, c), exp)


def test_sparse_bbox_uses_hash_table(oracle):
    """A bbox with far more than 32 cells per row takes the 32-bit-key hash
    table instead of the dense grid."""
    rng = np.random.default_rng(8)
    n = 20000
    c = np.zeros((n, 4), np.int32)
    c[:, 0] = rng.integers(0, 2, n)
    c[:, 1:] = rng.integers(0, 1000, (n, 3))
    c[:2000, 1:] = c[2000:4000, 1:] + rng.integers(-1, 2, (2000, 3))  # planted neighbours
    c[:2000, 0] = c[2000:4000, 0]
    c[-50:] = c[-100:-50]                                              # duplicates
    c[:, 1:] = np.maximum(c[:, 1:], 0)
    cells = float(np.prod([c[:, j].max() - c[:, j].min() + 1 for j in range(4)]))
    assert cells > 32 * n and cells < 2.0 ** 32
    cfg = F.SparseSubmConvConfig(1, 1)
    exp = oracle.build_neighbor_rows(ocfg(oracle, cfg), c)
    assert (exp >= 0).sum() > n + 1000  # centre taps + planted pairs
    assert np.array_equal(gpu_map(cfg, c), exp)


def test_negative_coordinate_is_rejected():
    cfg = F.SparseSubmConvConfig(1, 1)
    c = line_coords(64)
    c[10, 2] = -5
    with pytest.raises(SparseConvError) as e:
        gpu_map(cfg, c)
    assert e.value.status == 6


def test_empty_and_single():
    cfg = F.SparseSubmConvConfig(1, 1)
    assert gpu_map(cfg, np.zeros((0, 4), np.int32)).shape == (0, 27)
    one = gpu_map(cfg, np.array([[0, 5, 5, 5]], np.int32))
    assert one.reshape(-1).tolist() == [-1] * 13 + [0] + [-1] * 13


def test_config1_geometry(oracle):
    coords = synth.config1_coords()
    cfg = F.SparseSubmConvConfig(64, 64)
    got = gpu_map(cfg, coords)
    assert np.array_equal(got, oracle.build_neighbor_rows(ocfg(oracle, cfg), coords))
    assert int((got >= 0).sum()) == 261416


def test_config3_geometry_full_size(oracle):
    coords = synth.config3_coords()
    cfg = F.SparseSubmConvConfig(128, 128)
    got = gpu_map(cfg, coords)
    exp = oracle.build_neighbor_rows(ocfg(oracle, cfg), coords)
    assert np.array_equal(got, exp)
    # rebuild is deterministic
    assert np.array_equal(gpu_map(cfg, coords), got)


def test_shuffled_rows_relabel_consistently(oracle):
    """Order independence at full config-2 size: permuting the coord rows
    permutes and relabels the map."""
    coords = synth.config2_coords()
    cfg = F.SparseSubmConvConfig(1, 1)
    base = gpu_map(cfg, coords)
    perm = np.random.default_rng(0).permutation(len(coords))
    inv = np.empty_like(perm)
    inv[perm] = np.arange(len(perm))
    shuf = gpu_map(cfg, coords[perm])
    relabeled = np.where(base[perm] >= 0, inv[np.maximum(base[perm], 0)], -1)
    assert np.array_equal(shuf, relabeled)


def _map_and_mode(cfg, coords, query_rows=None):
    c = dev(coords.astype(np.int32))
    ws = F.NeighborMapWorkspace(c.device).get(len(coords))
    q = len(coords) if query_rows is None else query_rows
    out = torch.empty((q, F.kernel_rows(cfg)), dtype=torch.int32, device=c.device)
    F.neighbor_map_build_into(cfg, c, out, ws, q)
    F.neighbor_map_check(ws)
    return out.cpu().numpy(), F.neighbor_map_table_mode(ws)


def test_table_modes_by_row_order(oracle):
    """Sorted unique rows take the rank bitmap; any row order that is not
    strictly increasing in (b, x, y, z) takes the dense grid or a hash table;
    every mode gives the oracle's map."""
    cfg = F.SparseSubmConvConfig(1, 1)
    oc = ocfg(oracle, cfg)
    base = synth.config2_coords()
    assert np.array_equal(np.unique(base, axis=0), base)  # argwhere order: sorted, unique
    got, mode = _map_and_mode(cfg, base)
    assert mode == "rank_bitmap"
    exp = oracle.build_neighbor_rows(oc, base)
    assert np.array_equal(got, exp)
    # one swapped pair across a wave and a block boundary of the bbox pass,
    # inside a wave, and at the very end: all fall back to the dense grid
    for i in (63, 255, 4000, len(base) - 2):
        c = base.copy()
        c[[i, i + 1]] = c[[i + 1, i]]
        got, mode = _map_and_mode(cfg, c)
        assert mode == "dense_grid", i
        assert np.array_equal(got, oracle.build_neighbor_rows(oc, c)), i
    # a duplicated row (not strictly increasing) keeps the lowest-row rule
    c = np.insert(base, 1000, base[1000], axis=0)
    got, mode = _map_and_mode(cfg, c)
    assert mode == "dense_grid"
    assert np.array_equal(got, oracle.build_neighbor_rows(oc, c))
    # query rows map against the full sorted set
    got, mode = _map_and_mode(cfg, base, query_rows=777)
    assert mode == "rank_bitmap" and np.array_equal(got, exp[:777])


def _c2s_children(coords, levels, frac, seed):
    """`levels` C2S subdivisions below coords, each child kept with
    probability frac (parent-major, child index ascending: the order the
    decoder's subdivision emits)."""
    rng = np.random.default_rng(seed)
    for _ in range(levels):
        mask = (rng.random((len(coords), 8)) < frac).astype(np.uint8)
        coords = synth.child_expand(coords, mask)
    return coords


@pytest.mark.parametrize("levels", [1, 2, 3])
def test_rank_bitmap_c2s_order(oracle, levels):
    """Children in C2S order below a sorted set are strictly increasing in the
    rank bitmap's key with that many octree levels: they keep the rank bitmap
    (not the dense grid), and the map equals the oracle's -- on the 3x3x3
    path (per-axis key terms) and with a permuted, sign-flipped 3x3x1 kernel
    (the per-entry path).  Two batches, one of them offset so that the root
    bbox starts at odd coordinates."""
    base = synth.config1_coords()[::2]
    shifted = base.copy()
    shifted[:, 0] = 1
    shifted[:, 1:] += (3, 5, 1)
    roots = np.concatenate([base, shifted])                         # sorted: batch 0, then batch 1
    # 45 % of the children kept: the set stays within the bitmap's budget of
    # 512 cells per row (a sparser set legitimately takes a hash table)
    coords = _c2s_children(roots, levels, 0.45, seed=levels)
    for cfg in (F.SparseSubmConvConfig(1, 1),
                F.SparseSubmConvConfig(1, 1, 3, 3, 1, axis_order=(2, 0, 1), axis_sign=(1, -1, 1))):
        c = dev(coords.astype(np.int32))
        ws = F.NeighborMapWorkspace(c.device).get(len(coords))
        out = torch.empty((len(coords), F.kernel_rows(cfg)), dtype=torch.int32, device=c.device)
        F.neighbor_map_build_into(cfg, c, out, ws)
        F.neighbor_map_check(ws)
        assert F.neighbor_map_table_mode(ws) == "rank_bitmap"
        assert F.neighbor_map_rank_levels(ws) == levels
        assert np.array_equal(out.cpu().numpy(), oracle.build_neighbor_rows(ocfg(oracle, cfg), coords))
    # the same children through the device subdivision (the decoder's path)
    cur = dev(roots.astype(np.int32))
    rng = np.random.default_rng(levels)
    for _ in range(levels):
        mask = (rng.random((cur.shape[0], 8)) < 0.45).astype(np.uint8)
        cur, _, _ = F.subdivision_build(cur, mask=dev(mask), with_pairs=False)
    got, mode = _map_and_mode(F.SparseSubmConvConfig(1, 1), cur.cpu().numpy())
    assert mode == "rank_bitmap"
    assert np.array_equal(got, oracle.build_neighbor_rows(ocfg(oracle, F.SparseSubmConvConfig(1, 1)),
                                                          cur.cpu().numpy()))


def test_c2s_order_broken_falls_back(oracle):
    """One pair of children out of C2S order: no octree level fits, the map
    takes the dense grid or a hash table (by density) and still equals the
    oracle's."""
    coords = _c2s_children(synth.config1_coords(), 2, 0.4, seed=5)
    c = coords.copy()
    i = len(c) // 2
    c[[i, i + 1]] = c[[i + 1, i]]
    cfg = F.SparseSubmConvConfig(1, 1)
    got, mode = _map_and_mode(cfg, c)
    assert mode in ("dense_grid", "hash32")
    assert np.array_equal(got, oracle.build_neighbor_rows(ocfg(oracle, cfg), c))
    got, mode = _map_and_mode(cfg, coords)  # the intact order keeps the bitmap
    assert mode == "rank_bitmap"


def test_rank_bitmap_sparse_bbox(oracle):
    """Sorted unique coords over a bbox of more than 32 cells per row (beyond
    the dense grid's budget) still take the rank bitmap; two batches, words
    holding many rows and words holding none."""
    rng = np.random.default_rng(9)
    n = 30000
    c = np.zeros((n, 4), np.int32)
    c[:, 0] = rng.integers(0, 2, n)
    c[:, 1:] = rng.integers(0, 90, (n, 3))
    c[:3000, 1:] = c[3000:6000, 1:] + rng.integers(-1, 2, (3000, 3))
    c[:3000, 0] = c[3000:6000, 0]
    c[5000:5040] = [0, 7, 7, 0] + np.array([[0, 0, 0, z] for z in range(40)])  # 40 consecutive cells
    c[:, 1:] = np.maximum(c[:, 1:], 0)
    c = np.unique(c, axis=0)                                             # sorted, unique
    cells = float(np.prod([c[:, j].max() - c[:, j].min() + 1 for j in range(4)]))
    assert cells > 32 * len(c)
    for kernel in ((3, 3, 3), (5, 5, 5)):
        cfg = F.SparseSubmConvConfig(1, 1, *kernel)
        got, mode = _map_and_mode(cfg, c)
        assert mode == "rank_bitmap"
        assert np.array_equal(got, oracle.build_neighbor_rows(ocfg(oracle, cfg), c))
    # the same rows in another order: a hash table, the same map up to relabelling
    cfg = F.SparseSubmConvConfig(1, 1)
    perm = rng.permutation(len(c))
    got, mode = _map_and_mode(cfg, c[perm])
    assert mode == "hash32"
    assert np.array_equal(got, oracle.build_neighbor_rows(ocfg(oracle, cfg), c[perm]))


def test_config3_shuffled_takes_dense_grid(oracle):
    """Config 3 at full size in a shuffled row order (dense grid) relabels to
    the sorted order's map (rank bitmap)."""
    coords = synth.config3_coords()
    cfg = F.SparseSubmConvConfig(1, 1)
    base, mode = _map_and_mode(cfg, coords)
    assert mode == "rank_bitmap"
    perm = np.random.default_rng(1).permutation(len(coords))
    inv = np.empty_like(perm)
    inv[perm] = np.arange(len(perm))
    shuf, mode = _map_and_mode(cfg, coords[perm])
    assert mode == "dense_grid"
    assert np.array_equal(shuf, np.where(base[perm] >= 0, inv[np.maximum(base[perm], 0)], -1))
    # one swapped pair across the bbox pass's grid stride (1024 blocks x 256 rows)
    i = 1024 * 256 - 1
    sw = np.arange(len(coords))
    sw[[i, i + 1]] = sw[[i + 1, i]]
    got, mode = _map_and_mode(cfg, coords[sw])
    assert mode == "dense_grid"
    assert np.array_equal(got, np.where(base[sw] >= 0, sw[np.maximum(base[sw], 0)], -1))


@pytest.mark.parametrize("kernel", [(3, 3, 3), (3, 3, 1), (1, 1, 1), (2, 2, 2), (5, 5, 5), (1, 3, 5)])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_rank_bitmap_small_dense_bboxes(oracle, kernel, seed):
    """Sorted unique coords in small bboxes (rows at every face and corner of
    the bbox, 32-cell words crossed by neighbour runs, a partial last word,
    a batch holding one voxel): the rank bitmap against the oracle."""
    rng = np.random.default_rng(100 + seed)
    ext = rng.integers(1, 12, 3)
    cells = np.stack(np.meshgrid(*[np.arange(e) for e in ext], indexing="ij"), -1).reshape(-1, 3)
    keep = rng.random(len(cells)) < rng.uniform(0.2, 0.9)
    c = np.zeros((int(keep.sum()) + 1, 4), np.int32)
    c[:-1, 1:] = cells[keep] + rng.integers(0, 5, 3)
    c[-1] = [1, 3, 2, 1]                                       # second batch, one voxel
    c = np.unique(c, axis=0)
    cfg = F.SparseSubmConvConfig(1, 1, *kernel)
    got, mode = _map_and_mode(cfg, c)
    assert mode == "rank_bitmap"
    assert np.array_equal(got, oracle.build_neighbor_rows(ocfg(oracle, cfg), c))


@pytest.mark.parametrize("kernel", [(3, 3, 3), (3, 3, 1), (1, 1, 1), (2, 2, 2), (1, 3, 5), (5, 5, 5)])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_dense_grid_sweep_shuffled(oracle, kernel, seed):
    """Unique coords in a random row order take the dense grid, whose query
    sweeps the grid's cells (64 cells of a z line per wave unit) and writes
    each row's map row through LDS: z extents below, at and across 64 cells,
    several batches, every axis order and sign draw, and partial queries on
    both sides of the sweep's half-the-rows threshold, against the oracle.
    K = 125 exceeds the sweep's 32 entries and takes the per-entry query."""
    rng = np.random.default_rng(200 + seed)
    ext = np.array([rng.integers(1, 9), rng.integers(1, 9), [1, 64, 97][seed]])
    cells = np.stack(np.meshgrid(*[np.arange(e) for e in ext], indexing="ij"), -1).reshape(-1, 3)
    parts = []
    for b in range(1 + seed):
        keep = rng.random(len(cells)) < rng.uniform(0.2, 0.9)
        c = np.zeros((int(keep.sum()), 4), np.int32)
        c[:, 0] = 2 * b
        c[:, 1:] = cells[keep] + rng.integers(0, 4, 3)
        parts.append(c)
    c = np.concatenate(parts)
    c = c[rng.permutation(len(c))]
    order = tuple(int(v) for v in rng.permutation(3))
    sign = tuple(int(v) for v in rng.choice([-1, 1], 3))
    cfg = F.SparseSubmConvConfig(1, 1, *kernel, axis_order=order, axis_sign=sign)
    exp = oracle.build_neighbor_rows(ocfg(oracle, cfg), c)
    got, mode = _map_and_mode(cfg, c)
    assert mode == "dense_grid"
    assert np.array_equal(got, exp)
    for q in (len(c) * 3 // 5, len(c) // 3, 1):
        got, mode = _map_and_mode(cfg, c, query_rows=q)
        assert mode == "dense_grid"
        assert np.array_equal(got, exp[:q]), q


def test_dense_grid_sweep_duplicates_fall_back(oracle):
    """Shuffled coords with duplicated cells: the grid names each cell's
    lowest row, so the query maps row by row and every duplicate row gets
    its own map row."""
    rng = np.random.default_rng(5)
    c = np.zeros((30000, 4), np.int32)
    c[:, 1:] = rng.integers(0, 48, (30000, 3))
    assert len(np.unique(c, axis=0)) < len(c)
    cfg = F.SparseSubmConvConfig(1, 1)
    got, mode = _map_and_mode(cfg, c)
    assert mode == "dense_grid"
    assert np.array_equal(got, oracle.build_neighbor_rows(ocfg(oracle, cfg), c))

"""Seeded synthetic workloads for the sparse-conv path (coords, features, weights).

The geometries realise the workload descriptions of the benchmark configs; the
reference has no generator of its own for them.  Conventions:

* a voxel's centre is ``coord + 0.5`` (reference convention,
  crates/burn_trellis/src/staged_pipeline_decode.rs:2392);
* rows come out in lexicographic (batch, x, y, z) order, batch 0, unique;
* coords are ``int32 [N, 4]`` (batch, x, y, z), as the device path takes them
  (crates/burn_flex_gmm/src/wgpu/neighbor.rs:252-263).

Exact sizes (checked by tests/test_synth.py):
    config 1: N = 14,648, P = 261,416 valid (row, offset) pairs
    config 3: N = 1,040,679 (seed 13)
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def _argwhere_coords(mask: np.ndarray, x0: int = 0) -> np.ndarray:
    idx = np.argwhere(mask).astype(np.int32)
    if x0:
        idx[:, 0] += x0
    out = np.zeros((idx.shape[0], 4), dtype=np.int32)
    out[:, 1:] = idx
    return out


def _centres(lo: int, hi: int) -> np.ndarray:
    return np.arange(lo, hi, dtype=np.float64) + 0.5


def sphere_shell_coords(grid: int = 64, radius: float = 24.0, half_width: float = 1.0,
                        centre=(32.0, 32.0, 32.0)) -> np.ndarray:
    """Config 1: voxels whose centre lies within ``half_width`` of the sphere."""
    g = _centres(0, grid)
    X, Y, Z = np.meshgrid(g - centre[0], g - centre[1], g - centre[2], indexing="ij")
    d = np.sqrt(X * X + Y * Y + Z * Z)
    return _argwhere_coords(np.abs(d - radius) <= half_width)


def config1_coords() -> np.ndarray:
    return sphere_shell_coords(64, 24.0, 1.0, (32.0, 32.0, 32.0))


@dataclass(frozen=True)
class ShellCubeGeometry:
    """Config 2: union of a sphere shell (|d - r| <= 1.5) and a one-voxel cube
    surface layer (|Chebyshev distance - side/2| <= 0.5), both centres jittered
    by U(-4, 4) per axis from a seeded generator."""

    grid: int = 128
    radius: float = 50.0
    shell_half_width: float = 1.5
    cube_side: float = 60.0
    cube_offset: float = 20.0
    cube_half_width: float = 0.5
    jitter: float = 4.0
    seed: int = 2

    def centres(self):
        rng = np.random.default_rng(self.seed)
        js = rng.uniform(-self.jitter, self.jitter, 3)
        jc = rng.uniform(-self.jitter, self.jitter, 3)
        sphere_c = self.grid / 2.0 + js
        cube_c = self.cube_offset + self.cube_side / 2.0 + jc
        return sphere_c, cube_c

    def distance_fields(self, lo: int, hi: int):
        """Signed distances (sphere shell, cube surface) for x in [lo, hi)."""
        sc, cc = self.centres()
        g = _centres(0, self.grid)
        gx = _centres(lo, hi)
        X, Y, Z = np.meshgrid(gx, g, g, indexing="ij")
        d_s = np.sqrt((X - sc[0]) ** 2 + (Y - sc[1]) ** 2 + (Z - sc[2]) ** 2) - self.radius
        cheb = np.maximum(np.maximum(np.abs(X - cc[0]), np.abs(Y - cc[1])), np.abs(Z - cc[2]))
        d_c = cheb - self.cube_side / 2.0
        return d_s, d_c

    def coords(self) -> np.ndarray:
        parts = []
        for lo in range(0, self.grid, 32):
            hi = min(self.grid, lo + 32)
            d_s, d_c = self.distance_fields(lo, hi)
            m = (np.abs(d_s) <= self.shell_half_width) | (np.abs(d_c) <= self.cube_half_width)
            parts.append(_argwhere_coords(m, lo))
        return np.concatenate(parts, 0)

    def surface_distance(self, pts: np.ndarray) -> np.ndarray:
        """Unsigned distance (grid units) from points [M,3] to the union of the
        sphere surface and the cube surface."""
        sc, cc = self.centres()
        d_s = np.abs(np.sqrt(((pts - sc) ** 2).sum(1)) - self.radius)
        q = np.abs(pts - cc) - self.cube_side / 2.0
        outside = np.sqrt((np.maximum(q, 0.0) ** 2).sum(1))
        inside = np.minimum(q.max(1), 0.0)
        d_c = np.abs(outside + inside)
        return np.minimum(d_s, d_c)


def config2_coords(seed: int = 2) -> np.ndarray:
    return ShellCubeGeometry(seed=seed).coords()


@dataclass(frozen=True)
class EllipsoidShellGeometry:
    """Config 3 (and config 5 scaled): union over 8 seeded ellipsoids of the
    shell |d_i| <= 1.5, with d_i the first-order distance (F - 1) * F / |grad
    of the normalised radius|, F = |(p - c_i) / a_i|.  Semi-axes ~ U(20, 90)
    (scaled by grid/256), centres ~ U(a + 2, grid - a - 2) per axis."""

    grid: int = 256
    n_ellipsoids: int = 8
    axis_lo: float = 20.0
    axis_hi: float = 90.0
    half_width: float = 1.5
    seed: int = 13

    def params(self):
        rng = np.random.default_rng(self.seed)
        s = self.grid / 256.0
        a = rng.uniform(self.axis_lo * s, self.axis_hi * s, (self.n_ellipsoids, 3))
        c = np.stack([rng.uniform(a[:, j] + 2.0, self.grid - a[:, j] - 2.0) for j in range(3)], 1)
        return a, c

    def coords(self, slab: int = 16) -> np.ndarray:
        a, c = self.params()
        g = _centres(0, self.grid)
        parts = []
        for lo in range(0, self.grid, slab):
            hi = min(self.grid, lo + slab)
            X, Y, Z = np.meshgrid(_centres(lo, hi), g, g, indexing="ij")
            m = np.zeros(X.shape, dtype=bool)
            for i in range(self.n_ellipsoids):
                u = (X - c[i, 0]) / a[i, 0]
                v = (Y - c[i, 1]) / a[i, 1]
                w = (Z - c[i, 2]) / a[i, 2]
                F = np.sqrt(u * u + v * v + w * w)
                gn = np.sqrt((u / a[i, 0]) ** 2 + (v / a[i, 1]) ** 2 + (w / a[i, 2]) ** 2)
                d = (F - 1.0) * F / np.maximum(gn, 1e-12)
                m |= np.abs(d) <= self.half_width
            parts.append(_argwhere_coords(m, lo))
        return np.concatenate(parts, 0)


def config3_coords(seed: int = 13) -> np.ndarray:
    return EllipsoidShellGeometry(seed=seed).coords()


def config3_spread_coords(seed: int = 13, gap: int = 1024, shuffle_seed: int = 11) -> np.ndarray:
    """Config 3's rows with its eight octants (halves of the 256^3 box per
    axis) moved gap cells apart along x, in a random row order: the same
    local neighbourhoods (but across the cuts) in a bounding box far above the
    dense grid's budget -- the map's hash-table mode."""
    c = config3_coords(seed).copy()
    octant = ((c[:, 1] >= 128).astype(np.int32) | ((c[:, 2] >= 128).astype(np.int32) << 1) |
              ((c[:, 3] >= 128).astype(np.int32) << 2))
    c[:, 1] += octant * gap
    return c[np.random.default_rng(shuffle_seed).permutation(len(c))]


def ellipsoid_shell_distance(geom: EllipsoidShellGeometry, pts: np.ndarray) -> np.ndarray:
    """min_i |d_i(p)| over the union's ellipsoids, the first-order distance the
    shell set uses, at arbitrary points (grid units of ``geom``)."""
    a, c = geom.params()
    p = np.asarray(pts, dtype=np.float64)
    best = np.full(len(p), np.inf)
    for i in range(geom.n_ellipsoids):
        u = (p[:, 0] - c[i, 0]) / a[i, 0]
        v = (p[:, 1] - c[i, 1]) / a[i, 1]
        w = (p[:, 2] - c[i, 2]) / a[i, 2]
        F = np.sqrt(u * u + v * v + w * w)
        gn = np.sqrt((u / a[i, 0]) ** 2 + (v / a[i, 1]) ** 2 + (w / a[i, 2]) ** 2)
        best = np.minimum(best, np.abs((F - 1.0) * F / np.maximum(gn, 1e-12)))
    return best


def child_expand(parent_coords: np.ndarray, mask: np.ndarray) -> np.ndarray:
    """Children of the masked (parent, c) pairs in argwhere order (parent-major,
    c ascending): (b, 2x + (c&1), 2y + (c>>1&1), 2z + (c>>2&1))."""
    pairs = np.argwhere(mask)
    p = parent_coords[pairs[:, 0]].astype(np.int64)
    c = pairs[:, 1]
    out = np.empty((len(pairs), 4), dtype=np.int32)
    out[:, 0] = p[:, 0]
    out[:, 1] = 2 * p[:, 1] + (c & 1)
    out[:, 2] = 2 * p[:, 2] + ((c >> 1) & 1)
    out[:, 3] = 2 * p[:, 3] + ((c >> 2) & 1)
    return out


def config5_stack_inputs(seed: int = 13, start_grid: int = 64, stages: int = 3):
    """Config 5 geometry: the config-3 ellipsoid union scaled to each
    resolution.  Returns the start coords (the shell set at ``start_grid``)
    and, per stage, the [P, 8] u8 mask of the children of the stage's parents
    that lie on the shell at twice the resolution (child centre within the
    shell's half-width, in child grid units)."""
    coords = EllipsoidShellGeometry(grid=start_grid, seed=seed).coords()
    masks = []
    parents = coords
    for s in range(stages):
        child = EllipsoidShellGeometry(grid=start_grid * 2 ** (s + 1), seed=seed)
        mask = np.zeros((len(parents), 8), dtype=np.uint8)
        base = 2.0 * parents[:, 1:4].astype(np.float64) + 0.5
        for c in range(8):
            off = np.array([c & 1, (c >> 1) & 1, (c >> 2) & 1], dtype=np.float64)
            mask[:, c] = ellipsoid_shell_distance(child, base + off) <= child.half_width
        masks.append(mask)
        parents = child_expand(parents, mask)
    return coords, masks


def subdivision_mask_near_surface(parent_coords: np.ndarray, geom: ShellCubeGeometry,
                                  max_distance: float = 1.0) -> np.ndarray:
    """Config 4: [P, 8] u8 mask of children whose centre lies within
    ``max_distance`` (parent grid units) of the parent-resolution surface.
    Child c of parent p has centre p + ((c&1), (c>>1&1), (c>>2&1)) * 0.5 + 0.25."""
    p = parent_coords[:, 1:4].astype(np.float64)
    mask = np.zeros((p.shape[0], 8), dtype=np.uint8)
    for c in range(8):
        off = np.array([(c & 1), (c >> 1) & 1, (c >> 2) & 1], dtype=np.float64) * 0.5 + 0.25
        mask[:, c] = geom.surface_distance(p + off) <= max_distance
    return mask


def normal_f32(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    return (rng.standard_normal(shape, dtype=np.float64) * std).astype(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round f32 -> bf16 with the reference's rule (crates/burn_flex_gmm/src/wgpu.rs:63-66)
    and return the upper 16 bits as uint16."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return (r >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def conv_weight(rng: np.random.Generator, cout: int, k: int, cin: int, std: float) -> np.ndarray:
    """Weights [Cout, K, Cin] (the reference's [Cout, KD, KH, KW, Cin_g] with
    the three kernel axes flattened, crates/burn_flex_gmm/src/wgpu/sparse_conv.rs:453-465)."""
    return normal_f32(rng, (cout, k, cin), std)


def int8_weight(rng: np.random.Generator, cout: int, k: int, cin: int):
    """Per-output-channel symmetric int8 weights: q ~ U{-127..127}, scale ~ U(0.5, 1.5)/127."""
    q = rng.integers(-127, 128, size=(cout, k, cin), dtype=np.int8)
    scale = (rng.uniform(0.5, 1.5, cout) / 127.0).astype(np.float32)
    return q, scale

"""Row samples for the full-size parity checks.

A sample always holds the rows of the tiles where a tiling bug would show:
the first and the last (partial) 256-row tile of the conv plan's order, every
tile whose halo overflowed to the direct kernel, and the first and last query
rows; the rest is drawn at random up to ``k`` rows."""
import numpy as np


def tile_rows(plan, tiles):
    """Query rows of the given plan tiles (padding dropped)."""
    h = plan.to_host()
    order = h["order"]
    rows = order[np.asarray(tiles, dtype=np.int64)].ravel() if len(tiles) else np.zeros(0, np.int32)
    return rows[rows >= 0]


def sample_rows(n, rng, k=2000, plan=None, extra=()):
    """About ``k`` distinct rows of [0, n), sorted, covering the first / last /
    overflow tiles of ``plan`` (if given) and the rows in ``extra``."""
    must = [np.array([0, n - 1], np.int64), np.asarray(extra, np.int64)]
    if plan is not None:
        h = plan.to_host()
        nt = h["n_tiles"]
        tiles = sorted({0, nt - 1, *h["overflow"].tolist()[:8]})
        must.append(tile_rows(plan, tiles).astype(np.int64))
    must = np.unique(np.concatenate(must))
    must = must[(must >= 0) & (must < n)]
    pool = np.setdiff1d(np.arange(n, dtype=np.int64), must, assume_unique=True)
    left = min(max(0, k - len(must)), len(pool))
    rand = rng.choice(pool, size=left, replace=False) if left else np.zeros(0, np.int64)
    return np.unique(np.concatenate([must, rand]))

"""Seeded synthetic CSR graphs for the parity tests (host numpy)."""

import numpy as np


def skewed_csr(seed, n_dst, n_src, mean_deg=6, hubs=(), empty_frac=0.1, hot_src=None,
               hot_frac=0.0):
    """Random destination-row CSR with sorted neighbour lists.

    hubs: degrees forced on the first len(hubs) rows (split rows);
    hot_src: a source id that receives hot_frac of all edges (a transposed hub).
    """
    rng = np.random.default_rng(seed)
    deg = rng.poisson(mean_deg, size=n_dst)
    deg[rng.random(n_dst) < empty_frac] = 0
    for r, d in enumerate(hubs):
        deg[r] = d
    row_ptr = np.zeros(n_dst + 1, dtype=np.int64)
    np.cumsum(deg, out=row_ptr[1:])
    E = int(row_ptr[-1])
    col = rng.integers(0, n_src, size=E)
    if hot_src is not None and hot_frac > 0:
        col[rng.random(E) < hot_frac] = hot_src
    for i in range(n_dst):
        col[row_ptr[i]:row_ptr[i + 1]].sort()
    return row_ptr, col.astype(np.int64)


def rmat_csr(seed, scale, edge_factor=16, probs=(0.57, 0.19, 0.19, 0.05)):
    """R-MAT graph (Chakrabarti et al. 2004): each of edge_factor * 2**scale
    tuples picks one quadrant per level; duplicates removed; the first
    coordinate is the destination row.  Returns a dst-row CSR (sorted cols)."""
    rng = np.random.default_rng(seed)
    n = 1 << scale
    m = edge_factor * n
    a, b, c, _ = probs
    row = np.zeros(m, dtype=np.int64)
    col = np.zeros(m, dtype=np.int64)
    for level in range(scale):
        r = rng.random(m)
        down = r >= a + b                       # quadrants c, d: row bit 1
        right = ((r >= a) & (r < a + b)) | (r >= a + b + c)   # quadrants b, d
        row |= down.astype(np.int64) << level
        col |= right.astype(np.int64) << level
    keys = np.unique(row * n + col)
    row, col = keys // n, keys % n
    row_ptr = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(np.bincount(row, minlength=n), out=row_ptr[1:])
    return row_ptr, col

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

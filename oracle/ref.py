"""CPU restatement (numpy, fp64) of the reference's CSR message-passing path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as a
checker or a timed CPU baseline; the product (``tiga-lang_amd/``) never does.

Every function cites the reference code it restates.  Pinning (what checks
this restatement independently of retyping it) is listed per function; see
tests/test_oracle.py for the checks themselves.
"""

from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# Graph indexing


def validate_csr(row_ptr, col_idx, num_src):
    """Graph._validate_csr_values (python/tiga/interop/torch/graph.py:604-617).

    Pinned by: error-message cases in tests/test_host.py (same inputs raise in
    the product's Graph.from_csr(validate="full")).
    """
    row_ptr = np.asarray(row_ptr)
    col_idx = np.asarray(col_idx)
    if int(row_ptr[0]) != 0:
        raise ValueError("row_ptr[0] must be zero")
    if int(row_ptr[-1]) != col_idx.size:
        raise ValueError("row_ptr[-1] must equal the number of edges")
    if np.any(row_ptr[1:] < row_ptr[:-1]):
        raise ValueError("row_ptr must be monotonic")
    if col_idx.size and (col_idx.min() < 0 or col_idx.max() >= num_src):
        raise ValueError("col_idx contains an out-of-range source index")


def destination_index(row_ptr):
    """Graph.destination_index (interop/torch/graph.py:1212-1222):
    repeat_interleave(arange(num_dst), degree).

    Pinned by: brute-force loop on small graphs (tests/test_oracle.py).
    """
    row_ptr = np.asarray(row_ptr, dtype=np.int64)
    return np.repeat(np.arange(row_ptr.size - 1, dtype=np.int64), np.diff(row_ptr))


def transpose(row_ptr, col_idx, num_src):
    """Graph.transpose -> from_coo (interop/torch/graph.py:675-685, 193-231):
    stable argsort of col_idx, bincount, cumsum.  Returns (row_ptr_t, col_t, perm)
    with perm = argsort(col_idx, stable=True) and col_t = destination[perm].

    Pinned by: brute force (per-source scan in edge order) and the round trip
    transpose(transpose(G)) == G (tests/test_oracle.py).
    """
    col_idx = np.asarray(col_idx, dtype=np.int64)
    dst = destination_index(row_ptr)
    perm = np.argsort(col_idx, kind="stable")
    counts = np.bincount(col_idx, minlength=num_src)
    row_ptr_t = np.zeros(num_src + 1, dtype=np.int64)
    np.cumsum(counts, out=row_ptr_t[1:])
    return row_ptr_t, dst[perm], perm


def from_coo(src, dst, num_src=None, num_dst=None):
    """Graph.from_coo (interop/torch/graph.py:193-231): stable argsort of dst,
    col_idx = src[order], row_ptr = [0, cumsum(bincount(dst))].

    Pinned by: brute force (per destination, edges in input order) and the
    round trip from_coo(destination_index, col_idx) == the CSR it came from
    (tests/test_oracle.py).
    """
    src = np.asarray(src, dtype=np.int64)
    dst = np.asarray(dst, dtype=np.int64)
    if num_src is None:
        num_src = int(src.max()) + 1 if src.size else 0
    if num_dst is None:
        num_dst = int(dst.max()) + 1 if dst.size else 0
    order = np.argsort(dst, kind="stable")
    counts = np.bincount(dst, minlength=num_dst)
    row_ptr = np.zeros(num_dst + 1, dtype=np.int64)
    np.cumsum(counts, out=row_ptr[1:])
    return row_ptr, src[order], num_src


def cu_seqlens_csr(cu_seqlens, causal=True):
    """Graph.cu_seqlens (interop/torch/graph.py:260-294): row i of sequence k
    gathers [s_k, i] (causal) or [s_k, s_{k+1}).

    Pinned by: brute force over (sequence, position) and the reference test's
    equality cat([triangular(L)]) == cu_seqlens(cumsum(L))
    (tests/python/test_graph_constructors.py:56-110).
    """
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    rows, cols = [0], []
    for k in range(cu.size - 1):
        s, e = int(cu[k]), int(cu[k + 1])
        for i in range(s, e):
            end = i + 1 if causal else e
            cols.extend(range(s, end))
            rows.append(rows[-1] + (end - s))
    return np.asarray(rows, dtype=np.int64), np.asarray(cols, dtype=np.int64)


def cat_csr(blocks):
    """Graph.cat (interop/torch/graph.py:297-340): block-diagonal packing.
    blocks = [(row_ptr, col_idx, num_src), ...]."""
    rows = [np.zeros(1, dtype=np.int64)]
    cols = []
    e_off = s_off = 0
    for row_ptr, col_idx, num_src in blocks:
        row_ptr = np.asarray(row_ptr, dtype=np.int64)
        cols.append(np.asarray(col_idx, dtype=np.int64) + s_off)
        rows.append(row_ptr[1:] + e_off)
        e_off += int(row_ptr[-1])
        s_off += num_src
    return np.concatenate(rows), (np.concatenate(cols) if cols else np.zeros(0, np.int64)), s_off


# ---------------------------------------------------------------------------
# Row partition (the MI355X device plan) and the reference planner


def degree_bins(row_ptr, upper_bounds):
    """Stable degree-bin partition: bin b = rows with ub[b-1] < deg <= ub[b]
    (last bin takes everything above), ascending row ids inside a bin.
    Restates the reference worklist ABI (include/tiga/Dialect/Task/TaskOps.td:
    63-82; histogram/prefix/scatter Translate.cpp:4043-4187) with the scatter
    made order-preserving.  Returns (rows, offsets[n_bins+1]).

    Pinned by: sorted-membership equality with a brute-force degree filter.
    """
    deg = np.diff(np.asarray(row_ptr, dtype=np.int64))
    ub = list(upper_bounds)
    bins = np.zeros(deg.size, dtype=np.int64)
    for b in range(len(ub) - 1):
        bins += deg > ub[b]
    order = np.argsort(bins, kind="stable")
    counts = np.bincount(bins, minlength=len(ub))
    offsets = np.zeros(len(ub) + 1, dtype=np.int64)
    np.cumsum(counts, out=offsets[1:])
    return order.astype(np.int64), offsets


def row_plan(row_ptr, wave_max, chunk_edges):
    """The partition consumed by the sparse kernels: (rows, n_empty, n_wave,
    n_split, chunk_offsets) with bins {0, wave_max, inf} and
    chunk_offsets = exclusive prefix of ceil(deg / chunk_edges) over split rows
    (the reference's row split uses 64-edge partials, PlanSplitRows.cpp:136-147)."""
    rows, off = degree_bins(row_ptr, [0, wave_max, 1 << 62])
    deg = np.diff(np.asarray(row_ptr, dtype=np.int64))
    split = rows[off[2]:off[3]]
    per = (deg[split] + chunk_edges - 1) // chunk_edges
    chunk_offsets = np.zeros(split.size + 1, dtype=np.int64)
    np.cumsum(per, out=chunk_offsets[1:])
    return rows, int(off[1] - off[0]), int(off[2] - off[1]), int(off[3] - off[2]), chunk_offsets


# ---------------------------------------------------------------------------
# Sum reducer


def sum_fwd(row_ptr, col_idx, x, w=None):
    """reduce_sum (interop/torch/reducer_oracle.py:44-57) of message w_e * x[col_e]:
    out = zeros.index_add_(0, dst, msg).  fp64.

    Pinned by: the README known answer (README.md:91-111) and brute-force
    per-row loops (tests/test_oracle.py).
    """
    x = np.asarray(x, dtype=np.float64)
    dst = destination_index(row_ptr)
    col_idx = np.asarray(col_idx, dtype=np.int64)
    msg = x[col_idx]
    if w is not None:
        wv = np.asarray(w, dtype=np.float64).reshape(-1)
        msg = msg * wv.reshape(-1, *([1] * (x.ndim - 1)))
    out = np.zeros((np.asarray(row_ptr).size - 1, *x.shape[1:]), dtype=np.float64)
    np.add.at(out, dst, msg)
    return out


def sum_bwd(row_ptr, col_idx, x, w, dout):
    """Adjoint of sum_fwd (the reference replays index_add in Torch autograd,
    interop/torch/message_passing.py:387-409): dx[j] = sum_{e: col=j} w_e dout[dst_e],
    dw[e] = <dout[dst_e], x[col_e]>.

    Pinned by: README known answer dx=[7,10,3], dw=[1,3,2,1,2] and central
    finite differences (tests/test_oracle.py).
    """
    x = np.asarray(x, dtype=np.float64)
    dout = np.asarray(dout, dtype=np.float64)
    dst = destination_index(row_ptr)
    col_idx = np.asarray(col_idx, dtype=np.int64)
    E = col_idx.size
    wv = np.ones(E) if w is None else np.asarray(w, dtype=np.float64).reshape(-1)
    g = dout[dst]
    dx = np.zeros_like(x)
    np.add.at(dx, col_idx, g * wv.reshape(-1, *([1] * (x.ndim - 1))))
    dw = (g * x[col_idx]).reshape(E, -1).sum(axis=1)
    return dx, dw


# ---------------------------------------------------------------------------
# Online softmax (segment softmax over destination rows, per lane)


def segment_softmax(row_ptr, score, value):
    """reduce_online_softmax (interop/torch/reducer_oracle.py:60-137), fp64:
    per (row, lane) max shift, exp, sum, weighted sum; empty row -> 0.
    score [E, *lanes], value [E, *lanes, *payload].  Returns (out, lse) with
    lse[row, lanes] = log sum exp(score) (-inf for an empty row).

    Pinned by: the reference known answer at scores ~1000
    (tests/python/test_message_passing_autograd.py:318-351), the multi-head
    empty-row case vs per-row softmax (tests/python/test_reference.py:416-444)
    and the closed form for a single edge (alpha = 1).
    """
    score = np.asarray(score, dtype=np.float64)
    value = np.asarray(value, dtype=np.float64)
    dst = destination_index(row_ptr)
    n = np.asarray(row_ptr).size - 1
    lanes = score.shape[1:]
    payload = value.ndim - score.ndim
    m = np.full((n, *lanes), -np.inf)
    np.maximum.at(m, dst, score)
    p = np.exp(score - m[dst])
    den = np.zeros((n, *lanes))
    np.add.at(den, dst, p)
    num = np.zeros((n, *value.shape[1:]))
    np.add.at(num, dst, value * p.reshape(*p.shape, *([1] * payload)))
    d = den.reshape(*den.shape, *([1] * payload))
    with np.errstate(invalid="ignore", divide="ignore"):
        out = np.where(d > 0, num / np.where(d > 0, d, 1.0), 0.0)
        lse = np.where(den > 0, m + np.log(np.where(den > 0, den, 1.0)), -np.inf)
    return out, lse


def segment_softmax_bwd(row_ptr, score, value, dout):
    """Adjoint of segment_softmax: alpha = softmax, d_value = alpha * dout,
    d_score = alpha (<dout, value> - <dout, out>).  (Same Jacobian the
    reference's fused nn-attention backward applies,
    python/tiga/compiler/edge_nn_attention.py:569-575.)

    Pinned by: the known answer dscore/dvalue of the ~1000-score case and
    central finite differences.
    """
    score = np.asarray(score, dtype=np.float64)
    value = np.asarray(value, dtype=np.float64)
    dout = np.asarray(dout, dtype=np.float64)
    dst = destination_index(row_ptr)
    out, lse = segment_softmax(row_ptr, score, value)
    payload = value.ndim - score.ndim
    alpha = np.exp(score - lse[dst])
    a = alpha.reshape(*alpha.shape, *([1] * payload))
    g = dout[dst]
    dvalue = a * g
    axes = tuple(range(score.ndim, value.ndim))
    dalpha = (g * value).sum(axis=axes) if axes else g * value
    delta = (g * out[dst]).sum(axis=axes) if axes else g * out[dst]
    dscore = alpha * (dalpha - delta)
    return dscore, dvalue


# ---------------------------------------------------------------------------
# GAT additive attention


def _leaky(z, slope):
    return np.where(z > 0, z, z * slope)


def gat_scores(row_ptr, col_idx, h, a_src, a_dst, slope, h_dst=None):
    """z_e = sum_d h[j]*a_src + sum_d h_dst[i]*a_dst, s = LeakyReLU(z): the
    edge() (src.h*a_src).sum(-1) + (dst.h*a_dst).sum(-1) evaluated per edge as
    in _evaluate_reference (interop/torch/message_passing.py:2848-2894).
    h_dst=None: one feature tensor for both roles (homogeneous relation)."""
    h = np.asarray(h, dtype=np.float64)
    hd = h if h_dst is None else np.asarray(h_dst, dtype=np.float64)
    a_src = np.asarray(a_src, dtype=np.float64)
    a_dst = np.asarray(a_dst, dtype=np.float64)
    dst = destination_index(row_ptr)
    col_idx = np.asarray(col_idx, dtype=np.int64)
    ss = (h * a_src).sum(-1)
    sd = (hd * a_dst).sum(-1)
    z = ss[col_idx] + sd[dst]
    return z, _leaky(z, slope)


def gat_fwd(row_ptr, col_idx, h, a_src, a_dst, slope, h_dst=None):
    """GAT forward = segment_softmax(score = LeakyReLU(z), value = h[col]);
    h holds the source features, h_dst (default: h) the destinations'.

    Pinned by: reduction to segment_softmax (itself pinned) and the closed
    form a_src = a_dst = 0 -> uniform mean of neighbours."""
    _, s = gat_scores(row_ptr, col_idx, h, a_src, a_dst, slope, h_dst)
    h = np.asarray(h, dtype=np.float64)
    return segment_softmax(row_ptr, s, h[np.asarray(col_idx, dtype=np.int64)])


def gat_bwd_bipartite(row_ptr, col_idx, h_src, h_dst, a_src, a_dst, slope, dout):
    """Gradients (dh_src, dh_dst, da_src, da_dst) of gat_fwd with two feature
    tensors (LeakyReLU'(0) = slope, as torch.nn.functional.leaky_relu's
    backward).

    Pinned by: central finite differences on small bipartite graphs, and
    dh_src + dh_dst == gat_bwd's dh when both tensors are one
    (tests/test_oracle.py)."""
    hs = np.asarray(h_src, dtype=np.float64)
    hd = np.asarray(h_dst, dtype=np.float64)
    col_idx = np.asarray(col_idx, dtype=np.int64)
    dst = destination_index(row_ptr)
    z, s = gat_scores(row_ptr, col_idx, hs, a_src, a_dst, slope, hd)
    dscore, dvalue = segment_softmax_bwd(row_ptr, s, hs[col_idx], dout)
    dz = np.where(z > 0, dscore, dscore * slope)
    a_src = np.asarray(a_src, dtype=np.float64)
    a_dst = np.asarray(a_dst, dtype=np.float64)
    dhs = np.zeros_like(hs)
    dhd = np.zeros_like(hd)
    np.add.at(dhs, col_idx, dvalue + dz[..., None] * a_src)
    np.add.at(dhd, dst, dz[..., None] * a_dst)
    da_src = (dz[..., None] * hs[col_idx]).sum(0)
    da_dst = (dz[..., None] * hd[dst]).sum(0)
    return dhs, dhd, da_src, da_dst


def gat_bwd(row_ptr, col_idx, h, a_src, a_dst, slope, dout):
    """Gradients of gat_fwd w.r.t. h, a_src, a_dst for one feature tensor
    (both roles' terms summed into dh).

    Pinned by: central finite differences on small graphs (tests/test_oracle.py).
    """
    dhs, dhd, da_src, da_dst = gat_bwd_bipartite(row_ptr, col_idx, h, h, a_src, a_dst, slope,
                                                 dout)
    return dhs + dhd, da_src, da_dst


# ---------------------------------------------------------------------------
# Dot-product attention with optional per-edge bias


def dot_fwd(row_ptr, col_idx, q, k, v, scale, bias=None):
    """score = (k[j]*q[i]).sum(-1)*scale (+bias[e]), value = v[j], segment softmax.
    fp64 math (the 2e-2 bf16 tolerance absorbs the reference eager path's bf16
    rounding of q*k, interop/torch/reducer_oracle.py:22-41, 87-91, 137)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    col_idx = np.asarray(col_idx, dtype=np.int64)
    dst = destination_index(row_ptr)
    s = (k[col_idx] * q[dst]).sum(-1) * scale
    if bias is not None:
        s = s + np.asarray(bias, dtype=np.float64)
    return segment_softmax(row_ptr, s, v[col_idx])


def dot_bwd(row_ptr, col_idx, q, k, v, scale, bias, dout):
    """Gradients (dq, dk, dv, dbias) of dot_fwd.  Pinned by finite differences."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    col_idx = np.asarray(col_idx, dtype=np.int64)
    dst = destination_index(row_ptr)
    s = (k[col_idx] * q[dst]).sum(-1) * scale
    if bias is not None:
        s = s + np.asarray(bias, dtype=np.float64)
    dscore, dvalue = segment_softmax_bwd(row_ptr, s, v[col_idx], dout)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    np.add.at(dq, dst, dscore[..., None] * k[col_idx] * scale)
    np.add.at(dk, col_idx, dscore[..., None] * q[dst] * scale)
    np.add.at(dv, col_idx, dvalue)
    return dq, dk, dv, dscore


# ---------------------------------------------------------------------------
# Varlen causal attention (dense per sequence)


def _block_scores(qs, ks, scale, causal, r0=0, c0=0):
    """scale * q.k per head as [H, rows, cols], -inf where the boundary
    excludes the pair (key index > query index when causal)."""
    sc = np.einsum("ihd,jhd->hij", qs, ks) * scale
    if causal:
        rows = np.arange(qs.shape[0])[:, None] + r0
        cols = np.arange(ks.shape[0])[None, :] + c0
        sc = np.where((cols <= rows)[None], sc, -np.inf)
    return sc


def block_attention_fwd(cu_q, cu_k, q, k, v, scale, causal):
    """Softmax attention per block of a block-diagonal relation, fp64: block b
    relates queries [cu_q[b], cu_q[b+1]) to keys [cu_k[b], cu_k[b+1]), all
    pairs or key <= query (causal, square blocks).  Covers Graph.cu_seqlens
    (interop/torch/graph.py:260-294), Graph.dense and Graph.triangular
    (:535-592) under the dot-product edge function and online softmax
    (reducer_oracle.py:60-137).  A query with no keys gets 0 and lse -inf.

    Pinned by: equality with dot_fwd on the materialized CSR of the same
    relation and with the reference's per-sequence SDPA property
    (tests/python/test_attention_examples.py:25-72), tests/test_oracle.py.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    out = np.zeros(q.shape[:2] + v.shape[2:])
    lse = np.full(q.shape[:2], -np.inf)
    cu_q = np.asarray(cu_q, dtype=np.int64)
    cu_k = np.asarray(cu_k, dtype=np.int64)
    for b in range(cu_q.size - 1):
        q0, q1, k0, k1 = int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b]), int(cu_k[b + 1])
        if q1 == q0 or k1 == k0:
            continue
        sc = _block_scores(q[q0:q1], k[k0:k1], scale, causal, q0, k0)
        m = sc.max(-1, keepdims=True)
        p = np.exp(sc - m)
        den = p.sum(-1, keepdims=True)
        out[q0:q1] = np.einsum("hij,jhd->ihd", p / den, v[k0:k1])
        lse[q0:q1] = (m[..., 0] + np.log(den[..., 0])).T
    return out, lse


def block_attention_bwd(cu_q, cu_k, q, k, v, scale, causal, dout):
    """Gradients of block_attention_fwd (Jacobian d_s = alpha (<dout, v> -
    <dout, out>), compiler/edge_nn_attention.py:569-575).  Pinned by finite
    differences (tests/test_oracle.py)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    dout = np.asarray(dout, dtype=np.float64)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    cu_q = np.asarray(cu_q, dtype=np.int64)
    cu_k = np.asarray(cu_k, dtype=np.int64)
    for b in range(cu_q.size - 1):
        q0, q1, k0, k1 = int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b]), int(cu_k[b + 1])
        if q1 == q0 or k1 == k0:
            continue
        qs, ks, vs, gs = q[q0:q1], k[k0:k1], v[k0:k1], dout[q0:q1]
        sc = _block_scores(qs, ks, scale, causal, q0, k0)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        p = p / p.sum(-1, keepdims=True)
        o = np.einsum("hij,jhd->ihd", p, vs)
        dv[k0:k1] = np.einsum("hij,ihd->jhd", p, gs)
        dp = np.einsum("ihd,jhd->hij", gs, vs)
        delta = np.einsum("ihd,ihd->hi", gs, o)[..., None]
        ds = p * (dp - delta)
        dq[q0:q1] = np.einsum("hij,jhd->ihd", ds, ks) * scale
        dk[k0:k1] = np.einsum("hij,ihd->jhd", ds, qs) * scale
    return dq, dk, dv


def block_pruned_attention_fwd(cu_q, cu_k, q, k, v, scale, threshold, causal,
                               block_m=128, block_n=64):
    """online_softmax(block_prune_threshold=threshold) on a dense relation,
    restating the reference's tile admission (lib/Target/Triton/
    Translate.cpp:1760-1815): for each head and block of `block_m` queries,
    key tiles of `block_n` are visited in order; a tile whose maximum scaled
    log2 score (over the query block, masked pairs excluded) is below the
    block's running maximum by more than log2(threshold) is skipped, else the
    running maximum absorbs it and its keys count.  The result is exact
    softmax over the admitted tiles.  The schedule (block_m x block_n) is part
    of the semantics; this build's tiles are 128 queries x 64 keys.

    Pinned by: threshold -> 0 equals block_attention_fwd, and a hand-built
    case whose pruned tile is known (tests/test_oracle.py).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    H = q.shape[1]
    out = np.zeros(q.shape[:2] + v.shape[2:])
    lse = np.full(q.shape[:2], -np.inf)
    prune_log2 = np.log2(threshold)
    cu_q = np.asarray(cu_q, dtype=np.int64)
    cu_k = np.asarray(cu_k, dtype=np.int64)
    for b in range(cu_q.size - 1):
        q0, q1, k0, k1 = int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b]), int(cu_k[b + 1])
        for r0 in range(q0, q1, block_m):
            r1 = min(r0 + block_m, q1)
            kend = min(r0 + block_m, k1) if causal else k1
            for h in range(H):
                sc = _block_scores(q[r0:r1, h:h + 1], k[k0:kend, h:h + 1], scale, causal,
                                   r0, k0)[0]
                keep = np.zeros(kend - k0, dtype=bool)
                block_max = -np.inf
                for c0 in range(0, kend - k0, block_n):
                    tile = sc[:, c0:c0 + block_n] * np.log2(np.e)
                    tile_max = tile.max()
                    diff = tile_max - block_max
                    if diff < prune_log2:      # NaN (both -inf) is admitted
                        continue
                    block_max = max(block_max, tile_max)
                    keep[c0:c0 + block_n] = True
                s = np.where(keep[None, :], sc, -np.inf)
                m = s.max(-1, keepdims=True)
                ok = np.isfinite(m[:, 0])
                p = np.where(ok[:, None], np.exp(s - np.where(ok[:, None], m, 0)), 0.0)
                den = p.sum(-1)
                out[r0:r1, h] = np.where(den[:, None] > 0, p @ v[k0:kend, h] /
                                         np.where(den > 0, den, 1)[:, None], 0.0)
                lse[r0:r1, h] = np.where(den > 0, m[:, 0] + np.log(np.where(den > 0, den, 1)),
                                         -np.inf)
    return out, lse


def varlen_causal_fwd(cu_seqlens, q, k, v, scale):
    """Per-sequence causal softmax attention, fp64: the dot-product relation
    on Graph.cu_seqlens(causal=True).  Pinned by equality with dot_fwd on the
    materialized cu_seqlens CSR and by the reference's per-sequence SDPA check
    (tests/python/test_attention_examples.py:53-72)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    out = np.zeros_like(v)
    lse = np.zeros(q.shape[:2])
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    for b in range(cu.size - 1):
        s0, s1 = int(cu[b]), int(cu[b + 1])
        L = s1 - s0
        if L == 0:
            continue
        qs, ks, vs = q[s0:s1], k[s0:s1], v[s0:s1]
        sc = np.einsum("ihd,jhd->hij", qs, ks) * scale
        mask = np.tril(np.ones((L, L), dtype=bool))
        sc = np.where(mask[None], sc, -np.inf)
        m = sc.max(-1, keepdims=True)
        p = np.exp(sc - m)
        den = p.sum(-1, keepdims=True)
        out[s0:s1] = np.einsum("hij,jhd->ihd", p / den, vs)
        lse[s0:s1] = (m[..., 0] + np.log(den[..., 0])).T
    return out, lse


def varlen_causal_bwd(cu_seqlens, q, k, v, scale, dout):
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    dout = np.asarray(dout, dtype=np.float64)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    for b in range(cu.size - 1):
        s0, s1 = int(cu[b]), int(cu[b + 1])
        L = s1 - s0
        if L == 0:
            continue
        qs, ks, vs, gs = q[s0:s1], k[s0:s1], v[s0:s1], dout[s0:s1]
        sc = np.einsum("ihd,jhd->hij", qs, ks) * scale
        mask = np.tril(np.ones((L, L), dtype=bool))
        sc = np.where(mask[None], sc, -np.inf)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        p = p / p.sum(-1, keepdims=True)
        o = np.einsum("hij,jhd->ihd", p, vs)
        dv[s0:s1] = np.einsum("hij,ihd->jhd", p, gs)
        dp = np.einsum("ihd,jhd->hij", gs, vs)
        delta = np.einsum("ihd,ihd->hi", gs, o)[..., None]
        ds = p * (dp - delta)
        dq[s0:s1] = np.einsum("hij,jhd->ihd", ds, ks) * scale
        dk[s0:s1] = np.einsum("hij,ihd->jhd", ds, qs) * scale
    return dq, dk, dv


# ---------------------------------------------------------------------------
# nn-scored edge attention


def _act(name, z, p):
    from scipy.special import erf

    if name == "relu":
        return np.maximum(z, 0.0)
    if name == "leaky_relu":
        return np.where(z > 0, z, p * z)
    if name == "tanh":
        return np.tanh(z)
    if name == "sigmoid":
        return 1.0 / (1.0 + np.exp(-z))
    if name == "silu":
        return z / (1.0 + np.exp(-z))
    if name == "gelu":
        return 0.5 * z * (1.0 + erf(z / np.sqrt(2.0)))
    if name == "elu":
        return np.where(z > 0, z, p * (np.exp(np.minimum(z, 0.0)) - 1.0))
    return z


def _act_grad(name, z, p):
    from scipy.special import erf

    if name == "relu":
        return (z > 0).astype(np.float64)
    if name == "leaky_relu":
        return np.where(z > 0, 1.0, p)
    if name == "tanh":
        return 1.0 - np.tanh(z) ** 2
    if name == "sigmoid":
        s = 1.0 / (1.0 + np.exp(-z))
        return s * (1.0 - s)
    if name == "silu":
        s = 1.0 / (1.0 + np.exp(-z))
        return s * (1.0 + z * (1.0 - s))
    if name == "gelu":
        return 0.5 * (1.0 + erf(z / np.sqrt(2.0))) + z * np.exp(-0.5 * z * z) / np.sqrt(2 * np.pi)
    if name == "elu":
        return np.where(z > 0, 1.0, p * np.exp(np.minimum(z, 0.0)))
    return np.ones_like(z)


def _edge_inputs(row_ptr, col_idx, inputs):
    dst = destination_index(row_ptr)
    col = np.asarray(col_idx, dtype=np.int64)
    parts = []
    for role, arr in inputs:
        arr = np.asarray(arr, dtype=np.float64)
        arr = arr.reshape(arr.shape[0], -1)
        parts.append(arr[col] if role == "src" else arr[dst] if role == "dst" else arr)
    return np.concatenate(parts, axis=1), dst, col


def nn_attention_fwd(row_ptr, col_idx, inputs, layers, value):
    """online_softmax(score = net(concat of gathered fields), value = src.v),
    fp64: the eager semantics of a tg.nn.trace score (compiler/nn_capture.py:
    1-33: the module applied to the feature-concatenation of its inputs)
    under _evaluate_reference + reduce_online_softmax (message_passing.py:
    2848-2894, reducer_oracle.py:60-137).  inputs = [(role, [rows, w])],
    layers = [(W [out, in], b [out] or None, act, param)], activation after
    every layer but the last.  Returns (out, lse).

    Pinned by: finite differences of nn_attention_bwd and equality with Torch
    float64 autograd of the same composition (tests/test_oracle.py), and the
    single-Linear reduction to a bias-only score.
    """
    x, dst, col = _edge_inputs(row_ptr, col_idx, inputs)
    a = x
    for i, (W, b, act, p) in enumerate(layers):
        a = a @ np.asarray(W, dtype=np.float64).T + (0.0 if b is None else np.asarray(b, np.float64))
        if i + 1 < len(layers):
            a = _act(act, a, p)
    value = np.asarray(value, dtype=np.float64)
    return segment_softmax(row_ptr, a[:, 0], value[col])


def nn_attention_bwd(row_ptr, col_idx, inputs, layers, value, dout):
    """Gradients of nn_attention_fwd: (d inputs list, d value, [(dW, db)])."""
    x, dst, col = _edge_inputs(row_ptr, col_idx, inputs)
    acts, zs = [x], []
    a = x
    for i, (W, b, act, p) in enumerate(layers):
        z = a @ np.asarray(W, dtype=np.float64).T + (0.0 if b is None else np.asarray(b, np.float64))
        zs.append(z)
        if i + 1 < len(layers):
            a = _act(act, z, p)
            acts.append(a)
    s = zs[-1][:, 0]
    value = np.asarray(value, dtype=np.float64)
    dout = np.asarray(dout, dtype=np.float64)
    out, lse = segment_softmax(row_ptr, s, value[col])
    alpha = np.exp(s - lse[dst])
    dvalue = np.zeros_like(value)
    np.add.at(dvalue, col, alpha[:, None] * dout[dst])
    dalpha = (dout[dst] * value[col]).sum(-1)
    n = np.asarray(row_ptr).size - 1
    red = np.zeros(n)
    np.add.at(red, dst, alpha * dalpha)
    g = (alpha * (dalpha - red[dst]))[:, None]             # d z_last
    grads = [None] * len(layers)
    for i in range(len(layers) - 1, -1, -1):
        W, b, act, p = layers[i]
        W = np.asarray(W, dtype=np.float64)
        grads[i] = (g.T @ acts[i], None if b is None else g.sum(0))
        g = g @ W
        if i > 0:
            _, _, act_prev, p_prev = layers[i - 1]
            g = g * _act_grad(act_prev, zs[i - 1], p_prev)
    dinputs, off = [], 0
    for role, arr in inputs:
        arr = np.asarray(arr, dtype=np.float64)
        w = arr.reshape(arr.shape[0], -1).shape[1]
        part = g[:, off:off + w]
        off += w
        d = np.zeros((arr.shape[0], w))
        if role == "src":
            np.add.at(d, col, part)
        elif role == "dst":
            np.add.at(d, dst, part)
        else:
            d = part.copy()
        dinputs.append(d.reshape(arr.shape))
    return dinputs, dvalue, grads

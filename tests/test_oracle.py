"""CPU checks that pin the oracle (oracle/ref.py, oracle/planner.py).

Each oracle function is checked against something other than its own
formula: the reference's golden vectors (tests/golden/reference_vectors.json),
brute-force loops, closed forms, round trips and central finite differences.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import chunked, planner, ref

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def random_csr(rng, n_dst, n_src, max_deg, empty_frac=0.2):
    deg = rng.integers(0, max_deg + 1, size=n_dst)
    deg[rng.random(n_dst) < empty_frac] = 0
    row_ptr = np.zeros(n_dst + 1, dtype=np.int64)
    np.cumsum(deg, out=row_ptr[1:])
    col = np.concatenate([np.sort(rng.integers(0, n_src, size=d)) for d in deg]) \
        if deg.sum() else np.zeros(0, np.int64)
    return row_ptr, col.astype(np.int64)


# ---- graph indexing ---------------------------------------------------------

def test_destination_index_brute_force():
    rng = np.random.default_rng(0)
    rp, col = random_csr(rng, 50, 40, 7)
    expect = [i for i in range(50) for _ in range(rp[i], rp[i + 1])]
    assert ref.destination_index(rp).tolist() == expect


def test_transpose_brute_force_and_round_trip():
    rng = np.random.default_rng(1)
    rp, col = random_csr(rng, 60, 45, 9)
    rpt, colt, perm = ref.transpose(rp, col, 45)
    # brute force: for each source, scan edges in original order
    dst = ref.destination_index(rp)
    exp_rpt, exp_col, exp_perm = [0], [], []
    for j in range(45):
        for e in range(col.size):
            if col[e] == j:
                exp_col.append(dst[e])
                exp_perm.append(e)
        exp_rpt.append(len(exp_col))
    assert rpt.tolist() == exp_rpt
    assert colt.tolist() == exp_col
    assert perm.tolist() == exp_perm
    rp2, col2, _ = ref.transpose(rpt, colt, 60)
    assert rp2.tolist() == rp.tolist() and col2.tolist() == col.tolist()


def test_from_coo_brute_force_and_round_trip():
    rng = np.random.default_rng(2)
    for n_src, n_dst, E in [(5, 7, 0), (9, 6, 40), (30, 25, 200)]:
        src = rng.integers(0, n_src, E)
        dst = rng.integers(0, n_dst, E)
        rp, col, ns = ref.from_coo(src, dst, num_src=n_src, num_dst=n_dst)
        exp_rp, exp_col = [0], []
        for i in range(n_dst):
            exp_col += [int(src[e]) for e in range(E) if dst[e] == i]
            exp_rp.append(len(exp_col))
        assert rp.tolist() == exp_rp and col.tolist() == exp_col and ns == n_src
        # from_coo over a CSR's own edge list gives the CSR back.
        rp2, col2, _ = ref.from_coo(col, ref.destination_index(rp), num_dst=n_dst)
        assert rp2.tolist() == rp.tolist() and col2.tolist() == col.tolist()
    # non-causal cu_seqlens relation equals the brute-force block-diagonal one
    rp, col = ref.cu_seqlens_csr([0, 2, 2, 5], causal=False)
    assert rp.tolist() == [0, 2, 4, 7, 10, 13]
    assert col.tolist() == [0, 1, 0, 1, 2, 3, 4, 2, 3, 4, 2, 3, 4]


def test_cu_seqlens_matches_cat_of_triangles():
    # Reference property: cat([triangular(L)]) == cu_seqlens(cumsum(L))
    # (tests/python/test_graph_constructors.py:56-110).
    lengths = [3, 1, 0, 5]
    cu = np.concatenate([[0], np.cumsum(lengths)])
    rp, col = ref.cu_seqlens_csr(cu, causal=True)
    blocks = []
    for L in lengths:
        brp = np.zeros(L + 1, np.int64)
        np.cumsum(np.arange(1, L + 1), out=brp[1:])
        bcol = np.concatenate([np.arange(i + 1) for i in range(L)]) if L else np.zeros(0, np.int64)
        blocks.append((brp, bcol, L))
    crp, ccol, ns = ref.cat_csr(blocks)
    assert rp.tolist() == crp.tolist() and col.tolist() == ccol.tolist() and ns == sum(lengths)
    rp_full, col_full = ref.cu_seqlens_csr(cu, causal=False)
    assert rp_full[-1] == sum(L * L for L in lengths)


def test_degree_bins_membership_brute_force():
    rng = np.random.default_rng(2)
    rp, _ = random_csr(rng, 300, 100, 40, empty_frac=0.3)
    ub = [0, 4, 16, 1 << 40]
    rows, off = ref.degree_bins(rp, ub)
    deg = np.diff(rp)
    lower = -1
    for b, u in enumerate(ub):
        members = rows[off[b]:off[b + 1]]
        assert members.tolist() == sorted(members.tolist())       # ascending
        expect = [i for i in range(300) if lower < deg[i] <= u]
        assert members.tolist() == expect
        lower = u


# ---- sum reducer -------------------------------------------------------------

def test_sum_readme_known_answer():
    g = GOLD["readme_weighted_sum"]
    out = ref.sum_fwd(g["row_ptr"], g["col_idx"], g["x"], g["weight"])
    dx, dw = ref.sum_bwd(g["row_ptr"], g["col_idx"], g["x"], g["weight"], np.ones(3))
    assert out.tolist() == g["out"]
    assert dx.tolist() == g["dx"]
    assert dw.tolist() == g["dw"]


def test_sum_brute_force_and_finite_differences():
    rng = np.random.default_rng(3)
    rp, col = random_csr(rng, 20, 15, 6)
    x = rng.standard_normal((15, 3))
    w = rng.random(col.size)
    out = ref.sum_fwd(rp, col, x, w)
    for i in range(20):
        s = np.zeros(3)
        for e in range(rp[i], rp[i + 1]):
            s += w[e] * x[col[e]]
        np.testing.assert_allclose(out[i], s, rtol=1e-14, atol=1e-14)
    dout = rng.standard_normal(out.shape)
    dx, dw = ref.sum_bwd(rp, col, x, w, dout)
    eps = 1e-6
    for (arr, grad) in ((x, dx), (w, dw)):
        flat = arr.reshape(-1)
        for idx in rng.choice(flat.size, size=min(8, flat.size), replace=False):
            old = flat[idx]
            flat[idx] = old + eps
            fp = (ref.sum_fwd(rp, col, x, w) * dout).sum()
            flat[idx] = old - eps
            fm = (ref.sum_fwd(rp, col, x, w) * dout).sum()
            flat[idx] = old
            assert abs((fp - fm) / (2 * eps) - grad.reshape(-1)[idx]) < 1e-6


# ---- online softmax ---------------------------------------------------------

def test_online_softmax_reference_known_answer():
    g = GOLD["online_softmax_large_scores"]
    score = np.asarray(g["score"])[np.asarray(g["col_idx"])]
    value = np.asarray(g["value"])[np.asarray(g["col_idx"])]
    out, lse = ref.segment_softmax(g["row_ptr"], score, value)
    np.testing.assert_allclose(out, g["out"], atol=10 ** -g["places"])
    dscore_e, dvalue_e = ref.segment_softmax_bwd(g["row_ptr"], score, value,
                                                 np.ones_like(out))
    # gradients w.r.t. the per-source fields: scatter edge grads by col
    col = np.asarray(g["col_idx"])
    dscore = np.zeros(3)
    np.add.at(dscore, col, dscore_e)
    dvalue = np.zeros((3, 2))
    np.add.at(dvalue, col, dvalue_e)
    np.testing.assert_allclose(dscore, g["dscore"], atol=10 ** -g["places"])
    np.testing.assert_allclose(dvalue, g["dvalue"], atol=10 ** -g["places"])
    assert np.all(np.isfinite(lse))


def test_online_softmax_empty_row_and_heads():
    g = GOLD["online_softmax_empty_row_heads"]
    rp, col = np.asarray(g["row_ptr"]), np.asarray(g["col_idx"])
    H, W = g["heads"], g["width"]
    value_src = np.arange(4 * H * W, dtype=np.float64).reshape(4, H, W)
    score = np.asarray(g["score"])
    out, lse = ref.segment_softmax(rp, score, value_src[col])
    assert np.all(out[1] == 0) and np.all(np.isneginf(lse[1]))
    for row in (0, 2):
        b, e = rp[row], rp[row + 1]
        s = score[b:e]
        p = np.exp(s - s.max(0)) / np.exp(s - s.max(0)).sum(0)
        np.testing.assert_allclose(out[row], (p[..., None] * value_src[col[b:e]]).sum(0),
                                   rtol=1e-12)


def test_single_edge_closed_form():
    rp = np.array([0, 1]); col = np.array([0])
    out, lse = ref.segment_softmax(rp, np.array([[3.5]]), np.array([[[2.0, -1.0]]]))
    assert out.tolist() == [[[2.0, -1.0]]] and lse.tolist() == [[3.5]]


def _fd_check(f, arrays, grads, rng, eps=1e-6, tol=1e-6, picks=6):
    for arr, grad in zip(arrays, grads):
        flat = arr.reshape(-1)
        for idx in rng.choice(flat.size, size=min(picks, flat.size), replace=False):
            old = flat[idx]
            flat[idx] = old + eps
            fp = f()
            flat[idx] = old - eps
            fm = f()
            flat[idx] = old
            num = (fp - fm) / (2 * eps)
            assert abs(num - grad.reshape(-1)[idx]) < tol * max(1.0, abs(num)), (num, grad.reshape(-1)[idx])


def test_gat_finite_differences_and_uniform_closed_form():
    rng = np.random.default_rng(4)
    rp, col = random_csr(rng, 12, 12, 5)
    H, D = 2, 3
    h = rng.standard_normal((12, H, D))
    a_s = rng.standard_normal((H, D)) * 0.5
    a_d = rng.standard_normal((H, D)) * 0.5
    dout = rng.standard_normal((12, H, D))
    dh, das, dad = ref.gat_bwd(rp, col, h, a_s, a_d, 0.2, dout)
    f = lambda: (ref.gat_fwd(rp, col, h, a_s, a_d, 0.2)[0] * dout).sum()
    _fd_check(f, [h, a_s, a_d], [dh, das, dad], rng)
    # a = 0 -> every score is 0 -> out is the neighbour mean
    out, _ = ref.gat_fwd(rp, col, h, np.zeros((H, D)), np.zeros((H, D)), 0.2)
    for i in range(12):
        if rp[i + 1] > rp[i]:
            np.testing.assert_allclose(out[i], h[col[rp[i]:rp[i + 1]]].mean(0), rtol=1e-12)
        else:
            assert np.all(out[i] == 0)


def test_gat_bipartite_finite_differences_and_the_homogeneous_sum():
    """Two feature tensors (12 destinations, 9 sources): every gradient by
    central differences; with one tensor for both roles, dh_src + dh_dst is
    the homogeneous dh."""
    rng = np.random.default_rng(14)
    rp, col = random_csr(rng, 12, 9, 5)
    H, D = 2, 3
    hs = rng.standard_normal((9, H, D))
    hd = rng.standard_normal((12, H, D))
    a_s = rng.standard_normal((H, D)) * 0.5
    a_d = rng.standard_normal((H, D)) * 0.5
    dout = rng.standard_normal((12, H, D))
    grads = ref.gat_bwd_bipartite(rp, col, hs, hd, a_s, a_d, 0.2, dout)
    f = lambda: (ref.gat_fwd(rp, col, hs, a_s, a_d, 0.2, h_dst=hd)[0] * dout).sum()
    _fd_check(f, [hs, hd, a_s, a_d], list(grads), rng)
    rp2, col2 = random_csr(rng, 10, 10, 4)
    h = rng.standard_normal((10, H, D))
    g2 = rng.standard_normal((10, H, D))
    dhs, dhd, das, dad = ref.gat_bwd_bipartite(rp2, col2, h, h, a_s, a_d, 0.2, g2)
    dh, das1, dad1 = ref.gat_bwd(rp2, col2, h, a_s, a_d, 0.2, g2)
    np.testing.assert_allclose(dhs + dhd, dh, rtol=1e-13, atol=1e-14)
    np.testing.assert_array_equal(das, das1)
    np.testing.assert_array_equal(dad, dad1)


def test_dot_finite_differences():
    rng = np.random.default_rng(5)
    rp, col = random_csr(rng, 10, 9, 6)
    H, D = 2, 4
    q = rng.standard_normal((10, H, D)); k = rng.standard_normal((9, H, D))
    v = rng.standard_normal((9, H, D)); bias = rng.standard_normal((col.size, H))
    dout = rng.standard_normal((10, H, D))
    dq, dk, dv, db = ref.dot_bwd(rp, col, q, k, v, 0.5, bias, dout)
    f = lambda: (ref.dot_fwd(rp, col, q, k, v, 0.5, bias)[0] * dout).sum()
    _fd_check(f, [q, k, v, bias], [dq, dk, dv, db], rng)


def test_varlen_matches_dot_on_materialized_csr():
    rng = np.random.default_rng(6)
    lengths = [5, 1, 7]
    cu = np.concatenate([[0], np.cumsum(lengths)])
    T, H, D = sum(lengths), 2, 4
    q, k, v = (rng.standard_normal((T, H, D)) for _ in range(3))
    rp, col = ref.cu_seqlens_csr(cu)
    o1, l1 = ref.varlen_causal_fwd(cu, q, k, v, 0.3)
    o2, l2 = ref.dot_fwd(rp, col, q, k, v, 0.3)
    np.testing.assert_allclose(o1, o2, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(l1, l2, rtol=1e-12)
    dout = rng.standard_normal((T, H, D))
    g1 = ref.varlen_causal_bwd(cu, q, k, v, 0.3, dout)
    g2 = ref.dot_bwd(rp, col, q, k, v, 0.3, None, dout)[:3]
    for a, b in zip(g1, g2):
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)


def _dense_csr(n_dst, n_src, causal):
    rows, cols = [0], []
    for i in range(n_dst):
        cols += list(range(min(i + 1, n_src) if causal else n_src))
        rows.append(len(cols))
    return np.asarray(rows), np.asarray(cols, dtype=np.int64)


@pytest.mark.parametrize("n_dst,n_src,causal", [(7, 5, False), (6, 6, True), (3, 9, False)])
def test_block_attention_matches_dot_on_materialized_dense(n_dst, n_src, causal):
    """Graph.dense / Graph.triangular as one block: the tile oracle equals the
    CSR oracle on the materialized relation, forward and backward."""
    rng = np.random.default_rng(n_dst * 10 + n_src)
    H, D = 2, 4
    q = rng.standard_normal((n_dst, H, D))
    k, v = (rng.standard_normal((n_src, H, D)) for _ in range(2))
    rp, col = _dense_csr(n_dst, n_src, causal)
    o1, l1 = ref.block_attention_fwd([0, n_dst], [0, n_src], q, k, v, 0.4, causal)
    o2, l2 = ref.dot_fwd(rp, col, q, k, v, 0.4)
    np.testing.assert_allclose(o1, o2, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(l1, l2, rtol=1e-12)
    dout = rng.standard_normal((n_dst, H, D))
    g1 = ref.block_attention_bwd([0, n_dst], [0, n_src], q, k, v, 0.4, causal, dout)
    g2 = ref.dot_bwd(rp, col, q, k, v, 0.4, None, dout)[:3]
    for a, b in zip(g1, g2):
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)
    # non-causal varlen blocks equal the materialized cu_seqlens(causal=False)
    cu = np.array([0, 3, 3, 7])
    qv, kv, vv = (rng.standard_normal((7, H, D)) for _ in range(3))
    rp, col = ref.cu_seqlens_csr(cu, causal=False)
    o1, _ = ref.block_attention_fwd(cu, cu, qv, kv, vv, 0.4, False)
    o2, _ = ref.dot_fwd(rp, col, qv, kv, vv, 0.4)
    np.testing.assert_allclose(o1, o2, rtol=1e-12, atol=1e-12)


def test_block_attention_bwd_finite_differences():
    rng = np.random.default_rng(12)
    q, k, v, g = (rng.standard_normal((4, 1, 3)) for _ in range(4))
    grads = ref.block_attention_bwd([0, 4], [0, 4], q, k, v, 0.7, True, g)
    eps = 1e-6
    for t, dt in zip((q, k, v), grads):
        for idx in np.ndindex(t.shape):
            t[idx] += eps
            fp = (ref.block_attention_fwd([0, 4], [0, 4], q, k, v, 0.7, True)[0] * g).sum()
            t[idx] -= 2 * eps
            fm = (ref.block_attention_fwd([0, 4], [0, 4], q, k, v, 0.7, True)[0] * g).sum()
            t[idx] += eps
            assert abs((fp - fm) / (2 * eps) - dt[idx]) < 1e-6


def test_block_pruned_attention_known_answers():
    """Tile admission (Translate.cpp:1793-1815) on hand-built scores: every
    query is the same vector u and each 4-key tile holds +a u or -a u keys, so
    every score of a tile is equal and the admitted set is known."""
    D, a, scale = 4, 3.0, 0.5
    u = np.ones(D)
    q = np.tile(u, (8, 1, 1))                       # 8 queries, H = 1
    signs = [+1, -1, +1]                             # three tiles of 4 keys
    k = np.concatenate([np.tile(s * a * u, (4, 1, 1)) for s in signs])
    v = np.arange(12 * D, dtype=np.float64).reshape(12, 1, D)
    # tile 1's log2 scores trail tile 0's by 2*a*|u|^2*scale*log2(e) = 17.3
    thr = 2.0 ** -10
    out, lse = ref.block_pruned_attention_fwd([0, 8], [0, 12], q, k, v, scale, thr, False,
                                              block_m=8, block_n=4)
    expect = v[[0, 1, 2, 3, 8, 9, 10, 11], 0].mean(0)          # tiles 0 and 2, equal weights
    np.testing.assert_allclose(out[:, 0], np.tile(expect, (8, 1)), rtol=1e-12)
    np.testing.assert_allclose(lse[:, 0], a * D * scale + np.log(8.0), rtol=1e-12)
    # a threshold the gap passes admits everything: exact softmax
    exact = ref.block_attention_fwd([0, 8], [0, 12], q, k, v, scale, False)
    loose = ref.block_pruned_attention_fwd([0, 8], [0, 12], q, k, v, scale, 2.0 ** -20, False,
                                           block_m=8, block_n=4)
    np.testing.assert_allclose(loose[0], exact[0], rtol=1e-12)
    # order matters: a low first tile is always admitted (running max -inf)
    k2 = k[[4, 5, 6, 7, 0, 1, 2, 3, 8, 9, 10, 11]]
    v2 = v[[4, 5, 6, 7, 0, 1, 2, 3, 8, 9, 10, 11]]
    out2, _ = ref.block_pruned_attention_fwd([0, 8], [0, 12], q, k2, v2, scale, thr, False,
                                             block_m=8, block_n=4)
    exact2 = ref.block_attention_fwd([0, 8], [0, 12], q, k2, v2, scale, False)[0]
    np.testing.assert_allclose(out2, exact2, rtol=1e-12)


# ---- planner ---------------------------------------------------------------

@pytest.mark.parametrize("case", GOLD["planner"], ids=lambda c: c["cite"].split(":")[0].split("/")[-1])
def test_planner_lit_vectors(case):
    res = planner.plan(case["rows"], case["max"], case["sum"], case["histogram"], case["has_node"])
    for key, value in case["expect"].items():
        assert res[key] == value, (key, res[key], value)


# ---- nn-scored attention ----------------------------------------------------

def _nn_case(seed):
    rng = np.random.default_rng(seed)
    rp, col = random_csr(rng, 7, 6, 4)
    E = col.size
    x = rng.standard_normal((6, 3))
    y = rng.standard_normal((7, 2))
    ef = rng.standard_normal((E, 2))
    inputs = [("src", x), ("dst", y), ("edge", ef)]
    layers = [(rng.standard_normal((5, 7)) * 0.5, rng.standard_normal(5) * 0.1, "gelu", 0.0),
              (rng.standard_normal((4, 5)) * 0.5, None, "leaky_relu", 0.2),
              (rng.standard_normal((1, 4)) * 0.5, rng.standard_normal(1) * 0.1, "identity", 0.0)]
    value = rng.standard_normal((6, 3))
    dout = rng.standard_normal((7, 3))
    return rp, col, inputs, layers, value, dout


def test_nn_attention_bwd_finite_differences():
    rp, col, inputs, layers, value, dout = _nn_case(21)
    dinputs, dvalue, dlayers = ref.nn_attention_bwd(rp, col, inputs, layers, value, dout)
    f = lambda: (ref.nn_attention_fwd(rp, col, inputs, layers, value)[0] * dout).sum()
    eps = 1e-6

    def check(arr, grad):
        for idx in np.ndindex(arr.shape):
            arr[idx] += eps
            fp = f()
            arr[idx] -= 2 * eps
            fm = f()
            arr[idx] += eps
            assert abs((fp - fm) / (2 * eps) - grad[idx]) < 1e-6, idx

    for (_, arr), g in zip(inputs, dinputs):
        check(arr, g)
    check(value, dvalue)
    for (W, b, _, _), (dW, db) in zip(layers, dlayers):
        check(W, dW)
        if b is not None:
            check(b, db)


def test_nn_attention_matches_torch_autograd_float64():
    """The same composition written with Torch ops in float64 (gather,
    concatenation, the nn.Module chain, segment softmax by index ops) and
    differentiated by autograd."""
    rp, col, inputs, layers, value, dout = _nn_case(22)
    dst = torch.as_tensor(ref.destination_index(rp))
    colt = torch.as_tensor(col)
    ts = [torch.tensor(a, requires_grad=True) for _, a in inputs]
    gathered = [t[colt] if r == "src" else t[dst] if r == "dst" else t
                for (r, _), t in zip(inputs, ts)]
    net = torch.nn.Sequential(torch.nn.Linear(7, 5), torch.nn.GELU(), torch.nn.Linear(5, 4, bias=False),
                              torch.nn.LeakyReLU(0.2), torch.nn.Linear(4, 1)).double()
    with torch.no_grad():
        for lin, (W, b, _, _) in zip([net[0], net[2], net[4]], layers):
            lin.weight.copy_(torch.as_tensor(W))
            if b is not None:
                lin.bias.copy_(torch.as_tensor(b))
    s = net(torch.cat(gathered, dim=1))[:, 0]
    v = torch.tensor(value, requires_grad=True)
    n = rp.size - 1
    m = torch.full((n,), -torch.inf, dtype=torch.float64).scatter_reduce(0, dst, s, "amax")
    p = torch.exp(s - m[dst])
    den = torch.zeros(n, dtype=torch.float64).index_add(0, dst, p)
    out = torch.zeros(n, 3, dtype=torch.float64).index_add(0, dst, v[colt] * p[:, None])
    out = torch.where(den[:, None] > 0, out / den.clamp_min(1e-300)[:, None], 0.0)
    e_out, _ = ref.nn_attention_fwd(rp, col, inputs, layers, value)
    np.testing.assert_allclose(out.detach().numpy(), e_out, rtol=1e-12, atol=1e-12)
    params = [net[0].weight, net[0].bias, net[2].weight, net[4].weight, net[4].bias]
    got = torch.autograd.grad(out, ts + [v] + params, torch.as_tensor(dout))
    dinputs, dvalue, dlayers = ref.nn_attention_bwd(rp, col, inputs, layers, value, dout)
    expect = dinputs + [dvalue, dlayers[0][0], dlayers[0][1], dlayers[1][0], dlayers[2][0],
                        dlayers[2][1]]
    for a, b in zip(got, expect):
        np.testing.assert_allclose(a.numpy(), b, rtol=1e-10, atol=1e-12)


def test_chunked_nn_attention_matches_ref():
    """oracle/chunked.nn_attention (the Torch float64 checker of the
    full-size nn test) against ref.nn_attention_fwd/bwd, with a value that is
    also a source field, as in the reference's GAT example."""
    rp, col, inputs, layers, value, dout = _nn_case(23)
    value = inputs[0][1]   # the value is the source field x
    rpt, colt = torch.as_tensor(rp), torch.as_tensor(col)
    t_in = [(r, torch.as_tensor(a)) for r, a in inputs]
    t_layers = [(torch.as_tensor(W), None if b is None else torch.as_tensor(b), act, p)
                for W, b, act, p in layers]
    out, d_in, d_v, d_layers = chunked.nn_attention(rpt, colt, t_in, t_layers,
                                                    torch.as_tensor(value),
                                                    torch.as_tensor(dout[:, :3]))
    e_out, _ = ref.nn_attention_fwd(rp, col, inputs, layers, value)
    np.testing.assert_allclose(out.numpy(), e_out, rtol=1e-12, atol=1e-12)
    e_in, e_v, e_layers = ref.nn_attention_bwd(rp, col, inputs, layers, value, dout[:, :3])
    for a, b in zip(d_in + [d_v], e_in + [e_v]):
        np.testing.assert_allclose(a.numpy(), b, rtol=1e-10, atol=1e-12)
    for (dW, db), (eW, eb) in zip(d_layers, e_layers):
        np.testing.assert_allclose(dW.numpy(), eW, rtol=1e-10, atol=1e-12)
        assert (db is None) == (eb is None)
        if db is not None:
            np.testing.assert_allclose(db.numpy(), eb, rtol=1e-10, atol=1e-12)


# ---- timed CPU baselines (bench.py's cpu_baseline legs) ---------------------

def test_native_sum_loop_matches_oracle():
    """oracle/cpu_native.c: the README known answer exactly, the fp64 oracle
    within fp32 rounding, and the same bits for any thread count (chunking
    splits output elements, it never reorders a row's sum)."""
    from oracle import native

    g = GOLD["readme_weighted_sum"]
    x = np.asarray(g["x"], dtype=np.float32).reshape(-1, 1)
    out = native.csr_sum_fwd(g["row_ptr"], g["col_idx"], x, g["weight"], threads=2)
    assert out.reshape(-1).tolist() == g["out"]
    rng = np.random.default_rng(11)
    rp, col = random_csr(rng, 300, 120, 20)
    x = rng.standard_normal((120, 7)).astype(np.float32)
    w = rng.random(col.size).astype(np.float32)
    want = ref.sum_fwd(rp, col, x.astype(np.float64), w.astype(np.float64))
    one = native.csr_sum_fwd(rp, col, x, w, threads=1)
    np.testing.assert_allclose(one, want, rtol=1e-5, atol=1e-5)
    for t in (3, 8):
        assert np.array_equal(native.csr_sum_fwd(rp, col, x, w, threads=t), one)


def test_native_lowered_backward_matches_oracle():
    """oracle/cpu_native.c's restatement of the reference runtime's lowered
    backward: the README known answer (dx, dw) exactly and the fp64 oracle
    within fp32 rounding."""
    from oracle import native

    g = GOLD["readme_weighted_sum"]
    x = np.asarray(g["x"], dtype=np.float32).reshape(-1, 1)
    dout = np.ones((len(g["row_ptr"]) - 1, 1), dtype=np.float32)
    dx, dw = native.csr_sum_bwd_lowered(g["row_ptr"], g["col_idx"], x, g["weight"], dout)
    assert dx.reshape(-1).tolist() == g["dx"]
    assert dw.tolist() == g["dw"]
    rng = np.random.default_rng(12)
    rp, col = random_csr(rng, 60, 40, 12)
    x = rng.standard_normal((40, 5)).astype(np.float32)
    w = rng.random(col.size).astype(np.float32)
    dout = rng.standard_normal((60, 5)).astype(np.float32)
    e_dx, e_dw = ref.sum_bwd(rp, col, x.astype(np.float64), w.astype(np.float64),
                             dout.astype(np.float64))
    dx, dw = native.csr_sum_bwd_lowered(rp, col, x, w, dout)
    np.testing.assert_allclose(dx, e_dx, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(dw, np.asarray(e_dw).reshape(-1), rtol=1e-5, atol=1e-5)


def test_eager_torch_cpu_path_matches_oracle():
    """oracle/eager_torch.py (the reference's eager Torch CPU path) agrees
    with the pinned fp64 oracle for the sum, GAT and dot-product steps."""
    from oracle import eager_torch

    rng = np.random.default_rng(12)
    rp, col = random_csr(rng, 40, 40, 9)
    rpt, colt = torch.tensor(rp), torch.tensor(col)
    H, D = 2, 4
    x = rng.standard_normal((40, 5))
    w = rng.random(col.size)
    dout = rng.standard_normal((40, 5))
    out, dx, dw = eager_torch.sum_step(rpt, colt, torch.tensor(x), torch.tensor(w),
                                       torch.tensor(dout))
    e_dx, e_dw = ref.sum_bwd(rp, col, x, w, dout)
    np.testing.assert_allclose(out.detach().numpy(), ref.sum_fwd(rp, col, x, w), rtol=1e-12,
                               atol=1e-12)
    np.testing.assert_allclose(dx.numpy(), e_dx, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dw.numpy(), e_dw, rtol=1e-12, atol=1e-12)

    h = rng.standard_normal((40, H, D))
    a_s, a_d = rng.standard_normal((H, D)), rng.standard_normal((H, D))
    dout = rng.standard_normal((40, H, D))
    out, dh, das, dad = eager_torch.gat_step(rpt, colt, torch.tensor(h), torch.tensor(a_s),
                                             torch.tensor(a_d), 0.2, torch.tensor(dout))
    e_out, _ = ref.gat_fwd(rp, col, h, a_s, a_d, 0.2)
    e_grads = ref.gat_bwd(rp, col, h, a_s, a_d, 0.2, dout)
    np.testing.assert_allclose(out.detach().numpy(), e_out, rtol=1e-10, atol=1e-12)
    for got, want in zip((dh, das, dad), e_grads):
        np.testing.assert_allclose(got.numpy(), want, rtol=1e-10, atol=1e-12)

    q, k, v = (rng.standard_normal((40, H, D)) for _ in range(3))
    bias = rng.standard_normal((col.size, H))
    out = eager_torch.dot_step(rpt, colt, *(torch.tensor(a) for a in (q, k, v, bias)), 0.5)
    e_out, _ = ref.dot_fwd(rp, col, q, k, v, 0.5, bias)
    np.testing.assert_allclose(out.detach().numpy(), e_out, rtol=1e-10, atol=1e-12)


def test_eager_nn_step_matches_oracle():
    """oracle/eager_torch.nn_gat_step (the timed CPU leg of the nn bench)
    agrees with ref.nn_attention_fwd/bwd in float64."""
    from torch import nn

    from oracle import eager_torch

    rng = np.random.default_rng(13)
    rp, col = random_csr(rng, 30, 30, 6)
    x = rng.standard_normal((30, 4))
    disp = rng.standard_normal((col.size, 3))
    torch.manual_seed(0)
    net = nn.Sequential(nn.Linear(11, 6), nn.LeakyReLU(0.2), nn.Linear(6, 1)).double()
    dout = rng.standard_normal((30, 4))
    out, dx, ddisp = eager_torch.nn_gat_step(torch.tensor(rp), torch.tensor(col), torch.tensor(x),
                                             torch.tensor(disp), net, torch.tensor(dout))
    layers = [(net[0].weight.detach().numpy(), net[0].bias.detach().numpy(), "leaky_relu", 0.2),
              (net[2].weight.detach().numpy(), net[2].bias.detach().numpy(), "identity", 0.0)]
    inputs = [("edge", disp), ("src", x), ("dst", x)]
    e_out, _ = ref.nn_attention_fwd(rp, col, inputs, layers, x)
    np.testing.assert_allclose(out.detach().numpy(), e_out, rtol=1e-10, atol=1e-12)
    (d_edge, d_src, d_dst), d_value, _ = ref.nn_attention_bwd(rp, col, inputs, layers, x, dout)
    np.testing.assert_allclose(ddisp.numpy(), d_edge, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(dx.numpy(), d_src + d_dst + d_value, rtol=1e-9, atol=1e-12)


# ---- row-chunked fp64 restatement (oracle/chunked.py) ---------------------------

@pytest.mark.parametrize("edges_per_block", [1, 7, 1 << 20])
def test_chunked_gat_matches_ref(edges_per_block):
    """The full-size checker equals ref.gat_fwd/gat_bwd (itself pinned by
    finite differences and the uniform closed form) for any block size."""
    from oracle import chunked

    rng = np.random.default_rng(21)
    rp, col = random_csr(rng, 60, 60, 12, empty_frac=0.25)
    H, D = 3, 4
    h = rng.standard_normal((60, H, D))
    a_s, a_d = rng.standard_normal((H, D)), rng.standard_normal((H, D))
    dout = rng.standard_normal((60, H, D))
    t = lambda a: torch.tensor(a, dtype=torch.float64)
    rpt, colt = torch.tensor(rp), torch.tensor(col)
    out, lse = chunked.gat_fwd(rpt, colt, t(h), t(a_s), t(a_d), 0.2, edges_per_block)
    e_out, e_lse = ref.gat_fwd(rp, col, h, a_s, a_d, 0.2)
    np.testing.assert_allclose(out.numpy(), e_out, rtol=1e-12, atol=1e-13)
    np.testing.assert_array_equal(np.isinf(lse.numpy()), np.isinf(e_lse))
    np.testing.assert_allclose(lse.numpy()[np.isfinite(e_lse)], e_lse[np.isfinite(e_lse)],
                               rtol=1e-12)
    got = chunked.gat_bwd(rpt, colt, t(h), t(a_s), t(a_d), 0.2, t(dout), edges_per_block)
    for g, w in zip(got, ref.gat_bwd(rp, col, h, a_s, a_d, 0.2, dout)):
        np.testing.assert_allclose(g.numpy(), w, rtol=1e-11, atol=1e-12)


@pytest.mark.parametrize("with_bias", [False, True])
def test_chunked_dot_matches_ref(with_bias):
    from oracle import chunked

    rng = np.random.default_rng(22)
    rp, col = random_csr(rng, 50, 70, 15, empty_frac=0.3)
    H, D = 2, 8
    q = rng.standard_normal((50, H, D))
    k, v = rng.standard_normal((70, H, D)), rng.standard_normal((70, H, D))
    bias = rng.standard_normal((col.size, H)) if with_bias else None
    dout = rng.standard_normal((50, H, D))
    t = lambda a: None if a is None else torch.tensor(a, dtype=torch.float64)
    rpt, colt = torch.tensor(rp), torch.tensor(col)
    out, _ = chunked.dot_fwd(rpt, colt, t(q), t(k), t(v), 0.3, t(bias), edges_per_block=9)
    e_out, _ = ref.dot_fwd(rp, col, q, k, v, 0.3, bias)
    np.testing.assert_allclose(out.numpy(), e_out, rtol=1e-12, atol=1e-13)
    # a row subset evaluates exactly those rows
    rows = np.array([3, 4, 17, 49])
    sub, _ = chunked.dot_fwd(rpt, colt, t(q), t(k), t(v), 0.3, t(bias), rows=rows)
    np.testing.assert_allclose(sub.numpy()[rows], e_out[rows], rtol=1e-12, atol=1e-13)
    others = np.setdiff1d(np.arange(50), rows)
    assert not sub.numpy()[others].any()
    got = chunked.dot_bwd(rpt, colt, t(q), t(k), t(v), 0.3, t(bias), t(dout),
                          edges_per_block=5)
    for g, w in zip(got, ref.dot_bwd(rp, col, q, k, v, 0.3, bias, dout)):
        np.testing.assert_allclose(g.numpy(), w, rtol=1e-11, atol=1e-12)


@pytest.mark.parametrize("query_block", [1, 7, 64, 512])
def test_chunked_causal_sequence_matches_ref(query_block):
    """The full-size C5 checker equals ref.varlen_causal_fwd/bwd (pinned by
    equality with the dot-product relation on the materialized cu_seqlens
    CSR) for any query block, and its logsumexp equals the per-row closed
    form log(sum_j<=i exp(s_ij))."""
    from oracle import chunked

    rng = np.random.default_rng(24)
    L, H, D, scale = 70, 3, 8, 0.35
    q, k, v, dout = (rng.standard_normal((L, H, D)) for _ in range(4))
    t = lambda a: torch.tensor(a, dtype=torch.float64)
    out, lse, dq, dk, dv = chunked.causal_sequence(t(q), t(k), t(v), scale, t(dout),
                                                   query_block=query_block)
    cu = np.array([0, L])
    e_out, e_lse = ref.varlen_causal_fwd(cu, q, k, v, scale)
    np.testing.assert_allclose(out.numpy(), e_out, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(lse.numpy(), e_lse, rtol=1e-12)
    for g, w in zip((dq, dk, dv), ref.varlen_causal_bwd(cu, q, k, v, scale, dout)):
        np.testing.assert_allclose(g.numpy(), w, rtol=1e-11, atol=1e-12)
    i, h = 41, 2
    s = (q[i, h] * k[:i + 1, h]).sum(-1) * scale
    assert abs(lse.numpy()[i, h] - np.log(np.exp(s).sum())) < 1e-12
    fwd_only = chunked.causal_sequence(t(q), t(k), t(v), scale, query_block=query_block)
    assert len(fwd_only) == 2 and torch.equal(fwd_only[0], out)


def test_reference_bf16_dot_arithmetic_is_the_eager_path():
    """eager_torch.dot_reference: in float64 it equals the pinned ref
    forward and backward; in bf16 it differs from them by the bf16 rounding
    of q*k and of the output, well inside the 2e-2 bound."""
    from oracle import eager_torch

    rng = np.random.default_rng(23)
    rp, col = random_csr(rng, 40, 40, 10)
    H, D = 2, 16
    q, k, v = (rng.standard_normal((40, H, D)) for _ in range(3))
    bias = rng.standard_normal((col.size, H))
    dout = rng.standard_normal((40, H, D))
    rpt, colt = torch.tensor(rp), torch.tensor(col)
    got = eager_torch.dot_reference(rpt, colt, *(torch.tensor(a) for a in (q, k, v, bias)),
                                    0.25, torch.tensor(dout))
    want = (ref.dot_fwd(rp, col, q, k, v, 0.25, bias)[0],
            *ref.dot_bwd(rp, col, q, k, v, 0.25, bias, dout))
    for g, w in zip(got, want):
        np.testing.assert_allclose(g.numpy(), w, rtol=1e-11, atol=1e-12)
    b16 = lambda a: torch.tensor(a, dtype=torch.float32).to(torch.bfloat16)
    got16 = eager_torch.dot_reference(rpt, colt, b16(q), b16(k), b16(v),
                                      torch.tensor(bias, dtype=torch.float32), 0.25, b16(dout))
    assert got16[0].dtype == torch.bfloat16 and got16[4].dtype == torch.float32
    for g, w in zip(got16, want):
        err = np.abs(g.double().numpy() - w).max() / np.abs(w).max()
        assert 0 < err < 2e-2


def test_row_plan_chunk_offsets_brute_force():
    """ref.row_plan's split rows and chunk offsets against a direct walk:
    every split row in ascending order, cut into consecutive chunk_edges-edge
    pieces, the offsets counting the pieces before each row."""
    rng = np.random.default_rng(24)
    rp, _ = random_csr(rng, 200, 10, 30, empty_frac=0.2)
    deg = np.diff(rp)
    deg[[5, 77, 150]] = (130, 64, 1000)
    rp = np.concatenate([[0], np.cumsum(deg)])
    rows, n_empty, n_wave, n_split, offsets = ref.row_plan(rp, 40, 16)
    split = [i for i in range(200) if deg[i] > 40]
    assert rows[n_empty + n_wave:].tolist() == split
    pieces = []
    for i in split:
        e = rp[i]
        while e < rp[i + 1]:
            pieces.append((i, e, min(e + 16, rp[i + 1])))
            e += 16
    assert offsets[-1] == len(pieces)
    for j, i in enumerate(split):
        mine = [p for p in pieces if p[0] == i]
        assert offsets[j + 1] - offsets[j] == len(mine)
        assert pieces[offsets[j]] == mine[0]
    assert n_empty == int((deg == 0).sum()) and n_wave == int(((deg > 0) & (deg <= 40)).sum())


def test_eager_nn_message_sum_closed_form_and_nn_attention_agrees_with_ref():
    """oracle/eager_torch.nn_message_sum: for one Linear layer the row sum is
    W (sum of the row's gathered inputs) + degree * b; nn_attention equals
    the pinned ref.nn_attention_fwd/bwd for a two-layer tanh network."""
    from torch import nn

    from oracle import eager_torch

    rng = np.random.default_rng(31)
    rp, col = random_csr(rng, 30, 25, 8)
    rpt, colt = torch.tensor(rp), torch.tensor(col)
    xs = rng.standard_normal((25, 3))
    xd = rng.standard_normal((30, 2))
    xe = rng.standard_normal((col.size,))
    net = nn.Linear(6, 4).double()
    inputs = [("src", torch.tensor(xs)), ("dst", torch.tensor(xd)), ("edge", torch.tensor(xe))]
    dout = torch.tensor(rng.standard_normal((30, 4)))
    out, gin, gp = eager_torch.nn_message_sum(rpt, colt, inputs, net, dout)
    dst = ref.destination_index(rp)
    gathered = np.concatenate([xs[col], xd[dst], xe[:, None]], axis=1)
    rows = np.zeros((30, 6))
    np.add.at(rows, dst, gathered)
    W, b = net.weight.detach().numpy(), net.bias.detach().numpy()
    want = rows @ W.T + np.diff(rp)[:, None] * b
    np.testing.assert_allclose(out.numpy(), want, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(gp[0].numpy(), dout.numpy().T @ rows, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(gp[1].numpy(), (np.diff(rp)[:, None] * dout.numpy()).sum(0),
                               rtol=1e-12, atol=1e-12)
    # the src field's gradient: sum over its out-edges of dout[dst] W (first 3 columns)
    g_edge = dout.numpy()[dst] @ W
    e_src = np.zeros((25, 3))
    np.add.at(e_src, col, g_edge[:, :3])
    np.testing.assert_allclose(gin[0].numpy(), e_src, rtol=1e-12, atol=1e-12)

    net2 = nn.Sequential(nn.Linear(6, 5), nn.Tanh(), nn.Linear(5, 1)).double()
    value = rng.standard_normal((25, 4))
    dout2 = rng.standard_normal((30, 4))
    out2, gin2, gv2, gp2 = eager_torch.nn_attention(rpt, colt, inputs, net2,
                                                    torch.tensor(value), torch.tensor(dout2))
    layers = [(net2[0].weight.detach().numpy(), net2[0].bias.detach().numpy(), "tanh", 0.0),
              (net2[2].weight.detach().numpy(), net2[2].bias.detach().numpy(), "identity", 0.0)]
    np_inputs = [("src", xs), ("dst", xd), ("edge", xe)]
    e_out, _ = ref.nn_attention_fwd(rp, col, np_inputs, layers, value)
    e_din, e_dv, e_grads = ref.nn_attention_bwd(rp, col, np_inputs, layers, value, dout2)
    np.testing.assert_allclose(out2.numpy(), e_out, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(gv2.numpy(), e_dv, rtol=1e-10, atol=1e-12)
    for g, w in zip(gin2, e_din):
        np.testing.assert_allclose(g.numpy(), w, rtol=1e-10, atol=1e-12)
    for (gw, gb), (ew, eb) in zip(zip(gp2[0::2], gp2[1::2]), e_grads):
        np.testing.assert_allclose(gw.numpy(), ew, rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(gb.numpy(), eb, rtol=1e-10, atol=1e-11)

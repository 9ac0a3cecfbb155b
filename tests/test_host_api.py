"""CPU tests of the user-facing API added on top of the call form: ``ndata=``,
``prepare()``, the guarded warm-call cache's bookkeeping, the degree
statistics, ``planning_key``, the materialized ``Graph.cat`` and the
reference planner report.  Everything here runs on CPU tensors (the eager
evaluator) and the host-only parts of the C ABI."""

import numpy as np
import pytest
import torch

import tiga as tg
from oracle import planner, ref

from graphs import skewed_csr


class WeightedSum(tg.MessagePassing):
    reducer = tg.sum()

    def edge(self, src, dst, edge):
        return edge.w * src.x


def _graph(seed=0, n_dst=40, n_src=40, **kw):
    rp, col = skewed_csr(seed, n_dst, n_src, **kw)
    return tg.Graph.from_csr(torch.tensor(rp), torch.tensor(col), num_src=n_src), rp, col


def test_ndata_binds_both_roles_on_a_homogeneous_graph():
    g, rp, col = _graph(1)
    x = torch.randn(40, 3, dtype=torch.float64)
    w = torch.rand(g.num_edges, 1, dtype=torch.float64)

    class Mix(tg.MessagePassing):
        reducer = tg.sum()

        def edge(self, src, dst, edge):
            return edge.w * (src.x - dst.x)

    k = Mix()
    a = k(graph=g, ndata={"x": x}, edge={"w": w})
    b = k(graph=g, src={"x": x}, dst={"x": x}, edge={"w": w})
    assert torch.equal(a, b)
    dst_idx = ref.destination_index(rp)
    want = np.zeros((40, 3))
    np.add.at(want, dst_idx, w.numpy() * (x.numpy()[col] - x.numpy()[dst_idx]))
    assert np.allclose(a.numpy(), want, rtol=1e-12, atol=1e-12)


def test_ndata_errors_follow_the_reference():
    g, _, _ = _graph(2)
    x = torch.randn(40, 2)
    with pytest.raises(TypeError, match="cannot be combined"):
        WeightedSum()(graph=g, ndata={"x": x}, src={"x": x}, edge={})
    with pytest.raises(TypeError, match="requires ndata= or both"):
        WeightedSum()(graph=g, src={"x": x})
    bip, _, _ = _graph(3, n_dst=30, n_src=40)
    with pytest.raises(ValueError, match="homogeneous"):
        WeightedSum()(graph=bip, ndata={"x": x})


def test_prepare_requires_a_hip_launch():
    g, _, _ = _graph(4)
    x = torch.randn(40, 2)
    w = torch.rand(g.num_edges)
    with pytest.raises(NotImplementedError, match=r"ran cpu \(torch.sparse.mm\)"):
        WeightedSum().prepare(graph=g, src={"x": x}, dst={}, edge={"w": w[:, None]})


@pytest.mark.parametrize("x_shape,w_shape", [((40, 3), (None,)), ((40,), (None, 1))])
def test_host_weighted_sum_runs_the_reference_sparse_dispatch(x_shape, w_shape):
    """edge.w * src.x on host tensors: one sparse CSR matrix of the weights
    times the features, as the reference dispatches it
    (interop/torch/message_passing.py:3284-3345); values and both gradients
    against an fp64 brute force; an unweighted sum and mixed dtypes stay on
    the eager evaluator, as in the reference."""
    rng = np.random.default_rng(6)
    rows = [np.sort(rng.choice(40, size=d, replace=False)) for d in rng.integers(0, 9, 50)]
    rows[7] = np.arange(40)   # a row over every source
    rp = np.concatenate([[0], np.cumsum([r.size for r in rows])])
    col = np.concatenate(rows)
    g = tg.Graph.from_csr(torch.tensor(rp), torch.tensor(col), num_src=40)
    x = torch.randn(*x_shape, dtype=torch.float64, requires_grad=True)
    w = torch.rand(*[g.num_edges if d is None else d for d in w_shape], dtype=torch.float64,
                   requires_grad=True)
    k = WeightedSum()
    out = k(graph=g, src={"x": x}, dst={}, edge={"w": w})
    assert k.last_variant.provider == "torch.sparse.mm" and out.shape[1:] == x.shape[1:]
    dst = np.repeat(np.arange(50), np.diff(rp))
    xe = x.detach().numpy().reshape(40, -1)[col]
    we = w.detach().numpy().reshape(-1, 1)
    want = np.zeros((50, xe.shape[1]))
    np.add.at(want, dst, we * xe)
    np.testing.assert_allclose(out.detach().numpy().reshape(50, -1), want, rtol=1e-12,
                               atol=1e-12)
    dout = torch.randn(out.shape, dtype=torch.float64)
    out.backward(dout)
    d2 = dout.numpy().reshape(50, -1)
    dw = (d2[dst] * xe).sum(1)
    dx = np.zeros((40, xe.shape[1]))
    np.add.at(dx, col, we * d2[dst])
    np.testing.assert_allclose(w.grad.numpy().reshape(-1), dw, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(x.grad.numpy().reshape(40, -1), dx, rtol=1e-12, atol=1e-12)

    class Plain(tg.MessagePassing):
        reducer = tg.sum()

        def edge(self, src, dst, edge):
            return src.x

    p = Plain()
    p(graph=g, src={"x": x}, dst={})
    assert p.last_variant.backend == "torch-eager"
    k(graph=g, src={"x": x.detach().float()}, dst={}, edge={"w": w.detach().reshape(-1, 1)})
    assert k.last_variant.backend == "torch-eager"
    # Repeated (row, column) pairs: sparse without a weight gradient, eager
    # with one.
    gm = tg.Graph.from_csr(torch.tensor([0, 3, 4]), torch.tensor([1, 1, 0, 1]), num_src=2)
    xm = torch.tensor([[1.0], [2.0]], dtype=torch.float64)
    wm = torch.tensor([[1.0], [2.0], [3.0], [4.0]], dtype=torch.float64)
    torch.testing.assert_close(k(graph=gm, src={"x": xm}, dst={}, edge={"w": wm}),
                               torch.tensor([[9.0], [8.0]], dtype=torch.float64))
    assert k.last_variant.provider == "torch.sparse.mm"
    wm.requires_grad_(True)
    k(graph=gm, src={"x": xm}, dst={}, edge={"w": wm}).sum().backward()
    assert k.last_variant.backend == "torch-eager"
    torch.testing.assert_close(wm.grad,
                               torch.tensor([[2.0], [2.0], [1.0], [2.0]], dtype=torch.float64))


def test_cache_info_counts_cold_calls_on_the_eager_path():
    g, _, _ = _graph(5)
    x = torch.randn(40, 2)
    w = torch.rand(g.num_edges, 1)
    k = WeightedSum()
    for _ in range(3):
        k(graph=g, src={"x": x}, dst={}, edge={"w": w})
    info = k.cache_info
    assert info == {"hits": 0, "misses": 3, "variants": 1}
    assert "variant cache: hits=0, misses=3" in k.explain()
    with pytest.raises(KeyError):
        k.last_variant.code("ptx")


def test_degree_statistics_histogram_and_span_ratio_against_brute_force():
    g, rp, col = _graph(6, n_dst=300, n_src=250, hubs=(90, 70))
    deg = np.diff(rp)
    assert g.degree_bounds() == (int(deg.min()), int(deg.max()))
    assert g.degree_statistics() == (int(deg.min()), int(deg.max()), int(deg.sum()))
    hist = g.degree_histogram()
    assert isinstance(hist, tuple)
    assert list(hist) == np.bincount(deg, minlength=deg.max() + 1).tolist()
    # span ratio: mean |col - row| over evenly spaced slots, normalised
    E = col.size
    count = min(4096, E)
    slots = np.floor(np.arange(count) * ((E - 1) / (count - 1))).astype(np.int64)
    rows = np.searchsorted(rp[1:], slots, side="right")
    want = np.abs(col[slots] - rows).mean() / max(1, 250, 300)
    assert abs(g.source_index_span_ratio() - want) < 1e-12
    # a ring relation (col = row) is perfectly local
    ring = tg.Graph.from_csr(torch.arange(11), torch.arange(10), num_src=10)
    assert ring.source_index_span_ratio() == 0.0


def test_degree_statistics_of_implicit_relations_are_closed_forms():
    tri = tg.Graph.triangular(7)
    assert tri.degree_statistics() == (1, 7, 28)
    assert tri.degree_histogram() == (0, 1, 1, 1, 1, 1, 1, 1)
    dense = tg.Graph.dense(5, 3)
    assert dense.degree_statistics() == (5, 5, 15)
    assert dense.degree_histogram() == (0, 0, 0, 0, 0, 3)
    cu = torch.tensor([0, 3, 3, 7])
    var = tg.Graph.cu_seqlens(cu, causal=True)
    assert var.degree_statistics() == (1, 4, 6 + 10)
    assert var.degree_histogram() == (0, 2, 2, 2, 1)
    full = tg.Graph.cu_seqlens(cu, causal=False)
    assert full.degree_statistics() == (3, 4, 9 + 16)
    assert full.degree_histogram() == (0, 0, 0, 3, 4)
    # the implicit statistics equal those of the materialized CSR
    rp, _ = ref.cu_seqlens_csr(cu.numpy(), causal=True)
    deg = np.diff(rp)
    assert var.degree_statistics() == (int(deg.min()), int(deg.max()), int(deg.sum()))


def test_degree_histogram_limit():
    rp = torch.tensor([0, 5000])
    g = tg.Graph.from_csr(rp, torch.zeros(5000, dtype=torch.int64), num_src=1)
    with pytest.raises(ValueError, match="4096"):
        g.degree_histogram()


def test_planning_key_carries_degree_statistics_and_locality():
    g, rp, _ = _graph(7)
    key = g.planning_key()
    deg = np.diff(rp)
    assert (int(deg.min()), int(deg.max()), int(deg.sum())) in key
    assert g.source_index_span_ratio() in key
    assert key == g.planning_key()
    other, _, _ = _graph(8)
    assert other.planning_key() != key


def test_materialized_cat_matches_block_diagonal_brute_force():
    blocks, shift_e, shift_s = [], 0, 0
    want_rp, want_col = [0], []
    for seed, (nd, ns) in enumerate([(5, 7), (0, 3), (9, 4), (6, 6)]):
        rp, col = skewed_csr(seed + 20, nd, ns, mean_deg=3)
        blocks.append(tg.Graph.from_csr(torch.tensor(rp, dtype=torch.int32),
                                        torch.tensor(col, dtype=torch.int32), num_src=ns))
        want_rp += (rp[1:] + shift_e).tolist()
        want_col += (col + shift_s).tolist()
        shift_e += int(rp[-1])
        shift_s += ns
    g = tg.Graph.cat(blocks)
    rp, col = g.resolve_csr()
    assert rp.dtype == torch.int32
    assert rp.tolist() == want_rp and col.tolist() == want_col
    assert g.schema.num_src == shift_s and g.schema.num_dst == 20


@pytest.mark.parametrize("case", [
    dict(seed=0, n_dst=128, n_src=128, mean_deg=16, empty_frac=0.0),       # regular
    dict(seed=1, n_dst=512, n_src=600, mean_deg=4, hubs=(300, 200, 90)),  # power law
    dict(seed=2, n_dst=100, n_src=100, mean_deg=40, empty_frac=0.7),       # padding-poor
])
@pytest.mark.parametrize("has_node", [False, True])
def test_reference_plan_of_a_graph_matches_the_oracle_planner(case, has_node):
    rp, col = skewed_csr(**case)
    g = tg.Graph.from_csr(torch.tensor(rp), torch.tensor(col), num_src=case["n_src"])
    deg = np.diff(rp)
    hist = np.bincount(deg, minlength=deg.max() + 1).tolist()
    want = planner.plan(len(deg), int(deg.max()), int(deg.sum()), hist, has_node)
    got = g.reference_plan(has_node)
    for key, value in want.items():
        assert got[key] == value, key
    assert got["plan"] in tg.graph.describe_reference_plan(got)


def test_reference_plan_defers_above_the_histogram_limit():
    deg = np.array([5000, 3, 2, 0])
    rp = np.concatenate([[0], np.cumsum(deg)])
    g = tg.Graph.from_csr(torch.tensor(rp), torch.zeros(int(rp[-1]), dtype=torch.int64),
                          num_src=1)
    assert g.reference_plan()["plan"] == "provider-deferred-high-degree"


class Diffusion(tg.MessagePassing):
    """The reference's diffusion example (examples/diffusion.py), unchanged."""

    reducer = tg.sum()

    def edge(self, src, dst, edge):
        return edge.conductivity * (src.u + (-1.0) * dst.u)

    def node(self, dst, flux, dt):
        return dst.u + dt * flux


def test_reference_diffusion_example_with_ndata():
    """examples/diffusion.py: the stated flux and gradients, and the
    reference's ndata test (tests/python/test_reference.py:366-390)."""
    row_ptr = torch.tensor([0, 2, 4, 6, 8], dtype=torch.int64)
    col_idx = torch.tensor([3, 1, 0, 2, 1, 3, 2, 0], dtype=torch.int64)
    graph = tg.Graph.from_csr(row_ptr, col_idx, num_src=4, validate="full")
    u = torch.tensor([0.0, 1.0, 0.5, -0.5], requires_grad=True)
    conductivity = torch.tensor([1.0] * 8, requires_grad=True)
    next_u = Diffusion()(graph=graph, ndata={"u": u}, edge={"conductivity": conductivity},
                         dt=0.1)
    flux = torch.tensor([0.5, -1.5, -0.5, 1.5])
    torch.testing.assert_close(next_u, u.detach() + 0.1 * flux)
    du, dc = torch.autograd.grad(next_u.sum(), (u, conductivity))
    torch.testing.assert_close(du, torch.ones(4))
    dst = np.repeat(np.arange(4), 2)
    want = 0.1 * (u.detach().numpy()[col_idx.numpy()] - u.detach().numpy()[dst])
    torch.testing.assert_close(dc, torch.tensor(want, dtype=torch.float32))
    via_roles = Diffusion()(graph=graph, src={"u": u}, dst={"u": u},
                            edge={"conductivity": conductivity}, dt=0.1)
    torch.testing.assert_close(next_u, via_roles)
    with pytest.raises(TypeError, match="cannot be combined"):
        Diffusion()(graph=graph, ndata={"u": u}, dst={}, edge={})


def test_raw_score_softmax_recognition():
    from tiga import capture as cap

    class Attn(tg.MessagePassing):
        reducer = tg.online_softmax()

        def __init__(self, form):
            super().__init__()
            self.form = form

        def edge(self, src, dst, edge, t=2.0):
            score = {"src": src.s, "edge": edge.s * 0.5, "dst": -dst.s, "div": edge.s / t,
                     "sum": src.s + dst.s}[self.form]
            return self.reducer(score, src.v)

    want = {"src": ("src", 1.0), "edge": ("edge", 0.5), "dst": ("dst", -1.0),
            "div": ("edge", 0.5)}
    for form, (role, scale) in want.items():
        got = cap.recognize_score_softmax(Attn(form)._captured({"t": 2.0}))
        assert got == cap.ScoreSoftmax(role, "s", scale, "v"), form
    assert cap.recognize_score_softmax(Attn("sum")._captured({})) is None


def test_raw_score_softmax_known_answer_on_cpu_eager():
    """The reference's known answer on the eager evaluator (CPU tensors)."""
    import json
    from pathlib import Path

    g = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
    g = g["online_softmax_large_scores"]

    class OnlineAttention(tg.MessagePassing):
        reducer = tg.online_softmax()

        def edge(self, src, dst, edge):
            return self.reducer(src.score, src.value)

    graph = tg.Graph.from_csr(torch.tensor(g["row_ptr"]), torch.tensor(g["col_idx"]),
                              num_src=g["num_src"])
    score = torch.tensor(g["score"], requires_grad=True)
    value = torch.tensor(g["value"], requires_grad=True)
    out = OnlineAttention()(graph=graph, src={"score": score, "value": value}, dst={})
    dscore, dvalue = torch.autograd.grad(out.sum(), (score, value))
    np.testing.assert_allclose(out.detach().numpy(), g["out"], atol=5e-6, rtol=0)
    np.testing.assert_allclose(dscore.numpy(), g["dscore"], atol=5e-6, rtol=0)
    np.testing.assert_allclose(dvalue.numpy(), g["dvalue"], atol=5e-6, rtol=0)


def test_kernel_observability_surface_matches_the_reference():
    """ir("domain"), code(), diagnostics and schedules (reference
    kernel/model.py:113-195) on an eager-path call."""
    import tiga.kernel as tk

    class Copy(tg.MessagePassing):
        reducer = tg.sum()

        def edge(self, src, dst, edge):
            return src.x

    g = tg.Graph.from_csr(torch.tensor([0, 1, 2]), torch.tensor([1, 0]), num_src=2)
    k = Copy()
    k(graph=g, src={"x": torch.ones(2, 3)}, dst={})
    assert "backend:" in k.ir("domain") and k.ir() == k.ir("domain-plan")
    with pytest.raises(KeyError):
        k.ir("gf.kernel")
    with pytest.raises(KeyError):
        k.code()
    assert all(isinstance(f, tk.AnalysisFinding) for f in k.diagnostics)
    assert k.schedules == ()
    with pytest.raises(ValueError):
        tk.AnalysisFinding("planning", "maybe", "x")


GUARD_SCALE = 0.5


def test_warm_call_environment_tracks_outside_scalars():
    """The guard of a warm launch snapshots the scalars edge() reads from
    outside the call (instance and class attributes, module globals,
    closure cells) and fails when any changes; tensors and other objects
    are not part of it (they are operands or re-captured)."""
    global GUARD_SCALE
    from tiga.message_passing import _Environment

    offset = 1.0

    class K(tg.MessagePassing):
        reducer = tg.online_softmax()
        slope = 0.2
        weights = torch.ones(3)

        def edge(self, src, dst, edge):
            s = (src.k * dst.q).sum(-1) * GUARD_SCALE * self.slope + offset
            return self.reducer(s * self.weights.sum(), src.v)

    k = K()
    env = _Environment(k)
    kinds = {key for key in env.keys}
    assert ("attr", "slope") in kinds and ("global", "GUARD_SCALE") in kinds
    assert any(kind == "cell" for kind, _ in kinds)
    assert ("attr", "weights") not in kinds and ("attr", "reducer") not in kinds
    assert env.holds(k)
    k.slope = 0.2
    assert env.holds(k)
    k.slope = 0.3
    assert not env.holds(k)
    del k.slope
    assert env.holds(k)
    K.slope = 0.25
    assert not env.holds(k)
    K.slope = 0.2
    GUARD_SCALE = 0.75
    try:
        assert not env.holds(k)
    finally:
        GUARD_SCALE = 0.5
    assert env.holds(k)
    offset = 2.0          # the closure cell edge() reads
    assert not env.holds(k)
    offset = 1.0
    assert env.holds(k)
    k.slope = 1           # an int where a float was baked in
    assert not env.holds(k)

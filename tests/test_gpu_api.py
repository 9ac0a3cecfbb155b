"""GPU tests of the call forms around the HIP launches: field validation
before any launch, ``ndata=``, ``prepare()`` and the guarded warm-call cache
(every warm or prepared result bit-identical to a cold call), and the
reference planner report in ``explain()``."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import tiga as tg
from tiga import _native

from graphs import skewed_csr

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


@pytest.fixture(autouse=True)
def _strict():
    tg.config.strict = True
    yield
    tg.config.strict = False


class WeightedSum(tg.MessagePassing):
    reducer = tg.sum()

    def edge(self, src, dst, edge):
        return edge.w * src.x


class Dot(tg.MessagePassing):
    reducer = tg.online_softmax()

    def edge(self, src, dst, edge, scale):
        return self.reducer((src.k * dst.q).sum(dim=-1) * scale + edge.b, src.v)


class GatParams(tg.MessagePassing):
    reducer = tg.online_softmax()

    def edge(self, src, dst, edge, a_src, a_dst):
        s = F.leaky_relu((src.h * a_src).sum(-1) + (dst.h * a_dst).sum(-1), 0.2)
        return self.reducer(s, src.h)


def _graph(seed=0, n=3000, hubs=(900,), idx=torch.int64):
    rp, col = skewed_csr(seed, n, n, mean_deg=7, hubs=hubs)
    return tg.Graph.from_csr(torch.tensor(rp, device=DEV, dtype=idx),
                             torch.tensor(col, device=DEV, dtype=idx), num_src=n)


def test_host_edge_fields_are_rejected_before_any_launch():
    print("host edge fields", flush=True)
    g = _graph(1)
    x = torch.randn(3000, 8, device=DEV)
    with pytest.raises(ValueError, match="edge.w is on cpu"):
        WeightedSum()(graph=g, src={"x": x}, dst={}, edge={"w": torch.rand(g.num_edges)})
    q = torch.randn(3000, 2, 64, device=DEV).to(torch.bfloat16)
    with pytest.raises(ValueError, match="edge.b is on cpu"):
        Dot()(graph=g, src={"k": q, "v": q}, dst={"q": q},
              edge={"b": torch.randn(g.num_edges, 2)}, scale=0.125)
    with pytest.raises(ValueError, match="leading dimension"):
        WeightedSum()(graph=g, src={"x": x}, dst={},
                      edge={"w": torch.rand(g.num_edges + 1, device=DEV)})
    torch.cuda.synchronize()


def test_nn_score_width_mismatch_is_not_launched():
    print("nn width mismatch", flush=True)
    g = _graph(2)
    net = torch.nn.Sequential(torch.nn.Linear(5, 8), torch.nn.ReLU(),
                              torch.nn.Linear(8, 1)).to(DEV)

    class NnAttn(tg.MessagePassing):
        reducer = tg.online_softmax()

        def edge(self, src, dst, edge):
            return self.reducer(tg.nn.trace(net)(src.p, dst.p), src.v)

    p = torch.randn(3000, 3, device=DEV)    # 3 + 3 inputs for a 5-wide network
    v = torch.randn(3000, 4, device=DEV)
    tg.config.strict = False
    with pytest.raises(RuntimeError):
        NnAttn()(graph=g, src={"p": p, "v": v}, dst={"p": p})


def test_ndata_equals_src_dst_on_the_hip_path():
    print("ndata", flush=True)
    g = _graph(3)
    h = torch.randn(3000, 4, 32, device=DEV)
    a_s = 0.1 * torch.randn(4, 32, device=DEV)
    a_d = 0.1 * torch.randn(4, 32, device=DEV)
    k = GatParams()
    a = k(graph=g, ndata={"h": h}, a_src=a_s, a_dst=a_d)
    assert k.last_variant.backend == "hip"
    b = GatParams()(graph=g, src={"h": h}, dst={"h": h}, a_src=a_s, a_dst=a_d)
    assert torch.equal(a, b)


@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
def test_warm_calls_hit_the_guarded_launch_and_match_cold_calls(idx):
    print(f"guarded weighted sum {idx}", flush=True)
    g = _graph(4, idx=idx)
    x = torch.randn(3000, 16, device=DEV, requires_grad=True)
    w = torch.rand(g.num_edges, 1, device=DEV, requires_grad=True)
    k = WeightedSum()
    outs, grads = [], []
    for _ in range(3):
        x.grad = w.grad = None
        out = k(graph=g, src={"x": x}, dst={}, edge={"w": w})
        out.backward(torch.ones_like(out))
        outs.append(out.detach())
        grads.append((x.grad.clone(), w.grad.clone()))
    assert k.cache_info["misses"] == 1 and k.cache_info["hits"] == 2
    assert k.last_variant.backend == "hip"
    cold = WeightedSum()(graph=g, src={"x": x}, dst={}, edge={"w": w})
    for o, (gx, gw) in zip(outs, grads):
        assert torch.equal(o, cold.detach())
        assert torch.equal(gx, grads[0][0]) and torch.equal(gw, grads[0][1])
    # a different shape, dtype-preserving: the guard misses, the result is right
    x2 = torch.randn(3000, 8, device=DEV)
    out2 = k(graph=g, src={"x": x2}, dst={}, edge={"w": w})
    assert k.cache_info["misses"] == 2
    assert torch.equal(out2, WeightedSum()(graph=g, src={"x": x2}, dst={}, edge={"w": w}))
    # a different graph object misses too
    g2 = _graph(4, idx=idx)
    k(graph=g2, src={"x": x2}, dst={}, edge={"w": w})
    assert k.cache_info["misses"] == 3


def test_tensor_parameters_are_read_from_each_warm_call():
    print("guarded gat params", flush=True)
    g = _graph(5)
    h = torch.randn(3000, 4, 32, device=DEV)
    a_s = 0.1 * torch.randn(4, 32, device=DEV)
    a_d = 0.1 * torch.randn(4, 32, device=DEV)
    k = GatParams()
    first = k(graph=g, src={"h": h}, dst={"h": h}, a_src=a_s, a_dst=a_d)
    a_s2 = 0.1 * torch.randn(4, 32, device=DEV)
    warm = k(graph=g, src={"h": h}, dst={"h": h}, a_src=a_s2, a_dst=a_d)
    assert k.cache_info["hits"] == 1
    cold = GatParams()(graph=g, src={"h": h}, dst={"h": h}, a_src=a_s2, a_dst=a_d)
    assert torch.equal(warm, cold) and not torch.equal(warm, first)
    # a scalar parameter baked into the capture: a new value is a cold call
    kd = Dot()
    q = torch.randn(3000, 2, 64, device=DEV).to(torch.bfloat16)
    b = torch.randn(g.num_edges, 2, device=DEV)
    o1 = kd(graph=g, src={"k": q, "v": q}, dst={"q": q}, edge={"b": b}, scale=0.125)
    o2 = kd(graph=g, src={"k": q, "v": q}, dst={"q": q}, edge={"b": b}, scale=0.25)
    assert kd.cache_info == {"hits": 0, "misses": 2, "variants": 1}
    assert torch.equal(o2, Dot()(graph=g, src={"k": q, "v": q}, dst={"q": q}, edge={"b": b},
                                 scale=0.25))
    assert not torch.equal(o1, o2)


SCORE_SCALE = 0.125


class GatSlopeAttr(tg.MessagePassing):
    reducer = tg.online_softmax()
    slope = 0.2

    def edge(self, src, dst, edge, a_src, a_dst):
        s = F.leaky_relu((src.h * a_src).sum(-1) + (dst.h * a_dst).sum(-1), self.slope)
        return self.reducer(s, src.h)


def _with_slope(slope):
    k = GatSlopeAttr()
    k.slope = slope
    return k


class DotGlobalScale(tg.MessagePassing):
    reducer = tg.online_softmax()

    def edge(self, src, dst, edge):
        return self.reducer((src.k * dst.q).sum(dim=-1) * SCORE_SCALE + edge.b, src.v)


def test_outside_scalars_changed_between_warm_calls_are_seen():
    """A slope or scale edge() reads from the kernel's attributes, its class,
    a module global or a closure is baked into the capture: changing it
    makes the next call a cold one, whose result is the new value's."""
    global SCORE_SCALE
    print("outside scalars", flush=True)
    g = _graph(7)
    h = torch.randn(3000, 4, 32, device=DEV)
    a_s = 0.1 * torch.randn(4, 32, device=DEV)
    a_d = 0.1 * torch.randn(4, 32, device=DEV)
    call = lambda k: k(graph=g, src={"h": h}, dst={"h": h}, a_src=a_s, a_dst=a_d)
    k = GatSlopeAttr()
    first = call(k)
    assert torch.equal(call(k), first) and k.cache_info["hits"] == 1
    k.slope = 0.2                                    # same value: still a hit
    call(k)
    assert k.cache_info == {"hits": 2, "misses": 1, "variants": 1}
    k.slope = 0.01                                   # instance attribute
    second = call(k)
    assert k.cache_info["misses"] == 2 and k.last_variant.backend == "hip"
    assert torch.equal(second, call(_with_slope(0.01)))
    assert not torch.equal(first, second)
    k2 = GatSlopeAttr()
    call(k2)
    try:                                             # class attribute
        GatSlopeAttr.slope = 0.05
        third = call(k2)
        assert k2.cache_info["misses"] == 2
        assert torch.equal(third, call(_with_slope(0.05)))
        assert not torch.equal(third, first)
    finally:
        GatSlopeAttr.slope = 0.2

    q = torch.randn(3000, 2, 64, device=DEV).to(torch.bfloat16)
    b = torch.randn(g.num_edges, 2, device=DEV)
    fields = dict(graph=g, src={"k": q, "v": q}, dst={"q": q}, edge={"b": b})
    kd = DotGlobalScale()
    o1 = kd(**fields)
    try:                                             # module global
        SCORE_SCALE = 0.25
        o2 = kd(**fields)
        assert kd.cache_info["misses"] == 2 and kd.last_variant.backend == "hip"
        assert torch.equal(o2, DotGlobalScale()(**fields)) and not torch.equal(o1, o2)
    finally:
        SCORE_SCALE = 0.125

    def closure_kernel():
        scale = 0.125

        class DotClosure(tg.MessagePassing):
            reducer = tg.online_softmax()

            def edge(self, src, dst, edge):
                return self.reducer((src.k * dst.q).sum(dim=-1) * scale + edge.b, src.v)

        def set_scale(value):
            nonlocal scale
            scale = value
        return DotClosure(), set_scale

    kc, set_scale = closure_kernel()
    c1 = kc(**fields)
    assert torch.equal(c1, o1)
    set_scale(0.25)                                  # closure cell
    c2 = kc(**fields)
    assert kc.cache_info["misses"] == 2 and torch.equal(c2, o2)


def test_closure_tensors_are_recaptured_every_call():
    print("closure tensors", flush=True)
    g = _graph(6)
    h = torch.randn(3000, 4, 32, device=DEV)
    holder = {"a": 0.1 * torch.randn(4, 32, device=DEV)}

    class Gat(tg.MessagePassing):
        reducer = tg.online_softmax()

        def edge(self, src, dst, edge):
            s = F.leaky_relu((src.h * holder["a"]).sum(-1) + (dst.h * holder["a"]).sum(-1))
            return self.reducer(s, src.h)

    k = Gat()
    first = k(graph=g, src={"h": h}, dst={"h": h})
    holder["a"] = 0.1 * torch.randn(4, 32, device=DEV)
    second = k(graph=g, src={"h": h}, dst={"h": h})
    assert k.cache_info["hits"] == 0
    a = holder["a"]

    class GatFixed(tg.MessagePassing):
        reducer = tg.online_softmax()

        def edge(self, src, dst, edge):
            s = F.leaky_relu((src.h * a).sum(-1) + (dst.h * a).sum(-1))
            return self.reducer(s, src.h)

    assert torch.equal(second, GatFixed()(graph=g, src={"h": h}, dst={"h": h}))
    assert not torch.equal(first, second)


def test_no_grad_launch_matches_autograd_launch():
    """Calls whose operands need no gradient launch the kernels without an
    autograd node; the result is the same launch's, bit for bit."""
    print("no-grad launch", flush=True)
    g = _graph(11)
    x = torch.randn(3000, 5, device=DEV)
    w = torch.rand(g.num_edges, device=DEV)
    plain = WeightedSum()(graph=g, src={"x": x}, dst={}, edge={"w": w})
    assert plain.grad_fn is None
    xg = x.clone().requires_grad_(True)
    tracked = WeightedSum()(graph=g, src={"x": xg}, dst={}, edge={"w": w})
    assert tracked.grad_fn is not None
    assert torch.equal(plain, tracked.detach())

    class ScoreSoftmax(tg.MessagePassing):
        reducer = tg.online_softmax()

        def edge(self, src, dst, edge):
            return self.reducer(src.s, src.v)

    s, v = torch.randn(3000, device=DEV), torch.randn(3000, 3, device=DEV)
    k = ScoreSoftmax()
    plain = k(graph=g, src={"s": s, "v": v}, dst={})
    assert k.last_variant.backend == "hip" and plain.grad_fn is None
    sg = s.clone().requires_grad_(True)
    tracked = ScoreSoftmax()(graph=g, src={"s": sg, "v": v}, dst={})
    assert torch.equal(plain, tracked.detach())
    tracked.sum().backward()
    assert sg.grad is not None and torch.isfinite(sg.grad).all()
    # GAT: a forward that a backward may follow also accumulates the
    # positive-branch rows (another instantiation of the same online
    # softmax); its output is the no-grad launch's to fp32 rounding.
    h = torch.randn(3000, 4, 32, device=DEV)
    a_s, a_d = 0.1 * torch.randn(4, 32, device=DEV), 0.1 * torch.randn(4, 32, device=DEV)
    gk = GatParams()
    plain = gk(graph=g, src={"h": h}, dst={"h": h}, a_src=a_s, a_dst=a_d)
    assert gk.last_variant.backend == "hip" and plain.grad_fn is None
    hg = h.clone().requires_grad_(True)
    tracked = GatParams()(graph=g, src={"h": hg}, dst={"h": hg}, a_src=a_s, a_dst=a_d)
    assert tracked.grad_fn is not None
    diff = (plain - tracked.detach()).abs().max().item() / plain.abs().max().item()
    print(f"  GAT no-grad vs autograd forward: max diff / max {diff:.2e}", flush=True)
    assert diff <= 1e-6
    # prepare() binds the native arguments of a no-grad sum; a strided x
    # (which the launch would copy) stays on the per-call path; both see
    # in-place updates, and a gradient requested later gets autograd.
    for xs in (torch.randn(3000, 5, device=DEV), torch.randn(3000, 10, device=DEV)[:, ::2]):
        launch = WeightedSum().prepare(graph=g, src={"x": xs}, dst={}, edge={"w": w})
        first = launch()
        assert torch.equal(first, WeightedSum()(graph=g, src={"x": xs}, dst={}, edge={"w": w}))
        xs.mul_(2.0)
        assert torch.equal(launch(), WeightedSum()(graph=g, src={"x": xs}, dst={},
                                                   edge={"w": w}))
        w.requires_grad_(True)
        again = launch()
        assert again.grad_fn is not None
        again.sum().backward()
        assert w.grad is not None
        w.grad = None
        w.requires_grad_(False)


def test_prepare_is_bit_identical_and_sees_in_place_updates():
    print("prepare", flush=True)
    g = _graph(7)
    x = torch.randn(3000, 16, device=DEV)
    w = torch.rand(g.num_edges, device=DEV)

    class Shifted(WeightedSum):
        def node(self, dst, aggregate, shift):
            return aggregate + shift

    k = Shifted()
    launch = k.prepare(graph=g, src={"x": x}, dst={}, edge={"w": w}, shift=2.0)
    assert launch.variant.backend == "hip" and launch.graph is g
    eager = Shifted()(graph=g, src={"x": x}, dst={}, edge={"w": w}, shift=2.0)
    assert torch.equal(launch(), eager)
    x.mul_(3.0)
    again = launch()
    assert torch.equal(again, Shifted()(graph=g, src={"x": x}, dst={}, edge={"w": w},
                                        shift=2.0))
    assert not torch.equal(again, eager)
    # nn-scored attention (operands from outside the call) can still be prepared
    net = torch.nn.Sequential(torch.nn.Linear(6, 16), torch.nn.Tanh(),
                              torch.nn.Linear(16, 1)).to(DEV)

    class NnAttn(tg.MessagePassing):
        reducer = tg.online_softmax()

        def edge(self, src, dst, edge):
            return self.reducer(tg.nn.trace(net)(src.p, dst.p), src.v)

    p = torch.randn(3000, 3, device=DEV)
    v = torch.randn(3000, 4, device=DEV)
    kn = NnAttn()
    run = kn.prepare(graph=g, src={"p": p, "v": v}, dst={"p": p})
    assert torch.equal(run(), NnAttn()(graph=g, src={"p": p, "v": v}, dst={"p": p}))


def test_explain_reports_the_row_plan_and_the_reference_planner():
    print("explain", flush=True)
    g = _graph(8, hubs=(900, 120))
    x = torch.randn(3000, 4, device=DEV)
    w = torch.rand(g.num_edges, device=DEV)
    k = WeightedSum()
    k(graph=g, src={"x": x}, dst={}, edge={"w": w})
    text = k.explain()
    assert "row plan:" in text
    assert "reference planner: high-degree-tail-chunked" in text, text
    assert "reference planner" in g.explain()

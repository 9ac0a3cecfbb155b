"""GPU parity of nn-scored edge attention (tg.nn.trace score networks) on the
HIP edge-MLP kernels against the fp64 oracle: outputs and the gradients of
every input field, the value and every weight and bias.

Tolerance (fp32 path): max|gpu - oracle| <= 1e-5 * max|oracle| per tensor;
weight and bias gradients, which sum over every edge, 3e-5 (bias gradients in
the scale of their layer's weight gradient: the last bias's exact gradient
is 0).
"""

import numpy as np
import pytest
import torch
from torch import nn

import tiga as tg
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
RTOL = 1e-5


def rel_err(actual, expected):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


def f64(t):
    return t.detach().double().cpu().numpy()


def random_graph(n_dst, n_src, mean_deg, seed, hub=0, empty=0.1):
    rng = np.random.default_rng(seed)
    deg = rng.poisson(mean_deg, n_dst)
    deg[rng.random(n_dst) < empty] = 0
    if hub:
        deg[n_dst // 2] = hub
    rp = np.concatenate([[0], np.cumsum(deg)])
    col = rng.integers(0, n_src, int(rp[-1]))
    return torch.as_tensor(rp, device=DEV), torch.as_tensor(col, device=DEV)


class GAT(tg.MessagePassing):
    """The reference example's kernel (examples/gat_edge_attention.py:18-29),
    with the displacement given as an explicit edge field."""

    reducer = tg.online_softmax()

    def __init__(self, attn):
        super().__init__()
        self.attn = tg.nn.trace(attn)

    def edge(self, src, dst, edge):
        return self.reducer(self.attn(edge.displacement, src.x, dst.x), src.x)


def layers_of(net):
    out, acts = [], []
    mods = list(net) if isinstance(net, nn.Sequential) else [net]
    for m in mods:
        if isinstance(m, nn.Linear):
            out.append([f64(m.weight), None if m.bias is None else f64(m.bias), "identity", 0.0])
        elif isinstance(m, nn.LeakyReLU):
            out[-1][2:] = ["leaky_relu", m.negative_slope]
        elif isinstance(m, nn.ELU):
            out[-1][2:] = ["elu", m.alpha]
        elif isinstance(m, nn.GELU):
            out[-1][2:] = ["gelu", 0.0]
        else:
            out[-1][2:] = [{nn.ReLU: "relu", nn.Tanh: "tanh", nn.Sigmoid: "sigmoid",
                            nn.SiLU: "silu"}[type(m)], 0.0]
    return [tuple(x) for x in out]


@pytest.fixture(autouse=True)
def strict():
    tg.config.strict = True
    yield
    tg.config.strict = False


def check(graph, kernel, net, inputs, value, fields, dout):
    """Run kernel forward + backward and compare with the oracle."""
    rp, col = (f64(t).astype(np.int64) for t in graph.resolve_csr())
    out = kernel(**fields)
    assert kernel.last_variant.backend == "hip"
    assert kernel.last_variant.pattern == "nn-attention"
    out.backward(dout)
    o_inputs = [(role, f64(t)) for role, t in inputs]
    layers = layers_of(net)
    e_out, _ = ref.nn_attention_fwd(rp, col, o_inputs, layers, f64(value))
    assert rel_err(f64(out), e_out) <= RTOL
    dinputs, dvalue, dlayers = ref.nn_attention_bwd(rp, col, o_inputs, layers, f64(value),
                                                    f64(dout))
    # a tensor used at several places (x as src, dst and value) sums its parts
    expect = {}
    for (role, t), d in zip(inputs, dinputs):
        expect[id(t)] = expect.get(id(t), 0) + d
    expect[id(value)] = expect.get(id(value), 0) + dvalue
    # A field whose score contribution is the same for every edge of a row
    # (dst fields under a single Linear score) has an exact gradient of 0 by
    # softmax shift invariance; gradients are compared in the scale of the
    # largest gradient of the check.
    scale = max(np.abs(g).max() for g in expect.values())
    for role, t in inputs + [("value", value)]:
        err = np.abs(f64(t.grad) - expect[id(t)]).max()
        assert err <= RTOL * max(np.abs(expect[id(t)]).max(), 0.1 * scale), role
    linears = [m for m in (net if isinstance(net, nn.Sequential) else [net])
               if isinstance(m, nn.Linear)]
    for lin, (dW, db) in zip(linears, dlayers):
        assert rel_err(f64(lin.weight.grad), dW) <= 3 * RTOL
        if db is not None:
            # The last layer's bias shifts every score of a row equally, so its
            # exact gradient is 0 (softmax shift invariance): bias gradients are
            # compared in the scale of their layer's weight gradient.
            scale = max(np.abs(db).max(), np.abs(dW).max())
            assert np.abs(f64(lin.bias.grad) - db).max() <= 3 * RTOL * scale


def test_reference_gat_example_shape():
    """nodes 512, f_in 8, hidden 16: Linear(3 + 2*8, 16), LeakyReLU(0.2),
    Linear(16, 1) over [displacement | x_src | x_dst], value x_src."""
    print("nn attention reference example", flush=True)
    torch.manual_seed(0)
    nodes, f_in, hidden = 512, 8, 16
    rp, col = random_graph(nodes, nodes, 7, 1)
    graph = tg.Graph.from_csr(rp, col, num_src=nodes)
    pos = torch.rand(nodes, 3, device=DEV)
    dst_idx = graph.destination_index()
    disp = (pos[col] - pos[dst_idx]).requires_grad_(True)
    x = torch.randn(nodes, f_in, device=DEV, requires_grad=True)
    attn = nn.Sequential(nn.Linear(3 + 2 * f_in, hidden), nn.LeakyReLU(0.2),
                         nn.Linear(hidden, 1)).to(DEV)
    kernel = GAT(attn)
    dout = torch.randn(nodes, f_in, device=DEV)
    check(graph, kernel, attn, [("edge", disp), ("src", x), ("dst", x)], x,
          dict(graph=graph, src={"x": x}, dst={"x": x}, edge={"displacement": disp}), dout)


def test_attention_keeps_no_per_edge_weights():
    """The forward keeps per destination row only its logsumexp and output:
    beside the caller's own per-edge fields, no [E] score, weight or score
    gradient is saved for the backward, which recomputes them per edge."""
    print("nn attention saved state", flush=True)
    torch.manual_seed(1)
    nodes, f_in = 700, 8
    rp, col = random_graph(nodes, nodes, 9, 3, hub=200)
    graph = tg.Graph.from_csr(rp, col, num_src=nodes)
    E = graph.num_edges
    disp = torch.randn(E, 3, device=DEV, requires_grad=True)
    x = torch.randn(nodes, f_in, device=DEV, requires_grad=True)
    attn = nn.Sequential(nn.Linear(3 + 2 * f_in, 16), nn.LeakyReLU(0.2),
                         nn.Linear(16, 1)).to(DEV)
    kernel = GAT(attn)
    out = kernel(graph=graph, src={"x": x}, dst={"x": x}, edge={"displacement": disp})
    assert kernel.last_variant.backend == "hip"
    saved = out.grad_fn.saved_tensors
    per_edge = [tuple(t.shape) for t in saved
                if t.ndim >= 1 and t.shape[0] == E and t.data_ptr() != disp.data_ptr()]
    assert per_edge == [], per_edge
    assert any(tuple(t.shape) == (nodes,) for t in saved)      # the row logsumexp
    dout = torch.randn(nodes, f_in, device=DEV)
    check(graph, kernel, attn, [("edge", disp), ("src", x), ("dst", x)], x,
          dict(graph=graph, src={"x": x}, dst={"x": x}, edge={"displacement": disp}), dout)


@pytest.mark.parametrize("width,acts,hub", [
    (12, ("tanh",), 0),                       # W = 16, two layers
    (40, ("gelu", "silu"), 300),               # W = 64, three layers, hub row > 64 edges
    (24, ("elu", "sigmoid"), 0),               # W = 24, three layers
    (30, ("relu",), 0),                        # W = 32, two layers
    (20, (), 0),                               # one Linear: bias-free linear score
    (16, ("leaky_relu", "leaky_relu"), 120),   # W = 16, three layers: the LeakyReLU kernel
    (24, ("leaky_relu", "tanh"), 0),           # mixed: the runtime activation switch
])
def test_score_chains(width, acts, hub):
    print(f"nn attention chain width={width} acts={acts} hub={hub}", flush=True)
    torch.manual_seed(width)
    n_dst, n_src = 300, 200
    rp, col = random_graph(n_dst, n_src, 9, width, hub=hub)
    graph = tg.Graph.from_csr(rp, col, num_src=n_src)
    E = col.numel()
    xs = torch.randn(n_src, 6, device=DEV, requires_grad=True)
    xd = torch.randn(n_dst, 5, device=DEV, requires_grad=True)
    ef = torch.randn(E, 3, device=DEV, requires_grad=True)
    v = torch.randn(n_src, 10, device=DEV, requires_grad=True)
    mods = []
    dims = [14] + [width] * len(acts) + [1]
    names = {"tanh": nn.Tanh, "gelu": nn.GELU, "silu": nn.SiLU, "elu": lambda: nn.ELU(0.7),
             "sigmoid": nn.Sigmoid, "relu": nn.ReLU,
             "leaky_relu": lambda: nn.LeakyReLU(0.1)}
    for i in range(len(dims) - 1):
        mods.append(nn.Linear(dims[i], dims[i + 1], bias=bool(acts) or i > 0))
        if i < len(acts):
            mods.append(names[acts[i]]())
    net = nn.Sequential(*mods).to(DEV)

    class Scored(tg.MessagePassing):
        reducer = tg.online_softmax()

        def __init__(self):
            super().__init__()
            self.net = tg.nn.trace(net)

        def edge(self, src, dst, edge):
            return self.reducer(self.net(src.a, dst.b, edge.c), src.v)

    dout = torch.randn(n_dst, 10, device=DEV)
    check(graph, Scored(), net, [("src", xs), ("dst", xd), ("edge", ef)], v,
          dict(graph=graph, src={"a": xs, "v": v}, dst={"b": xd}, edge={"c": ef}), dout)


def test_weights_updated_in_place_between_steps():
    """An optimizer updates the network in place between steps; every launch
    must read the current weights (the kernels load them through the scalar
    cache)."""
    print("nn attention: weights updated in place between steps", flush=True)
    torch.manual_seed(3)
    n = 400
    rp, col = random_graph(n, n, 8, 3)
    graph = tg.Graph.from_csr(rp, col, num_src=n)
    x = torch.randn(n, 8, device=DEV, requires_grad=True)
    disp = torch.randn(col.numel(), 3, device=DEV, requires_grad=True)
    net = nn.Sequential(nn.Linear(19, 16), nn.ReLU(), nn.Linear(16, 1)).to(DEV)
    kernel = GAT(net)
    opt = torch.optim.SGD(list(net.parameters()), lr=0.05)
    fields = dict(graph=graph, src={"x": x}, dst={"x": x}, edge={"displacement": disp})
    before = [p.detach().clone() for p in net.parameters()]
    for _ in range(3):
        opt.zero_grad(set_to_none=True)
        kernel(**fields).square().sum().backward()
        opt.step()
    assert all(not torch.equal(a, p) for a, p in zip(before, net.parameters()))
    opt.zero_grad(set_to_none=True)
    x.grad = disp.grad = None
    dout = torch.randn(n, 8, device=DEV)
    check(graph, kernel, net, [("edge", disp), ("src", x), ("dst", x)], x, fields, dout)


def test_uncovered_networks_fall_back_or_refuse():
    """Chains needing more than three layers (identity layers counted), a
    LayerNorm in a chain wider than 32, or widths above 64, are not covered:
    strict mode refuses, otherwise the eager evaluator runs them (reference
    fail-closed rungs)."""
    n = 50
    rp, col = random_graph(n, n, 4, 5)
    graph = tg.Graph.from_csr(rp, col, num_src=n)
    x = torch.randn(n, 4, device=DEV)
    for net in (nn.Sequential(nn.Linear(8, 8), nn.ReLU(), nn.Linear(8, 8), nn.ReLU(),
                              nn.LayerNorm(8), nn.Linear(8, 1)),
                nn.Sequential(nn.Linear(8, 40), nn.LayerNorm(40), nn.ReLU(), nn.Linear(40, 1)),
                nn.Sequential(nn.Linear(8, 100), nn.ReLU(), nn.Linear(100, 1))):
        net = net.to(DEV)

        class Scored(tg.MessagePassing):
            reducer = tg.online_softmax()

            def __init__(self):
                super().__init__()
                self.net = tg.nn.trace(net)

            def edge(self, src, dst, edge):
                return self.reducer(self.net(src.x, dst.x), src.x)

        k = Scored()
        with pytest.raises(RuntimeError, match="strict"):
            k(graph=graph, src={"x": x}, dst={"x": x})
        tg.config.strict = False
        out = k(graph=graph, src={"x": x}, dst={"x": x})
        tg.config.strict = True
        assert k.last_variant.backend == "torch-eager"
        dst = graph.destination_index()
        s = net(torch.cat([x[col], x[dst]], 1))[:, 0]
        rp_np = f64(rp).astype(np.int64)
        e_out, _ = ref.segment_softmax(rp_np, f64(s), f64(x)[f64(col).astype(np.int64)])
        assert rel_err(f64(out), e_out) <= RTOL


def _bench_net(f_in=8, hidden=16):
    return nn.Sequential(nn.Linear(3 + 2 * f_in, hidden), nn.LeakyReLU(0.2),
                         nn.Linear(hidden, 1)).to(DEV)


@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
def test_many_steps_per_block_and_index_dtypes(idx):
    """About 330k edges: every block of the fused backward walks several
    256-edge steps and the last one is partial; int32 and int64 CSR."""
    print(f"nn attention 330k edges idx={idx}", flush=True)
    torch.manual_seed(7)
    nodes, f_in = 20000, 8
    rp, col = random_graph(nodes, nodes, 18, 11, hub=2000)
    rp, col = rp.to(idx), col.to(idx)
    graph = tg.Graph.from_csr(rp, col, num_src=nodes)
    E = col.numel()
    assert E > 300000
    disp = torch.randn(E, 3, device=DEV, requires_grad=True)
    x = torch.randn(nodes, f_in, device=DEV, requires_grad=True)
    attn = _bench_net(f_in)
    dout = torch.randn(nodes, f_in, device=DEV)
    check(graph, GAT(attn), attn, [("edge", disp), ("src", x), ("dst", x)], x,
          dict(graph=graph, src={"x": x}, dst={"x": x}, edge={"displacement": disp}), dout)


def test_weight_gradients_bit_identical_across_runs():
    """Weight and bias gradients are block sums added in a fixed order."""
    torch.manual_seed(3)
    nodes = 5000
    rp, col = random_graph(nodes, nodes, 20, 5)
    graph = tg.Graph.from_csr(rp, col, num_src=nodes)
    disp = torch.randn(col.numel(), 3, device=DEV)
    x = torch.randn(nodes, 8, device=DEV)
    attn = _bench_net()
    kernel = GAT(attn)
    dout = torch.randn(nodes, 8, device=DEV)
    grads = []
    for _ in range(3):
        attn.zero_grad(set_to_none=True)
        kernel(graph=graph, src={"x": x}, dst={"x": x}, edge={"displacement": disp}).backward(dout)
        assert kernel.last_variant.backend == "hip"
        grads.append([p.grad.clone() for p in attn.parameters()])
    for other in grads[1:]:
        for a, b in zip(grads[0], other):
            assert torch.equal(a, b)


def test_graph_without_edges():
    """No edges: zero outputs and zero gradients everywhere."""
    nodes = 40
    rp = torch.zeros(nodes + 1, dtype=torch.int64, device=DEV)
    col = torch.zeros(0, dtype=torch.int64, device=DEV)
    graph = tg.Graph.from_csr(rp, col, num_src=nodes)
    disp = torch.randn(0, 3, device=DEV, requires_grad=True)
    x = torch.randn(nodes, 8, device=DEV, requires_grad=True)
    attn = _bench_net()
    kernel = GAT(attn)
    out = kernel(graph=graph, src={"x": x}, dst={"x": x}, edge={"displacement": disp})
    assert kernel.last_variant.backend == "hip"
    out.backward(torch.randn(nodes, 8, device=DEV))
    assert torch.count_nonzero(out) == 0
    assert torch.count_nonzero(x.grad) == 0
    for p in attn.parameters():
        assert p.grad is not None and torch.count_nonzero(p.grad) == 0

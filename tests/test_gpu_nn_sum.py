"""Edge networks on the HIP path: tg.sum() over a tg.nn.trace message (the
reference's edge-NN tile, compiler/edge_nn_tile.py, message_passing.py:
2134-2300) and nn-scored attention with the wider activation set and scalar
arithmetic (compiler/nn_capture.py:17-31): exp, log, sqrt, rsqrt, abs, sin,
cos, squares, powers and c / x among the functions, scalar maps after them
folded into the next Linear layer, LayerNorm between hidden layers and their
functions, hidden widths that leave padding columns in the kernels' 4-wide
blocks.

Checked against Torch float64 autograd of the same module on the gathered
fields (oracle/eager_torch.nn_message_sum / nn_attention, the reference's
eager semantics, pinned in tests/test_oracle.py): outputs and the gradients
of every field within 1e-5 relative (max-norm); weight and bias gradients,
which sum over every edge, within 3e-5.
"""

import copy

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

import tiga as tg
from oracle import eager_torch

from graphs import skewed_csr

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


@pytest.fixture(autouse=True)
def _strict():
    tg.config.strict = True
    yield
    tg.config.strict = False


def rel(a, e):
    a, e = a.detach().double().cpu(), e.detach().double().cpu()
    return float((a - e).abs().max() / e.abs().max().clamp_min(1e-30))


class Affine(nn.Module):
    """Scalar arithmetic straight after Linear layers (folded into them)."""

    def __init__(self, i, h, o):
        super().__init__()
        self.a, self.b = nn.Linear(i, h), nn.Linear(h, o)

    def forward(self, x):
        return self.b(F.softplus(2.0 - self.a(x) * 0.5, beta=2.0)) / 4.0 + 1.0


class ThreeLayer(nn.Module):
    """Linear a -> f -> Linear b -> g -> Linear c with the component-wise
    functions of `kind` and scalar arithmetic before and after them."""

    def __init__(self, i, kind, h1, h2, o):
        super().__init__()
        self.kind = kind
        self.a, self.b, self.c = nn.Linear(i, h1), nn.Linear(h1, h2), nn.Linear(h2, o)

    def forward(self, x):
        if self.kind == "exp-log":
            h = torch.exp(self.a(x) * 0.5)
            h = torch.log(self.b(h) * 0.1 + 3.0)
            return self.c(h * 2.0 - 1.0)
        if self.kind == "roots":
            h = torch.sqrt(self.a(x) * 0.3 + 2.0)
            h = (self.b(h) * 0.5 + 2.0).rsqrt()
            return self.c(1.0 - 2.0 * h)
        if self.kind == "trig":
            h = torch.sin(self.a(x))
            return self.c(-self.b(h).cos())
        if self.kind == "powers":
            h = self.a(x).abs()
            return self.c(2.0 / (self.b(h) * 0.5 + 3.0))
        h = self.a(x)
        h = h * h
        h = (self.b(h) * 0.1 + 2.0) ** 1.5
        return self.c(h / 3.0)


class Normed(nn.Module):
    """LayerNorm between hidden Linear layers and their functions (with and
    without its affine parameters, constants around it)."""

    def __init__(self, i, h1, h2, o):
        super().__init__()
        self.a, self.b, self.c = nn.Linear(i, h1), nn.Linear(h1, h2), nn.Linear(h2, o)
        self.na = nn.LayerNorm(h1)
        self.nb = nn.LayerNorm(h2, elementwise_affine=False, eps=1e-3)
        with torch.no_grad():
            self.na.weight.uniform_(0.5, 1.5)
            self.na.bias.uniform_(-0.5, 0.5)

    def forward(self, x):
        h = F.gelu(self.na(self.a(x) * 3.0) * 2.0 + 0.5)
        return self.c(torch.tanh(self.nb(self.b(h))) - 0.25)


class TwoFunctions(nn.Module):
    """Two functions in a row (an identity layer between them)."""

    def __init__(self, i, h, o):
        super().__init__()
        self.a, self.b = nn.Linear(i, h), nn.Linear(h, o)

    def forward(self, x):
        return self.b(torch.exp(torch.sin(self.a(x)) * 0.5))


def nets(i):
    return {
        # Identity layers: a function after the last Linear layer, LayerNorm
        # before the first, two functions in a row.
        "act-last": nn.Sequential(nn.Linear(i, 12), nn.ReLU(), nn.Linear(12, 5), nn.Sigmoid()),
        "norm-first": nn.Sequential(nn.LayerNorm(i), nn.Linear(i, 8), nn.Tanh(),
                                    nn.Linear(8, 3)),
        "two-functions": TwoFunctions(i, 10, 4),
        "layernorm-3": Normed(i, 12, 7, 3),
        # 64-wide score chains (the two-pass backward) with the second set of
        # functions; as edge-network sums these run eager (wider than 32).
        "wide-trig": ThreeLayer(i, "trig", 40, 48, 3),
        "wide-powers": ThreeLayer(i, "powers", 36, 60, 2),
        "layernorm-2": nn.Sequential(nn.Linear(i, 16), nn.LayerNorm(16), nn.ReLU(),
                                     nn.Linear(16, 4)),
        "layernorm-32": nn.Sequential(nn.Linear(i, 30), nn.LayerNorm(30), nn.SiLU(),
                                      nn.Linear(30, 20), nn.LayerNorm(20), nn.Sigmoid(),
                                      nn.Linear(20, 2)),
        "exp-log": ThreeLayer(i, "exp-log", 10, 9, 3),
        "roots": ThreeLayer(i, "roots", 12, 7, 2),
        "trig": ThreeLayer(i, "trig", 11, 6, 4),
        "powers": ThreeLayer(i, "powers", 10, 30, 2),
        "squares": ThreeLayer(i, "squares", 9, 20, 3),
        "relu-2": nn.Sequential(nn.Linear(i, 16), nn.ReLU(), nn.Linear(16, 8)),
        "mish-selu-3": nn.Sequential(nn.Linear(i, 24), nn.Mish(), nn.Linear(24, 12), nn.SELU(),
                                     nn.Linear(12, 5)),
        "hard-3": nn.Sequential(nn.Linear(i, 20), nn.Hardswish(), nn.Linear(20, 16),
                                nn.Hardsigmoid(), nn.Linear(16, 3)),
        "relu6-hardtanh": nn.Sequential(nn.Linear(i, 12), nn.ReLU6(), nn.Linear(12, 9),
                                        nn.Hardtanh(-0.5, 2.0), nn.Linear(9, 4)),
        "linear-1": nn.Linear(i, 6, bias=False),
        "affine-softplus": Affine(i, 10, 7),
    }


@pytest.mark.parametrize("name", sorted(n for n in nets(1) if not n.startswith("wide")))
@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
def test_edge_network_sum_against_float64_autograd(name, idx):
    print(f"edge network sum {name} {idx}", flush=True)
    N = 2000
    rp, col = skewed_csr(41, N, N, mean_deg=8, hubs=(1500, 600), empty_frac=0.1)
    rng = np.random.default_rng(9)
    xs = torch.tensor(rng.standard_normal((N, 3)), dtype=torch.float32, device=DEV)
    xd = torch.tensor(rng.standard_normal((N, 2)), dtype=torch.float32, device=DEV)
    xe = torch.tensor(rng.standard_normal(col.size), dtype=torch.float32, device=DEV)
    torch.manual_seed(3)
    net = nets(6)[name].to(DEV)
    graph = tg.Graph.from_csr(torch.tensor(rp, device=DEV, dtype=idx),
                              torch.tensor(col, device=DEV, dtype=idx), num_src=N)

    class Msg(tg.MessagePassing):
        reducer = tg.sum()

        def edge(self, src, dst, edge):
            return tg.nn.trace(net)(src.s, dst.d, edge.e)

    leaves = [t.clone().requires_grad_(True) for t in (xs, xd, xe)]
    k = Msg()
    out = k(graph=graph, src={"s": leaves[0]}, dst={"d": leaves[1]}, edge={"e": leaves[2]})
    assert k.last_variant.backend == "hip" and k.last_variant.pattern == "edge-network-sum"
    dout = torch.tensor(rng.standard_normal(tuple(out.shape)), dtype=torch.float32, device=DEV)
    params = list(net.parameters())
    got = torch.autograd.grad(out, leaves + params, dout)
    ref_net = copy.deepcopy(net).double().cpu()
    inputs = [("src", xs.double().cpu()), ("dst", xd.double().cpu()),
              ("edge", xe.double().cpu())]
    e_out, e_in, e_par = eager_torch.nn_message_sum(torch.tensor(rp), torch.tensor(col), inputs,
                                                    ref_net, dout.double().cpu())
    assert rel(out, e_out) <= 1e-5
    for g, w in zip(got[:3], e_in):
        assert rel(g, w) <= 1e-5
    for g, w in zip(got[3:], e_par):
        assert rel(g, w) <= 3e-5


@pytest.mark.parametrize("name", ["mish-selu-3", "hard-3", "relu6-hardtanh", "affine-softplus",
                                  "exp-log", "roots", "trig", "powers", "squares",
                                  "layernorm-3", "layernorm-2", "layernorm-32", "wide-trig",
                                  "wide-powers", "act-last", "norm-first", "two-functions"])
def test_nn_attention_wider_op_set_against_float64_autograd(name):
    print(f"nn attention {name}", flush=True)
    N = 2000
    rp, col = skewed_csr(43, N, N, mean_deg=8, hubs=(900,), empty_frac=0.1)
    rng = np.random.default_rng(11)
    xs = torch.tensor(rng.standard_normal((N, 4)), dtype=torch.float32, device=DEV)
    xe = torch.tensor(rng.standard_normal((col.size, 2)), dtype=torch.float32, device=DEV)
    value = torch.tensor(rng.standard_normal((N, 5)), dtype=torch.float32, device=DEV)
    torch.manual_seed(4)
    body = nets(6)[name]
    name_last, last = [(n, m) for n, m in body.named_modules() if isinstance(m, nn.Linear)][-1]
    # one-output score network: the same body with its last layer cut to 1
    net = copy.deepcopy(body)
    setattr(net, name_last, nn.Linear(last.in_features, 1))
    net = net.to(DEV)
    graph = tg.Graph.from_csr(torch.tensor(rp, device=DEV), torch.tensor(col, device=DEV),
                              num_src=N)

    class Attn(tg.MessagePassing):
        reducer = tg.online_softmax()

        def edge(self, src, dst, edge):
            return self.reducer(tg.nn.trace(net)(src.x, edge.e) / 2.0, src.v)

    xl, el, vl = (t.clone().requires_grad_(True) for t in (xs, xe, value))
    k = Attn()
    out = k(graph=graph, src={"x": xl, "v": vl}, dst={}, edge={"e": el})
    assert k.last_variant.backend == "hip" and k.last_variant.pattern == "nn-attention"
    dout = torch.tensor(rng.standard_normal((N, 5)), dtype=torch.float32, device=DEV)
    params = list(net.parameters())
    got = torch.autograd.grad(out, [xl, el, vl] + params, dout)
    ref_net = copy.deepcopy(net).double().cpu()
    e_out, e_in, e_v, e_par = eager_torch.nn_attention(
        torch.tensor(rp), torch.tensor(col), [("src", xs.double().cpu()), ("edge", xe.double().cpu())],
        ref_net, value.double().cpu(), dout.double().cpu(), out_scale=0.5)
    assert rel(out, e_out) <= 1e-5
    assert rel(got[0], e_in[0]) <= 1e-5 and rel(got[1], e_in[1]) <= 1e-5
    assert rel(got[2], e_v) <= 1e-5
    # Parameters in (weight, bias) pairs; a bias in its layer's weight-gradient
    # scale (the last bias's exact gradient is 0: it shifts a whole row).
    for (gw, gb), (ew, eb) in zip(zip(got[3::2], got[4::2]), zip(e_par[0::2], e_par[1::2])):
        scale = float(ew.abs().max())
        assert float((gw.double().cpu() - ew).abs().max()) <= 3e-5 * scale
        assert float((gb.double().cpu() - eb).abs().max()) <= 3e-5 * max(scale, float(eb.abs().max()))


def test_edge_network_sum_edgeless_graph_and_warm_calls():
    print("edge network sum, edgeless graph", flush=True)
    net = nn.Sequential(nn.Linear(3, 8), nn.Tanh(), nn.Linear(8, 2)).to(DEV)

    class Msg(tg.MessagePassing):
        reducer = tg.sum()

        def edge(self, src, dst, edge):
            return tg.nn.trace(net)(src.s)

    graph = tg.Graph.from_csr(torch.zeros(5, dtype=torch.int64, device=DEV),
                              torch.zeros(0, dtype=torch.int64, device=DEV), num_src=3)
    s = torch.randn(3, 3, device=DEV, requires_grad=True)
    k = Msg()
    out = k(graph=graph, src={"s": s}, dst={})
    assert out.shape == (4, 2) and not out.any()
    out.sum().backward()
    assert not s.grad.any()

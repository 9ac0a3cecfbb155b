"""Capture of edge networks (tg.nn.trace) into the kernels' layer chain, on
the CPU: which modules become a chain of folded Linear (and LayerNorm)
layers, and that the folded weights and the gradient unfolding reproduce the
module itself.

The reference captures the same op set (compiler/nn_capture.py:17-31,
281-380: Linear, the component-wise functions, scalar arithmetic).  The
checks run the module in float64 and the captured chain in float64 (each
activation code evaluated by its Torch function) on random inputs; the
gradients of the module's own weights and biases come from autograd through
the module and, for the chain, from autograd at the folded weights mapped
back by the same routine the HIP path uses (_ops._unfolded_grads).
"""

import operator

import pytest
import torch
import torch.nn.functional as F
from torch import nn

from tiga import _ops
from tiga.nn import _extract_chain

# Each activation code evaluated in float64 by Torch (the kernels' functions
# are compared against these through the GPU tests).
ACT = {
    "identity": lambda z, p, q: z,
    "relu": lambda z, p, q: torch.relu(z),
    "leaky_relu": lambda z, p, q: F.leaky_relu(z, p),
    "tanh": lambda z, p, q: torch.tanh(z),
    "sigmoid": lambda z, p, q: torch.sigmoid(z),
    "silu": lambda z, p, q: F.silu(z),
    "gelu": lambda z, p, q: F.gelu(z),
    "elu": lambda z, p, q: F.elu(z, p),
    "hardtanh": lambda z, p, q: torch.clamp(z, p, q),
    "softplus": lambda z, p, q: F.softplus(z, p, q),
    "exp": lambda z, p, q: torch.exp(z),
    "log": lambda z, p, q: torch.log(z),
    "sqrt": lambda z, p, q: torch.sqrt(z),
    "rsqrt": lambda z, p, q: torch.rsqrt(z),
    "abs": lambda z, p, q: torch.abs(z),
    "sin": lambda z, p, q: torch.sin(z),
    "cos": lambda z, p, q: torch.cos(z),
    "square": lambda z, p, q: z * z,
    "reciprocal": lambda z, p, q: p / z,
    "pow": lambda z, p, q: torch.pow(z, p),
}


class ExpLog(nn.Module):
    def __init__(self):
        super().__init__()
        self.a, self.b, self.c = nn.Linear(5, 10), nn.Linear(10, 9), nn.Linear(9, 3)

    def forward(self, x):
        h = torch.exp(self.a(x) * 0.5)
        h = torch.log(self.b(h) * 0.1 + 3.0)
        return self.c(h * 2.0 - 1.0)


class Roots(nn.Module):
    def __init__(self):
        super().__init__()
        self.a, self.b, self.c = nn.Linear(5, 12), nn.Linear(12, 7), nn.Linear(7, 2)

    def forward(self, x):
        h = torch.sqrt(self.a(x) * 0.2 + 2.0)
        h = (self.b(h) * 0.1 + 1.5).rsqrt()
        return self.c(0.5 - h)


class Trig(nn.Module):
    def __init__(self):
        super().__init__()
        self.a, self.b, self.c = nn.Linear(5, 11), nn.Linear(11, 6), nn.Linear(6, 4)

    def forward(self, x):
        h = torch.sin(self.a(x))
        h = self.b(h).cos()
        return self.c(-h)


class Powers(nn.Module):
    def __init__(self):
        super().__init__()
        self.a, self.b, self.c = nn.Linear(5, 10), nn.Linear(10, 10), nn.Linear(10, 2)

    def forward(self, x):
        h = self.a(x).abs()
        h = 2.0 / (self.b(h) * 0.1 + 3.0)
        return self.c(h)


class Squares(nn.Module):
    def __init__(self):
        super().__init__()
        self.a, self.b, self.c = nn.Linear(5, 9), nn.Linear(9, 12), nn.Linear(12, 3)

    def forward(self, x):
        h = self.a(x)
        h = h * h
        h = (self.b(h) * 0.1 + 2.0) ** 1.5
        return self.c(h / 3.0)


class Square2(nn.Module):
    def __init__(self):
        super().__init__()
        self.a, self.b = nn.Linear(5, 8), nn.Linear(8, 1)

    def forward(self, x):
        return self.b(torch.square(self.a(x)) + 1.0) * 2.0


class Normed(nn.Module):
    """LayerNorm after hidden Linear layers, with and without its affine
    parameters, constants between it and the function."""

    def __init__(self):
        super().__init__()
        self.a, self.b, self.c = nn.Linear(5, 12), nn.Linear(12, 7), nn.Linear(7, 3)
        self.na = nn.LayerNorm(12)
        self.nb = nn.LayerNorm(7, elementwise_affine=False, eps=1e-3)
        with torch.no_grad():
            self.na.weight.uniform_(0.5, 1.5)
            self.na.bias.uniform_(-0.5, 0.5)

    def forward(self, x):
        h = F.gelu(self.na(self.a(x) * 3.0) * 2.0 + 0.5)
        h = torch.tanh(self.nb(self.b(h)))
        return self.c(h)


class TwoFunctions(nn.Module):
    def __init__(self):
        super().__init__()
        self.a, self.b = nn.Linear(5, 4), nn.Linear(4, 1)

    def forward(self, x):
        return self.b(torch.exp(torch.sin(self.a(x))))


class ShiftAtEnd(nn.Module):
    def __init__(self):
        super().__init__()
        self.a = nn.Linear(5, 4)

    def forward(self, x):
        return torch.exp(self.a(x)) + 1.0


class Rounded(nn.Module):
    def __init__(self):
        super().__init__()
        self.a, self.b = nn.Linear(5, 4), nn.Linear(4, 1)

    def forward(self, x):
        return self.b(torch.div(self.a(x), 2.0, rounding_mode="floor"))


class Before(nn.Module):
    def __init__(self):
        super().__init__()
        self.a = nn.Linear(5, 1)

    def forward(self, x):
        return self.a(x * 2.0)


NETS = {
    "exp-log": (ExpLog, [("exp", 0.0), ("log", 0.0), ("identity", 0.0)]),
    "roots": (Roots, [("sqrt", 0.0), ("rsqrt", 0.0), ("identity", 0.0)]),
    "trig": (Trig, [("sin", 0.0), ("cos", 0.0), ("identity", 0.0)]),
    "powers": (Powers, [("abs", 0.0), ("reciprocal", 2.0), ("identity", 0.0)]),
    "squares": (Squares, [("square", 0.0), ("pow", 1.5), ("identity", 0.0)]),
    "square-2": (Square2, [("square", 0.0), ("identity", 0.0)]),
    "layernorm": (Normed, [("gelu", 0.0), ("tanh", 0.0), ("identity", 0.0)]),
    "layernorm-sequential": (lambda: nn.Sequential(nn.Linear(5, 10), nn.LayerNorm(10),
                                                   nn.ReLU(), nn.Linear(10, 1)),
                             [("relu", 0.0), ("identity", 0.0)]),
    # Identity layers: two functions in a row, arithmetic and a function after
    # the last Linear layer, arithmetic before the first, LayerNorm after a
    # function and before the first Linear layer.
    "two-functions": (lambda: TwoFunctions(), [("sin", 0.0), ("exp", 0.0), ("identity", 0.0)]),
    "shift-at-end": (lambda: ShiftAtEnd(), [("exp", 0.0), ("identity", 0.0)]),
    "before": (lambda: Before(), [("identity", 0.0)]),
    "norm-after-act": (lambda: nn.Sequential(nn.Linear(5, 6), nn.ReLU(), nn.LayerNorm(6),
                                             nn.Linear(6, 1)),
                       [("relu", 0.0), ("identity", 0.0), ("identity", 0.0)]),
    "norm-first": (lambda: nn.Sequential(nn.LayerNorm(5), nn.Linear(5, 4), nn.Sigmoid()),
                   [("identity", 0.0), ("sigmoid", 0.0), ("identity", 0.0)]),
    "norm-last": (lambda: nn.Sequential(nn.Linear(5, 4), nn.ReLU(), nn.Linear(4, 2),
                                        nn.LayerNorm(2)),
                  [("relu", 0.0), ("identity", 0.0), ("identity", 0.0)]),
    "sequential": (lambda: nn.Sequential(nn.Linear(5, 8), nn.Softplus(2.0), nn.Linear(8, 8),
                                         nn.ELU(0.5), nn.Linear(8, 1)),
                   [("softplus", 2.0), ("elu", 0.5), ("identity", 0.0)]),
}


def run_chain(chain, x, weights):
    """The captured chain in float64 with the folded weights `weights`
    ([(W', b' or None, gamma' or None, beta' or None)] per layer)."""
    a = x
    for layer, (w, b, g, beta) in zip(chain, weights):
        z = a @ w.t()
        if b is not None:
            z = z + b
        if layer.norm is not None:
            z = F.layer_norm(z, (z.shape[1],), g, beta, layer.norm.eps)
        a = ACT[layer.act](z, layer.param, layer.param2)
    return a


def folded_weights(chain, params):
    out = []
    for i, layer in enumerate(chain):
        w, b = _ops._folded(layer, params[4 * i], params[4 * i + 1])
        g = beta = None
        if layer.norm is not None:
            g, beta = _ops._folded_norm(layer, params[4 * i + 2], params[4 * i + 3])
        out.append((w, b, g, beta))
    return out


@pytest.mark.parametrize("name", sorted(NETS))
def test_capture_codes_and_folded_chain_match_the_module(name):
    make, codes = NETS[name]
    torch.manual_seed(7)
    net = make().double()
    chain = _extract_chain(net)
    assert [(l.act, l.param) for l in chain] == codes
    x = torch.randn(64, 5, dtype=torch.float64)
    params = _ops._layer_params(chain)
    folded = folded_weights(chain, params)
    expect = net(x)
    got = run_chain(chain, x, folded)
    assert torch.isfinite(expect).all()
    torch.testing.assert_close(got, expect, rtol=1e-12, atol=1e-12)

    # Gradients of the module's own parameters: through the module, and at
    # the folded weights then mapped back as the HIP path does.  The kernels
    # sum a bias gradient for every layer, also where the module has no bias
    # (it unfolds into the weight gradient through in_shift): the chain here
    # gets a zero bias in its place.
    dout = torch.randn_like(expect)
    present = [p is not None for p in params]
    # Identity layers' weights are fixed (no gradient; not module parameters).
    trained = [p is not None and p.requires_grad for p in params]
    grads = torch.autograd.grad(net(x), [p for p, t in zip(params, trained) if t], dout)
    grads = iter(grads)
    expect_grads = [next(grads) if t else None for t in trained]
    leaves = []
    for layer, (w, b, g, beta) in zip(chain, folded):
        b = torch.zeros(w.shape[0], dtype=torch.float64) if b is None else b
        if layer.norm is not None:
            g = torch.ones(w.shape[0], dtype=torch.float64) if g is None else g
            beta = torch.zeros(w.shape[0], dtype=torch.float64) if beta is None else beta
        leaves.append(tuple(None if t is None else t.clone().requires_grad_(True)
                            for t in (w, b, g, beta)))
    flat = [t for grp in leaves for t in grp if t is not None]
    dflat = iter(torch.autograd.grad(run_chain(chain, x, leaves), flat, dout))
    blocks = []
    for grp in leaves:
        blocks.append([None if t is None else next(dflat) for t in grp])
    W = 16
    dweights = torch.zeros(len(chain), _ops._block_floats(chain, W), dtype=torch.float64)
    for l, (layer, (dw, db, dg, dbeta)) in enumerate(zip(chain, blocks)):
        o, i = dw.shape
        dweights[l, :W * W].view(W, W)[:o, :i] = dw
        dweights[l, W * W:W * W + o] = db
        if dg is not None:
            dweights[l, W * W + W:W * W + W + o] = dg
            dweights[l, W * W + 2 * W:W * W + 2 * W + o] = dbeta
    got_grads = _ops._layer_grads(chain, dweights, W, present, trained, 0, len(chain))
    for k, (g, e) in enumerate(zip(got_grads, expect_grads)):
        assert (g is None) == (e is None), k
        if e is not None:
            torch.testing.assert_close(g, e, rtol=1e-10, atol=1e-12)


def test_affine_maps_fold_into_the_right_layer():
    """x * c / c + b directly after a Linear folds into its output map; after
    a LayerNorm into its gamma and beta; after an activation into the next
    Linear's input map."""
    chain = _extract_chain(ExpLog())
    assert (chain[0].scale, chain[0].shift) == (0.5, 0.0)
    assert (chain[1].scale, chain[1].shift) == (0.1, 3.0)
    assert (chain[2].in_scale, chain[2].in_shift) == (2.0, -1.0)
    chain = _extract_chain(Roots())
    assert (chain[2].in_scale, chain[2].in_shift) == (-1.0, 0.5)
    chain = _extract_chain(Square2())
    assert (chain[1].in_scale, chain[1].in_shift, chain[1].scale) == (1.0, 1.0, 2.0)
    chain = _extract_chain(Normed())
    assert (chain[0].scale, chain[0].norm_scale, chain[0].norm_shift) == (3.0, 2.0, 0.5)
    assert chain[1].norm is not None and chain[1].norm.eps == 1e-3


@pytest.mark.parametrize("net", [Rounded,
                                 lambda: nn.Sequential(nn.Linear(4, 4), nn.ReLU(),
                                                       nn.Linear(4, 4), nn.ReLU(),
                                                       nn.Linear(4, 2), nn.LayerNorm(2)),
                                 lambda: nn.Sequential(*[m for _ in range(4) for m in
                                                         (nn.Linear(4, 4), nn.ReLU())]),
                                 lambda: nn.Sequential(nn.Linear(4, 4), nn.ReLU(),
                                                       nn.Tanh(), nn.Sigmoid(),
                                                       nn.Linear(4, 1))])
def test_uncovered_networks_are_refused(net):
    """A rounding division, or chains that need more than three layers with
    the identity layers counted (a LayerNorm after the last Linear layer,
    four Linear layers, three functions in a row): not captured (the eager
    evaluator runs them)."""
    with pytest.raises(NotImplementedError):
        _extract_chain(net())


def test_operator_forms_are_the_same_codes():
    """x ** p, torch.pow, x.pow and c / x forms reach the same codes."""
    for fn, code in [(lambda h: h ** 2.5, ("pow", 2.5)), (lambda h: torch.pow(h, 3), ("pow", 3.0)),
                     (lambda h: h.pow(0.5), ("pow", 0.5)), (lambda h: 3.0 / h, ("reciprocal", 3.0)),
                     (lambda h: torch.div(1.0, h), ("reciprocal", 1.0)),
                     (lambda h: h.exp(), ("exp", 0.0)), (lambda h: torch.abs(h), ("abs", 0.0)),
                     (lambda h: operator.mul(h, h), ("square", 0.0))]:
        class Net(nn.Module):
            def __init__(self):
                super().__init__()
                self.a, self.b = nn.Linear(3, 3), nn.Linear(3, 1)

            def forward(self, x):
                return self.b(fn(self.a(x)))

        chain = _extract_chain(Net())
        assert (chain[0].act, chain[0].param) == code


def test_trace_accepts_the_reference_launch_geometry():
    """tg.nn.trace(module, block_e=..., num_warps=...) as in the reference:
    powers of two in [16, 1024] and [1, 16], else ValueError."""
    import tiga as tg

    net = nn.Linear(3, 1)
    assert tg.nn.trace(net, block_e=64, num_warps=4).module is net
    for kwargs in ({"block_e": 48}, {"block_e": 8}, {"num_warps": 32}, {"num_warps": 3}):
        with pytest.raises(ValueError):
            tg.nn.trace(net, **kwargs)

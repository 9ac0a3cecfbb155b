"""``tg.nn.trace``: torch.nn score networks inside ``edge()``.

Mirrors the reference (python/tiga/compiler/nn_capture.py:1-33,
python/tiga/nn/__init__.py): ``trace(module)`` wraps a module so one
``edge()`` source drives two paths:

* called with Torch tensors (eager evaluation) the inputs are concatenated
  along the feature dimension and passed to the module unchanged;
* called with capture proxies the call is recorded as an ``nn`` node over the
  field expressions, which the nn-attention recognizer lowers to the HIP edge
  MLP kernels when the module is a chain the kernels cover.

Covered chains: ``nn.Linear`` layers (bias optional), each optionally
followed by scalar-constant arithmetic (``x * c``, ``x / c``, ``x + c``,
``x - c``, ``c - x``, ``-x``: folded into that layer's weights and bias) and
by one component-wise function (relu, leaky_relu, tanh, sigmoid, silu,
exact gelu, elu, hardtanh / relu6 / clamp, softplus, selu, mish,
hardsigmoid, hardswish, exp, log, sqrt, rsqrt, abs, sin, cos, square,
``c / x``, ``x ** p``; module, functional or Tensor-method form;
``nn.Identity`` is skipped), whose output may again be scaled and shifted by
constants (folded into the next Linear layer's input), and feature-wise
``nn.LayerNorm`` (constants between it and the function folded into its
weight and bias).  A function or LayerNorm with no Linear layer of its own
in front -- two in a row, one before the first Linear layer or after the
last -- gets a fixed identity Linear layer, and the kernels take at most
three layers in all.  A score network ends with one output and every width
is at most 64 (32 with a LayerNorm); an edge-network message summed per row
(``tg.sum()``) may be of any width, its other widths at most 32.  Anything
else runs on the eager evaluator.
"""

from __future__ import annotations

import weakref
from dataclasses import dataclass

import torch
from torch import nn

# Score chains by module object: tracing a module with torch.fx costs
# milliseconds, and edge() usually wraps the same module on every call.
_CHAINS: "weakref.WeakKeyDictionary[nn.Module, object]" = weakref.WeakKeyDictionary()

_ACT = {"identity": 0, "relu": 1, "leaky_relu": 2, "tanh": 3, "sigmoid": 4, "silu": 5,
        "gelu": 6, "elu": 7, "hardtanh": 8, "softplus": 9, "selu": 10, "mish": 11,
        "hardsigmoid": 12, "hardswish": 13, "exp": 14, "log": 15, "sqrt": 16, "rsqrt": 17,
        "abs": 18, "sin": 19, "cos": 20, "square": 21, "reciprocal": 22, "pow": 23}

# Component-wise Torch functions without parameters that have a code of
# the same name.
_UNARY = ("exp", "log", "sqrt", "rsqrt", "abs", "sin", "cos", "square")


@dataclass(frozen=True)
class ScoreLayer:
    """One Linear layer of a chain: the scalar affine map on its input
    (in_scale * a + in_shift, from arithmetic after the previous
    activation), the one folded after it, z = scale * (W a' + b) + shift,
    an optional LayerNorm over z followed by the scalar map norm_scale * y +
    norm_shift, and the activation that follows."""

    linear: nn.Linear
    act: str = "identity"
    param: float = 0.0
    param2: float = 0.0
    scale: float = 1.0
    shift: float = 0.0
    in_scale: float = 1.0
    in_shift: float = 0.0
    norm: nn.LayerNorm | None = None
    norm_scale: float = 1.0
    norm_shift: float = 0.0


class TracedModule(nn.Module):
    """A module usable both on tensors and on edge() capture proxies."""

    def __init__(self, module: nn.Module):
        super().__init__()
        self.module = module

    def forward(self, *inputs):
        from .capture import Sym

        if any(isinstance(x, Sym) for x in inputs):
            return Sym("nn", (self, tuple(inputs)))
        tensors = [x if x.ndim > 1 else x.unsqueeze(-1) for x in inputs]
        return self.module(torch.cat(tensors, dim=-1))

    def __call__(self, *inputs):
        from .capture import Sym

        # Capture proxies bypass nn.Module hooks (they are not tensors).
        if any(isinstance(x, Sym) for x in inputs):
            return Sym("nn", (self, tuple(inputs)))
        return super().__call__(*inputs)

    def chain(self, vector: bool = False) -> tuple[ScoreLayer, ...] | None:
        """The module as a chain the HIP kernels cover, else None: a score
        chain (one output) or, with vector=True, an edge-network message of
        any output width.  Computed once per module object (a module whose
        layers are replaced afterwards must be wrapped by a new object)."""
        got = _CHAINS.get(self.module)
        if got is None:
            try:
                got = _extract_chain(self.module)
            except NotImplementedError:
                got = ()
            _CHAINS[self.module] = got
        if not got:
            return None
        if not vector and got[-1].linear.out_features != 1:
            return None
        return got


def _check_geometry(name: str, value, low: int, high: int) -> None:
    if value is not None and (value < low or value > high or value & (value - 1)):
        raise ValueError(f"{name} must be a power of two in [{low}, {high}], got {value}")


def trace(module: nn.Module, *, block_e: int | None = None,
          num_warps: int | None = None) -> TracedModule:
    """Wrap ``module`` for use inside ``MessagePassing.edge`` (reference
    compiler/nn_capture.py:418-428).  ``block_e`` and ``num_warps`` are the
    reference's launch geometry for its tiles (edges per program, warps);
    they are checked as the reference checks them and otherwise unused: the
    HIP kernels here run one edge per lane with their own geometry, and
    geometry never changes numerics."""
    _check_geometry("block_e", block_e, 16, 1024)
    _check_geometry("num_warps", num_warps, 1, 16)
    if isinstance(module, TracedModule):
        return module
    if not isinstance(module, nn.Module):
        raise TypeError("tg.nn.trace expects a torch.nn.Module")
    return TracedModule(module)


def _module_activation(m: nn.Module):
    simple = {nn.ReLU: "relu", nn.Tanh: "tanh", nn.Sigmoid: "sigmoid", nn.SiLU: "silu",
              nn.SELU: "selu", nn.Mish: "mish", nn.Hardsigmoid: "hardsigmoid",
              nn.Hardswish: "hardswish"}
    for cls, name in simple.items():
        if type(m) is cls:
            return name, 0.0, 0.0
    if type(m) is nn.LeakyReLU:
        return "leaky_relu", float(m.negative_slope), 0.0
    if type(m) is nn.ELU:
        return "elu", float(m.alpha), 0.0
    if type(m) is nn.GELU and m.approximate == "none":
        return "gelu", 0.0, 0.0
    if type(m) is nn.ReLU6:
        return "hardtanh", 0.0, 6.0
    if type(m) is nn.Hardtanh:
        return "hardtanh", float(m.min_val), float(m.max_val)
    if type(m) is nn.Softplus:
        return "softplus", float(m.beta), float(m.threshold)
    return None


def _arg(args, kwargs, index, name, default):
    if len(args) > index:
        return args[index]
    return kwargs.get(name, default)


def _number(v) -> bool:
    import numbers

    return isinstance(v, numbers.Number) and not isinstance(v, bool)


def _function_activation(target, args, kwargs, previous):
    import operator

    from torch.nn import functional as F

    # c / x (x / c is a scalar affine map, taken earlier).
    if target in (operator.truediv, torch.div, torch.true_divide) and len(args) == 2 and \
            args[1] is previous and _number(args[0]) and not kwargs:
        return "reciprocal", float(args[0]), 0.0
    if not args or args[0] is not previous:
        return None
    unary = {getattr(torch, name): name for name in _UNARY}
    if target in unary and len(args) == 1 and not kwargs:
        return unary[target], 0.0, 0.0
    if target in (operator.mul, torch.mul) and tuple(args) == (previous, previous) and \
            not kwargs:
        return "square", 0.0, 0.0
    if target in (operator.pow, torch.pow) and len(args) == 2 and _number(args[1]) and \
            not kwargs:
        return "pow", float(args[1]), 0.0
    simple = {torch.relu: "relu", F.relu: "relu", torch.tanh: "tanh", F.tanh: "tanh",
              torch.sigmoid: "sigmoid", F.sigmoid: "sigmoid", F.silu: "silu", F.selu: "selu",
              torch.selu: "selu", F.mish: "mish", F.hardsigmoid: "hardsigmoid",
              F.hardswish: "hardswish", F.relu6: "relu6"}
    if target in simple and len(args) == 1 and set(kwargs) <= {"inplace"}:
        name = simple[target]
        return ("hardtanh", 0.0, 6.0) if name == "relu6" else (name, 0.0, 0.0)
    if target is F.leaky_relu:
        return "leaky_relu", float(_arg(args, kwargs, 1, "negative_slope", 0.01)), 0.0
    if target is F.elu:
        return "elu", float(_arg(args, kwargs, 1, "alpha", 1.0)), 0.0
    if target is F.gelu and kwargs.get("approximate", "none") == "none":
        return "gelu", 0.0, 0.0
    if target is F.hardtanh:
        return ("hardtanh", float(_arg(args, kwargs, 1, "min_val", -1.0)),
                float(_arg(args, kwargs, 2, "max_val", 1.0)))
    if target is F.softplus:
        return ("softplus", float(_arg(args, kwargs, 1, "beta", 1.0)),
                float(_arg(args, kwargs, 2, "threshold", 20.0)))
    if target in (torch.clamp, torch.clip):
        lo = _arg(args, kwargs, 1, "min", None)
        hi = _arg(args, kwargs, 2, "max", None)
        if lo is None and hi is None:
            return None
        return ("hardtanh", -float("inf") if lo is None else float(lo),
                float("inf") if hi is None else float(hi))
    return None


def _scalar_affine(t, a, kwargs, previous):
    """(scale, shift) of scalar-constant arithmetic `t(*a, **kwargs)` applied
    to `previous`: y = scale * x + shift; None if it is not one."""
    import operator

    if not a or kwargs:
        return None
    number = _number
    if t in (operator.neg, torch.neg) and len(a) == 1 and a[0] is previous:
        return -1.0, 0.0
    if len(a) != 2:
        return None
    if t in (operator.mul, torch.mul):
        if a[0] is previous and number(a[1]):
            return float(a[1]), 0.0
        if a[1] is previous and number(a[0]):
            return float(a[0]), 0.0
    if t in (operator.truediv, torch.div) and a[0] is previous and number(a[1]) and a[1] != 0:
        return 1.0 / float(a[1]), 0.0
    if t in (operator.add, torch.add):
        if a[0] is previous and number(a[1]):
            return 1.0, float(a[1])
        if a[1] is previous and number(a[0]):
            return 1.0, float(a[0])
    if t in (operator.sub, torch.sub):
        if a[0] is previous and number(a[1]):
            return 1.0, -float(a[1])
        if a[1] is previous and number(a[0]):
            return -1.0, float(a[0])
    return None


def _identity_linear(n: int, like: torch.Tensor) -> nn.Linear:
    """A fixed n x n identity Linear layer (no bias, no gradient) on like's
    device and dtype: inserted where the chain has a function or LayerNorm
    with no Linear layer of its own in front (or after the last one)."""
    layer = nn.Linear(n, n, bias=False, device=like.device, dtype=like.dtype)
    with torch.no_grad():
        layer.weight.copy_(torch.eye(n, device=like.device, dtype=like.dtype))
    layer.weight.requires_grad_(False)
    return layer


def _chain_ops(module: nn.Module) -> list[tuple[str, object]]:
    """The module's fx graph as a list of ("linear", nn.Linear), ("norm",
    nn.LayerNorm), ("act", (name, param, param2)) and ("affine", (c, b))
    steps of a single-input chain."""
    import torch.fx

    gm = torch.fx.symbolic_trace(module)
    ops: list[tuple[str, object]] = []
    previous = None
    for node in gm.graph.nodes:
        if node.op == "placeholder":
            if previous is not None:
                raise NotImplementedError("networks take one input")
            previous = node
            continue
        if node.op == "output":
            if node.args[0] is not previous:
                raise NotImplementedError("network output is not the chain's end")
            break
        if node.op == "call_module":
            target = gm.get_submodule(node.target)
            if node.args != (previous,):
                raise NotImplementedError("networks must be single-input chains")
            if isinstance(target, nn.Identity):
                pass
            elif isinstance(target, nn.Linear):
                ops.append(("linear", target))
            elif isinstance(target, nn.LayerNorm):
                if len(target.normalized_shape) != 1:
                    raise NotImplementedError("feature-wise LayerNorm only")
                ops.append(("norm", target))
            else:
                act = _module_activation(target)
                if act is None:
                    raise NotImplementedError(f"unsupported module {type(target).__name__}")
                ops.append(("act", act))
        elif node.op in ("call_function", "call_method"):
            target = node.target
            if node.op == "call_method":
                # x.exp(), x.mul(c), x.pow(p), ...: the Torch function of the
                # same name on the same arguments.
                target = getattr(torch, target, None)
                if target is None:
                    raise NotImplementedError(f"unsupported method {node.target}")
            affine = _scalar_affine(target, node.args, node.kwargs, previous)
            if affine is not None:
                ops.append(("affine", affine))
            else:
                act = _function_activation(target, node.args, node.kwargs, previous)
                if act is None:
                    raise NotImplementedError(f"unsupported function {node.target}")
                ops.append(("act", act))
        else:
            raise NotImplementedError(f"unsupported network node {node.op}")
        previous = node
    return ops


def _extract_chain(module: nn.Module) -> tuple[ScoreLayer, ...]:
    """The kernels' chain of layers, each Linear [LayerNorm] [function], for
    a single-input network of Linear layers, component-wise functions,
    feature-wise LayerNorms and scalar arithmetic (via torch.fx; reference
    nn_capture.py:281-380 translates the same graphs).  A scalar affine map
    directly after a Linear layer folds into that layer's output, one after
    a LayerNorm into its gamma and beta, one after a function (or before the
    first Linear layer) into the next Linear layer's input.  A function or
    LayerNorm with no Linear layer of its own in front (two in a row, one
    before the first Linear layer or after the last) gets a fixed identity
    Linear layer; at most three layers in all."""
    if isinstance(module, nn.Linear):
        # A bare Linear traced as the root shows its functional body.
        if max(module.in_features, module.out_features) > 64:
            raise NotImplementedError("network widths above 64")
        return (ScoreLayer(module),)
    ops = _chain_ops(module)
    linears = [m for kind, m in ops if kind == "linear"]
    if not linears:
        raise NotImplementedError("networks have at least one Linear layer")
    like = linears[0].weight
    width = linears[0].in_features      # features flowing between the steps
    layers: list[dict] = []
    pending = (1.0, 0.0)   # affine map for the next layer's input

    def add_layer(linear):
        nonlocal pending
        layers.append({"linear": linear, "act": None, "param": 0.0, "param2": 0.0,
                       "scale": 1.0, "shift": 0.0, "in_scale": pending[0],
                       "in_shift": pending[1], "norm": None, "norm_scale": 1.0,
                       "norm_shift": 0.0})
        pending = (1.0, 0.0)

    for kind, op in ops:
        if kind == "linear":
            if op.in_features != width:
                raise NotImplementedError("network widths do not chain")
            add_layer(op)
            width = op.out_features
        elif kind == "affine":
            c, b = op
            last = layers[-1] if layers else None
            if last is not None and last["act"] is None and last["norm"] is not None:
                last["norm_scale"] *= c
                last["norm_shift"] = c * last["norm_shift"] + b
            elif last is not None and last["act"] is None:
                last["scale"] *= c
                last["shift"] = c * last["shift"] + b
            else:
                pending = (c * pending[0], c * pending[1] + b)
        elif kind == "norm":
            if tuple(op.normalized_shape) != (width,):
                raise NotImplementedError("LayerNorm over other than the stream's features")
            if not layers or layers[-1]["act"] is not None or layers[-1]["norm"] is not None \
                    or pending != (1.0, 0.0):
                add_layer(_identity_linear(width, like))
            layers[-1]["norm"] = op
        else:   # a component-wise function
            if not layers or layers[-1]["act"] is not None or pending != (1.0, 0.0):
                add_layer(_identity_linear(width, like))
            layers[-1]["act"], layers[-1]["param"], layers[-1]["param2"] = op
    if layers[-1]["act"] is not None or layers[-1]["norm"] is not None or \
            pending != (1.0, 0.0):
        # The chain must end in a Linear layer without LayerNorm or function.
        add_layer(_identity_linear(width, like))
    if len(layers) > 3:
        raise NotImplementedError("networks have one to three layers (identity layers counted)")
    widths = [l["linear"].in_features for l in layers] + \
        [l["linear"].out_features for l in layers[:-1]]
    if max(widths) > 64:
        raise NotImplementedError("network widths above 64")
    return tuple(ScoreLayer(l["linear"], l["act"] or "identity", l["param"], l["param2"],
                            l["scale"], l["shift"], l["in_scale"], l["in_shift"], l["norm"],
                            l["norm_scale"], l["norm_shift"])
                 for l in layers)


__all__ = ["ScoreLayer", "TracedModule", "trace"]

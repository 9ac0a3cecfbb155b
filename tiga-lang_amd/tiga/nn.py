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
constants (folded into the next Linear layer's input), and optionally by a
feature-wise ``nn.LayerNorm`` between a hidden Linear layer and its function
(constants between the two folded into its weight and bias), at most three
Linear layers.  A score network ends in a Linear layer with one output and
every width is at most 64 (32 with a LayerNorm); an edge-network message
summed per row (``tg.sum()``) ends in a Linear layer of any width and its
other widths are at most 32.  Anything else (two functions in a row, a
LayerNorm after the last Linear layer, ...) runs on the eager evaluator.
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


def trace(module: nn.Module) -> TracedModule:
    """Wrap ``module`` for use inside ``MessagePassing.edge``."""
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


def _extract_chain(module: nn.Module) -> tuple[ScoreLayer, ...]:
    """Linear [affine]* [LayerNorm [affine]*] [act [affine]*] ... Linear
    [affine]*, via torch.fx (reference nn_capture.py:281-380 translates the
    same graphs).  A scalar affine map directly after a Linear layer folds
    into that layer's output, one after a LayerNorm into its gamma and beta,
    one after an activation into the next Linear layer's input."""
    import torch.fx

    if isinstance(module, nn.Linear):
        # A bare Linear traced as the root shows its functional body.
        if max(module.in_features, module.out_features) > 64:
            raise NotImplementedError("network widths above 64")
        return (ScoreLayer(module),)
    gm = torch.fx.symbolic_trace(module)
    layers: list[dict] = []
    previous = None
    pending = (1.0, 0.0)   # affine map after the last activation, for the next Linear
    for node in gm.graph.nodes:
        if node.op == "placeholder":
            if previous is not None:
                raise NotImplementedError("networks take one input")
            previous = node
            continue
        if node.op == "output":
            if node.args[0] is not previous:
                raise NotImplementedError("network output is not the chain's end")
            if pending != (1.0, 0.0):
                raise NotImplementedError("scalar arithmetic after the last activation")
            break
        if node.op == "call_module":
            target = gm.get_submodule(node.target)
            if node.args != (previous,):
                raise NotImplementedError("networks must be single-input chains")
            if isinstance(target, nn.Identity):
                previous = node
                continue
            if isinstance(target, nn.Linear):
                layers.append({"linear": target, "act": None, "param": 0.0, "param2": 0.0,
                               "scale": 1.0, "shift": 0.0, "in_scale": pending[0],
                               "in_shift": pending[1], "norm": None, "norm_scale": 1.0,
                               "norm_shift": 0.0})
                pending = (1.0, 0.0)
                previous = node
                continue
            if isinstance(target, nn.LayerNorm):
                # Feature-wise LayerNorm of a Linear layer's output, before
                # its activation.
                if not layers or layers[-1]["act"] is not None or \
                        layers[-1]["norm"] is not None:
                    raise NotImplementedError("LayerNorm only directly after a Linear layer")
                if tuple(target.normalized_shape) != (layers[-1]["linear"].out_features,):
                    raise NotImplementedError("LayerNorm over other than the layer's features")
                layers[-1]["norm"] = target
                previous = node
                continue
            act = _module_activation(target)
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
                c, b = affine
                if not layers:
                    raise NotImplementedError("scalar arithmetic before the first Linear")
                if layers[-1]["act"] is None and layers[-1]["norm"] is not None:
                    # Between a LayerNorm and the activation: folded into the
                    # LayerNorm's gamma and beta.
                    layers[-1]["norm_scale"] *= c
                    layers[-1]["norm_shift"] = c * layers[-1]["norm_shift"] + b
                elif layers[-1]["act"] is None:
                    # Directly after a Linear: folded into that layer.
                    layers[-1]["scale"] *= c
                    layers[-1]["shift"] = c * layers[-1]["shift"] + b
                else:
                    # After an activation: folded into the next Linear's input.
                    pending = (c * pending[0], c * pending[1] + b)
                previous = node
                continue
            act = _function_activation(target, node.args, node.kwargs, previous)
        else:
            raise NotImplementedError(f"unsupported network node {node.op}")
        if act is None or not layers or layers[-1]["act"] is not None:
            raise NotImplementedError("activations must follow a Linear layer, one each")
        layers[-1]["act"], layers[-1]["param"], layers[-1]["param2"] = act
        previous = node
    if not layers or len(layers) > 3:
        raise NotImplementedError("networks have one to three Linear layers")
    if layers[-1]["act"] is not None:
        raise NotImplementedError("the chain must end in a Linear layer")
    if layers[-1]["norm"] is not None:
        raise NotImplementedError("LayerNorm after the last Linear layer")
    for a, b in zip(layers, layers[1:]):
        if a["linear"].out_features != b["linear"].in_features:
            raise NotImplementedError("network widths do not chain")
    widths = [l["linear"].in_features for l in layers] + \
        [l["linear"].out_features for l in layers[:-1]]
    if max(widths) > 64:
        raise NotImplementedError("network widths above 64")
    return tuple(ScoreLayer(l["linear"], l["act"] or "identity", l["param"], l["param2"],
                            l["scale"], l["shift"], l["in_scale"], l["in_shift"], l["norm"],
                            l["norm_scale"], l["norm_shift"])
                 for l in layers)


__all__ = ["ScoreLayer", "TracedModule", "trace"]

"""``tg.nn.trace``: torch.nn score networks inside ``edge()``.

Mirrors the reference (python/tiga/compiler/nn_capture.py:1-33,
python/tiga/nn/__init__.py): ``trace(module)`` wraps a module so one
``edge()`` source drives two paths:

* called with Torch tensors (eager evaluation) the inputs are concatenated
  along the feature dimension and passed to the module unchanged;
* called with capture proxies the call is recorded as an ``nn`` node over the
  field expressions, which the nn-attention recognizer lowers to the HIP edge
  MLP kernels when the module is a chain the kernels cover.

Covered chains: ``nn.Linear`` layers (bias optional) separated by one
component-wise activation each (relu, leaky_relu, tanh, sigmoid, silu, exact
gelu, elu; module or functional form; ``nn.Identity`` is skipped), ending in
a Linear layer with one output, at most three Linear layers, every width
at most 64.  Anything else runs on the eager evaluator.
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
        "gelu": 6, "elu": 7}


@dataclass(frozen=True)
class ScoreLayer:
    """One Linear layer of a score chain and the activation that follows it."""

    linear: nn.Linear
    act: str = "identity"
    param: float = 0.0


class TracedModule(nn.Module):
    """A module usable both on tensors and on edge() capture proxies."""

    def __init__(self, module: nn.Module):
        super().__init__()
        self.module = module
        self._chain: tuple[ScoreLayer, ...] | None | bool = False

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

    def chain(self) -> tuple[ScoreLayer, ...] | None:
        """The module as a score chain the HIP kernels cover, else None.
        Computed once per module object (a module whose layers are replaced
        afterwards must be wrapped anew by a fresh module object)."""
        if self._chain is False:
            got = _CHAINS.get(self.module, False)
            if got is False:
                try:
                    got = _extract_chain(self.module)
                except NotImplementedError:
                    got = None
                _CHAINS[self.module] = got
            self._chain = got
        return self._chain


def trace(module: nn.Module) -> TracedModule:
    """Wrap ``module`` for use inside ``MessagePassing.edge``."""
    if isinstance(module, TracedModule):
        return module
    if not isinstance(module, nn.Module):
        raise TypeError("tg.nn.trace expects a torch.nn.Module")
    return TracedModule(module)


def _module_activation(m: nn.Module):
    simple = {nn.ReLU: "relu", nn.Tanh: "tanh", nn.Sigmoid: "sigmoid", nn.SiLU: "silu"}
    for cls, name in simple.items():
        if type(m) is cls:
            return name, 0.0
    if type(m) is nn.LeakyReLU:
        return "leaky_relu", float(m.negative_slope)
    if type(m) is nn.ELU:
        return "elu", float(m.alpha)
    if type(m) is nn.GELU and m.approximate == "none":
        return "gelu", 0.0
    return None


def _function_activation(target, args, kwargs, previous):
    from torch.nn import functional as F

    if not args or args[0] is not previous:
        return None
    simple = {torch.relu: "relu", F.relu: "relu", torch.tanh: "tanh",
              torch.sigmoid: "sigmoid", F.silu: "silu"}
    if target in simple and len(args) == 1 and not kwargs:
        return simple[target], 0.0
    if target is F.leaky_relu:
        slope = kwargs.get("negative_slope", args[1] if len(args) > 1 else 0.01)
        return "leaky_relu", float(slope)
    if target is F.elu:
        return "elu", float(kwargs.get("alpha", args[1] if len(args) > 1 else 1.0))
    if target is F.gelu and kwargs.get("approximate", "none") == "none":
        return "gelu", 0.0
    return None


def _extract_chain(module: nn.Module) -> tuple[ScoreLayer, ...]:
    """Linear (act Linear)* with one output, via torch.fx (reference
    nn_capture.py:281-380 translates the same graphs)."""
    import torch.fx

    gm = torch.fx.symbolic_trace(module)
    layers: list[list] = []          # [linear, act, param]
    previous = None
    for node in gm.graph.nodes:
        if node.op == "placeholder":
            if previous is not None:
                raise NotImplementedError("score networks take one input")
            previous = node
            continue
        if node.op == "output":
            if node.args[0] is not previous:
                raise NotImplementedError("score network output is not the chain's end")
            break
        if node.op == "call_module":
            target = gm.get_submodule(node.target)
            if node.args != (previous,):
                raise NotImplementedError("score networks must be single-input chains")
            if isinstance(target, nn.Identity):
                previous = node
                continue
            if isinstance(target, nn.Linear):
                layers.append([target, None, 0.0])
                previous = node
                continue
            act = _module_activation(target)
        elif node.op == "call_function":
            act = _function_activation(node.target, node.args, node.kwargs, previous)
        else:
            raise NotImplementedError(f"unsupported score network node {node.op}")
        if act is None or not layers or layers[-1][1] is not None:
            raise NotImplementedError("activations must follow a Linear layer, one each")
        layers[-1][1], layers[-1][2] = act
        previous = node
    if not layers or len(layers) > 3:
        raise NotImplementedError("score networks have one to three Linear layers")
    if layers[-1][1] is not None or layers[-1][0].out_features != 1:
        raise NotImplementedError("the last layer must be a Linear with one output")
    for (a, _, _), (b, _, _) in zip(layers, layers[1:]):
        if a.out_features != b.in_features:
            raise NotImplementedError("score network widths do not chain")
    if max(max(l.in_features, l.out_features) for l, _, _ in layers) > 64:
        raise NotImplementedError("score network widths above 64")
    return tuple(ScoreLayer(l, a or "identity", p) for l, a, p in layers)


__all__ = ["ScoreLayer", "TracedModule", "trace"]

"""Symbolic capture of ``edge()`` and recognition of the HIP-backed patterns.

``edge()`` is run once on symbolic field proxies (as the reference does with
its ``FieldNamespace``/``Expr`` capture, python/tiga/compiler/capture.py:17-145).
The proxies also implement ``__torch_function__`` so ``F.leaky_relu``,
``torch.sum`` and tensor-on-the-left arithmetic record instead of executing.
The captured tree is then matched against the four patterns that have HIP
kernels:

* weighted sum   ``[edge.w *] src.x``                      with ``tg.sum()``
* edge network   ``tg.nn.trace(net)(fields...) [* c]``     with ``tg.sum()``
* GAT additive   ``leaky_relu((src.h*a_s).sum(-1) + (dst.h*a_d).sum(-1))``,
                 value ``src.h``                            with online softmax
* dot product    ``(src.k*dst.q).sum(-1) [* scale] [+ edge.b]``, value ``src.v``
* varlen / dense the dot product on ``Graph.cu_seqlens`` / ``dense`` / ``triangular``
* nn-scored      ``reducer(tg.nn.trace(net)(fields...), src.v)``
* raw score      ``reducer(role.s [* c], src.v)``, role src, dst or edge

Anything else is not an error: the call runs on the eager Torch evaluator.
"""

from __future__ import annotations

import numbers
from dataclasses import dataclass
from typing import Any

import torch

from .reducer import OnlineSoftmaxItem, ReducerCall


class CaptureError(Exception):
    """The edge function used an operation the capture does not model."""


class Sym:
    __slots__ = ("op", "args", "kw")

    def __init__(self, op: str, args: tuple = (), kw: dict | None = None):
        self.op = op
        self.args = args
        self.kw = kw or {}

    # arithmetic ------------------------------------------------------------
    def __mul__(self, other):
        return Sym("mul", (self, _lift(other)))

    def __rmul__(self, other):
        return Sym("mul", (_lift(other), self))

    def __add__(self, other):
        return Sym("add", (self, _lift(other)))

    def __radd__(self, other):
        return Sym("add", (_lift(other), self))

    def __sub__(self, other):
        return Sym("sub", (self, _lift(other)))

    def __rsub__(self, other):
        return Sym("sub", (_lift(other), self))

    def __truediv__(self, other):
        return Sym("div", (self, _lift(other)))

    def __rtruediv__(self, other):
        return Sym("div", (_lift(other), self))

    def __neg__(self):
        return Sym("neg", (self,))

    def sum(self, dim=None, keepdim=False):
        if keepdim:
            raise CaptureError("keepdim sums are not captured")
        return Sym("sum", (self,), {"dim": dim})

    def __getattr__(self, name):
        raise CaptureError(f"attribute {name!r} is not captured")

    def __bool__(self):
        raise CaptureError("data-dependent control flow is not captured")

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        name = getattr(func, "__name__", str(func))
        if name in ("mul", "__mul__", "multiply"):
            return Sym("mul", (_lift(args[0]), _lift(args[1])))
        if name == "__rmul__":
            return Sym("mul", (_lift(args[1]), _lift(args[0])))
        if name in ("add", "__add__"):
            return Sym("add", (_lift(args[0]), _lift(args[1])))
        if name == "__radd__":
            return Sym("add", (_lift(args[1]), _lift(args[0])))
        if name in ("sub", "__sub__", "subtract"):
            return Sym("sub", (_lift(args[0]), _lift(args[1])))
        if name == "__rsub__":
            return Sym("sub", (_lift(args[1]), _lift(args[0])))
        if name in ("div", "__truediv__", "true_divide", "divide"):
            return Sym("div", (_lift(args[0]), _lift(args[1])))
        if name == "__rtruediv__":
            return Sym("div", (_lift(args[1]), _lift(args[0])))
        if name == "sum":
            dim = args[1] if len(args) > 1 else kwargs.get("dim")
            return _lift(args[0]).sum(dim=dim, keepdim=kwargs.get("keepdim", False))
        if name == "leaky_relu":
            slope = args[1] if len(args) > 1 else kwargs.get("negative_slope", 0.01)
            return Sym("leaky_relu", (_lift(args[0]),), {"slope": float(slope)})
        if name in ("neg", "__neg__", "negative"):
            return Sym("neg", (_lift(args[0]),))
        raise CaptureError(f"torch function {name} is not captured")


def _lift(value) -> Any:
    if isinstance(value, Sym):
        return value
    if isinstance(value, torch.Tensor):
        return Sym("const", (value,))
    if isinstance(value, numbers.Number):
        return Sym("scalar", (float(value),))
    raise CaptureError(f"cannot capture operand of type {type(value).__name__}")


class FieldNamespace:
    def __init__(self, role: str):
        object.__setattr__(self, "_role", role)

    def __getattr__(self, name: str) -> Sym:
        if name.startswith("__"):
            raise AttributeError(name)
        return Sym("field", (self._role, name))


# --------------------------------------------------------------------------
# Pattern recognition.

@dataclass(frozen=True)
class WeightedSum:
    src_field: str
    edge_field: str | None


@dataclass(frozen=True)
class GatAdditive:
    h_field: str          # src.h (value and score source); dst field of the same name
    dst_field: str
    a_src: torch.Tensor
    a_dst: torch.Tensor
    slope: float


@dataclass(frozen=True)
class DotProduct:
    q_field: str          # dst.q
    k_field: str          # src.k
    v_field: str          # src.v
    scale: float
    bias_field: str | None  # edge.b


def _is_field(s, role=None):
    return isinstance(s, Sym) and s.op == "field" and (role is None or s.args[0] == role)


def _is_const(s):
    return isinstance(s, Sym) and s.op == "const"


def _is_scalar(s):
    return isinstance(s, Sym) and s.op == "scalar"


def _pair(s: Sym, pred_a, pred_b):
    """Match a commutative binary node; return (a, b) or None."""
    x, y = s.args
    if pred_a(x) and pred_b(y):
        return x, y
    if pred_a(y) and pred_b(x):
        return y, x
    return None


def _last_dim_sum(s) -> Sym | None:
    if isinstance(s, Sym) and s.op == "sum" and s.kw.get("dim") in (-1,):
        return s.args[0]
    return None


def recognize_weighted_sum(message) -> WeightedSum | None:
    if isinstance(message, ReducerCall):
        if len(message.messages) != 1:
            return None
        message = message.messages[0]
    if _is_field(message, "src"):
        return WeightedSum(message.args[1], None)
    if isinstance(message, Sym) and message.op == "mul":
        m = _pair(message, lambda s: _is_field(s, "src"), lambda s: _is_field(s, "edge"))
        if m is not None:
            return WeightedSum(m[0].args[1], m[1].args[1])
    return None


def _match_weighted_field_sum(s, role):
    """(role.f * C).sum(-1) -> (field name, const tensor)."""
    inner = _last_dim_sum(s)
    if inner is None or inner.op != "mul":
        return None
    m = _pair(inner, lambda x: _is_field(x, role), _is_const)
    if m is None:
        return None
    return m[0].args[1], m[1].args[0]


def recognize_gat(item) -> GatAdditive | None:
    if not isinstance(item, OnlineSoftmaxItem):
        return None
    score, value = item.score, item.value
    if not _is_field(value, "src"):
        return None
    if not (isinstance(score, Sym) and score.op == "leaky_relu"):
        return None
    slope = score.kw["slope"]
    z = score.args[0]
    if not (isinstance(z, Sym) and z.op == "add"):
        return None
    a, b = z.args
    ma, mb = _match_weighted_field_sum(a, "src"), _match_weighted_field_sum(b, "dst")
    if ma is None or mb is None:
        ma, mb = _match_weighted_field_sum(b, "src"), _match_weighted_field_sum(a, "dst")
    if ma is None or mb is None:
        return None
    if ma[0] != value.args[1]:
        return None
    return GatAdditive(h_field=ma[0], dst_field=mb[0], a_src=ma[1], a_dst=mb[1], slope=slope)


def _match_qk(s):
    inner = _last_dim_sum(s)
    if inner is None or inner.op != "mul":
        return None
    m = _pair(inner, lambda x: _is_field(x, "src"), lambda x: _is_field(x, "dst"))
    if m is None:
        return None
    return m[0].args[1], m[1].args[1]   # (k, q)


def _match_scaled_qk(s):
    qk = _match_qk(s)
    if qk is not None:
        return qk, 1.0
    if isinstance(s, Sym) and s.op == "mul":
        m = _pair(s, lambda x: _match_qk(x) is not None, _is_scalar)
        if m is not None:
            return _match_qk(m[0]), m[1].args[0]
    if isinstance(s, Sym) and s.op == "div" and _is_scalar(s.args[1]):
        qk = _match_qk(s.args[0])
        if qk is not None and s.args[1].args[0] != 0:
            return qk, 1.0 / s.args[1].args[0]
    return None


def recognize_dot(item) -> DotProduct | None:
    if not isinstance(item, OnlineSoftmaxItem):
        return None
    score, value = item.score, item.value
    if not _is_field(value, "src"):
        return None
    bias = None
    matched = _match_scaled_qk(score)
    if matched is None and isinstance(score, Sym) and score.op == "add":
        m = _pair(score, lambda x: _match_scaled_qk(x) is not None,
                  lambda x: _is_field(x, "edge"))
        if m is not None:
            matched = _match_scaled_qk(m[0])
            bias = m[1].args[1]
    if matched is None:
        return None
    (k, q), scale = matched
    return DotProduct(q_field=q, k_field=k, v_field=value.args[1], scale=float(scale),
                      bias_field=bias)


@dataclass(frozen=True)
class ScoreSoftmax:
    score_role: str       # src | dst | edge: where the raw score field lives
    score_field: str
    scale: float
    value_field: str      # src.v


def _scaled_field(s):
    """field, scalar * field, field * scalar, field / scalar or -field ->
    (field Sym, scale); else None."""
    if _is_field(s):
        return s, 1.0
    if isinstance(s, Sym) and s.op == "neg" and _is_field(s.args[0]):
        return s.args[0], -1.0
    if isinstance(s, Sym) and s.op == "mul":
        m = _pair(s, _is_field, _is_scalar)
        if m is not None:
            return m[0], m[1].args[0]
    if isinstance(s, Sym) and s.op == "div" and _is_field(s.args[0]) and \
            _is_scalar(s.args[1]) and s.args[1].args[0] != 0:
        return s.args[0], 1.0 / s.args[1].args[0]
    return None


def recognize_score_softmax(item) -> ScoreSoftmax | None:
    """reducer(score_field [* c], src.value): online softmax over a raw
    per-edge score read from a node or edge field (the reference's known
    answer, tests/python/test_message_passing_autograd.py:318-351)."""
    if not isinstance(item, OnlineSoftmaxItem):
        return None
    if not _is_field(item.value, "src"):
        return None
    got = _scaled_field(item.score)
    if got is None:
        return None
    field, scale = got
    return ScoreSoftmax(score_role=field.args[0], score_field=field.args[1], scale=float(scale),
                        value_field=item.value.args[1])


@dataclass(frozen=True)
class NnAttention:
    module: Any                               # tiga.nn.TracedModule
    inputs: tuple[tuple[str, str], ...]       # (role, field) in concatenation order
    value_field: str                          # src.v
    out_scale: float = 1.0                    # scalar applied to the score


def _scaled_nn(s):
    """trace(net)(fields...) optionally times a scalar: (nn Sym, scale)."""
    if isinstance(s, Sym) and s.op == "nn":
        return s, 1.0
    if isinstance(s, Sym) and s.op == "neg" and isinstance(s.args[0], Sym) and \
            s.args[0].op == "nn":
        return s.args[0], -1.0
    if isinstance(s, Sym) and s.op == "mul":
        m = _pair(s, lambda x: isinstance(x, Sym) and x.op == "nn", _is_scalar)
        if m is not None:
            return m[0], m[1].args[0]
    if isinstance(s, Sym) and s.op == "div" and isinstance(s.args[0], Sym) and \
            s.args[0].op == "nn" and _is_scalar(s.args[1]) and s.args[1].args[0] != 0:
        return s.args[0], 1.0 / s.args[1].args[0]
    return None


def _nn_fields(inputs):
    fields = []
    for x in inputs:
        if not _is_field(x):
            return None
        fields.append(tuple(x.args))
    return tuple(fields) if fields else None


def recognize_nn_attention(item) -> NnAttention | None:
    """reducer(trace(net)(fields...) [* c], src.v) with a score chain the
    edge MLP kernels cover (reference compiler/edge_nn_attention.py:66-107)."""
    if not isinstance(item, OnlineSoftmaxItem):
        return None
    value = item.value
    if not _is_field(value, "src"):
        return None
    got = _scaled_nn(item.score)
    if got is None:
        return None
    node, scale = got
    module, inputs = node.args
    fields = _nn_fields(inputs)
    if fields is None or module.chain() is None:
        return None
    return NnAttention(module=module, inputs=fields, value_field=value.args[1],
                       out_scale=float(scale))


@dataclass(frozen=True)
class NnSum:
    module: Any                               # tiga.nn.TracedModule
    inputs: tuple[tuple[str, str], ...]
    out_scale: float = 1.0


def recognize_nn_sum(message) -> NnSum | None:
    """tg.sum() of trace(net)(fields...) [* c]: the reference's edge-NN tile
    (compiler/edge_nn_tile.py:1-30, message_passing.py:2134-2300)."""
    if isinstance(message, ReducerCall):
        if len(message.messages) != 1:
            return None
        message = message.messages[0]
    got = _scaled_nn(message)
    if got is None:
        return None
    node, scale = got
    module, inputs = node.args
    fields = _nn_fields(inputs)
    if fields is None or module.chain(vector=True) is None:
        return None
    return NnSum(module=module, inputs=fields, out_scale=float(scale))


def capture(edge_fn, params: dict[str, Any]):
    """Run ``edge_fn`` on symbolic namespaces; None when it cannot be captured."""
    sym_params = {}
    for name, value in params.items():
        if isinstance(value, numbers.Number) and not isinstance(value, bool):
            sym_params[name] = value
        elif isinstance(value, torch.Tensor):
            sym_params[name] = value
        else:
            sym_params[name] = value
    try:
        return edge_fn(FieldNamespace("src"), FieldNamespace("dst"), FieldNamespace("edge"),
                       sym_params)
    except CaptureError:
        return None
    except (TypeError, AttributeError, RuntimeError, ValueError):
        return None


__all__ = [
    "CaptureError",
    "DotProduct",
    "FieldNamespace",
    "GatAdditive",
    "NnAttention",
    "NnSum",
    "ScoreSoftmax",
    "Sym",
    "WeightedSum",
    "capture",
    "recognize_dot",
    "recognize_gat",
    "recognize_nn_attention",
    "recognize_nn_sum",
    "recognize_score_softmax",
    "recognize_weighted_sum",
]

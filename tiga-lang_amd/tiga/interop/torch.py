"""MessagePassing specializations as ``torch.library`` operators.

Public surface kept from the reference (python/tiga/interop/torch/
library.py:63-205): ``register_message_passing(kernel, graph=..., src=...,
dst=..., edge=..., name=None, **params)`` returns a
``RegisteredMessagePassingOp`` (``qualified_name``, ``operation``,
``topology``, ``bindings``, ``static_params``; callable with ``src=``,
``dst=``, ``edge=``; ``opcheck(*values)``), and the operator's schema is
``tiga::<name>(Tensor row_ptr, Tensor col_idx, Tensor input_0, ...) ->
Tensor`` with the field tensors in (src, dst, edge) order, names sorted.

Design.  A ``_Specialization`` object owns everything one registration
fixes: the kernel, the graph (and with it the per-graph device structures:
row plans, transposed CSR), the operand layout, the non-tensor parameters
and the output's shape and dtype.  Two dispatcher operators are defined
from it:

* ``tiga::<name>`` runs the MessagePassing kernel below autograd, so on
  ROCm tensors it is the HIP path;
* ``tiga::<name>_backward(grad, row_ptr, col_idx, inputs..., needs)``
  recomputes the forward with autograd enabled and differentiates it, which
  on the HIP path replays the HIP forward and runs the fused HIP backward.
  Being an operator of its own, AOT autograd and ``torch.compile`` treat it
  as opaque instead of tracing into the ctypes calls.

Fake kernels give both operators their shapes, so FakeTensor tracing and
``torch.compile(fullgraph=True)`` work.  No hot-path entry point allocates,
copies or synchronises, so the registered op can be captured in a HIP graph
once the per-graph structures exist.
"""

from __future__ import annotations

import hashlib
import re
from dataclasses import dataclass
from typing import Any, Mapping

import torch

_ROLES = ("src", "dst", "edge")
# Registered operators by qualified name; the Library objects must stay alive
# for their dispatcher registrations to stay valid.
_OPS: dict[str, "RegisteredMessagePassingOp"] = {}
_KEEP_ALIVE: list[torch.library.Library] = []


@dataclass(frozen=True)
class RegisteredMessagePassingOp:
    """A registered specialization: call it with the field mappings, or
    call ``operation`` with (row_ptr, col_idx, *inputs) in ``bindings`` order."""

    qualified_name: str
    operation: Any
    topology: tuple[Any, Any]
    bindings: tuple[tuple[str, str], ...]
    static_params: Mapping[str, Any]

    def __call__(self, *, src: Mapping[str, Any], dst: Mapping[str, Any],
                 edge: Mapping[str, Any] | None = None):
        given = {"src": src, "dst": dst, "edge": {} if edge is None else edge}
        for role in _ROLES:
            want = sorted(name for r, name in self.bindings if r == role)
            if sorted(given[role]) != want:
                raise ValueError(f"{role} fields must be {want}, got {sorted(given[role])}")
        inputs = [given[role][name] for role, name in self.bindings]
        return self.operation(*self.topology, *inputs)

    def opcheck(self, *values: Any) -> dict[str, str]:
        """torch.library.opcheck (schema, autograd registration, fake kernel,
        AOT dispatch) on the registered topology and these field values."""
        return torch.library.opcheck(self.operation, (*self.topology, *values))


class _Specialization:
    """What one registration fixes, and the three functions the dispatcher
    calls: forward, backward and the fake (shape-only) forward."""

    def __init__(self, kernel, graph, bindings, params, out_shape, out_dtype):
        self.kernel = kernel
        self.graph = graph
        self.bindings = bindings
        self.params = dict(params)
        self.out_shape = out_shape
        self.out_dtype = out_dtype
        row_ptr, col_idx = graph.resolve_csr()
        self.topology = (row_ptr, col_idx)

    # -- operand handling ----------------------------------------------------
    def graph_for(self, row_ptr, col_idx):
        """The registered graph when the op receives its own topology tensors
        (so its cached device structures are reused), else a new CSR graph
        over the given tensors."""
        from ..graph import Graph

        if row_ptr is self.topology[0] and col_idx is self.topology[1]:
            return self.graph
        same = all(a.data_ptr() == b.data_ptr() and a.shape == b.shape and
                   a.device == b.device for a, b in zip((row_ptr, col_idx), self.topology))
        if same:
            return self.graph
        return Graph.from_csr(row_ptr, col_idx, num_src=self.graph.schema.num_src)

    @staticmethod
    def merge_aliases(inputs):
        """Operands that view the same memory the same way become one tensor
        object again (a field bound both as src and dst, like GAT's h, must
        be one object for the kernel to see the alias)."""
        first: dict[tuple, torch.Tensor] = {}
        merged = []
        for t in inputs:
            key = (t.data_ptr(), t.dtype, t.device, tuple(t.shape), t.stride())
            merged.append(first.setdefault(key, t))
        return merged

    def fields(self, inputs):
        groups: dict[str, dict[str, torch.Tensor]] = {role: {} for role in _ROLES}
        for (role, name), t in zip(self.bindings, inputs):
            groups[role][name] = t
        return groups

    def run(self, row_ptr, col_idx, inputs):
        groups = self.fields(inputs)
        return self.kernel(graph=self.graph_for(row_ptr, col_idx), src=groups["src"],
                           dst=groups["dst"], edge=groups["edge"], **self.params)

    # -- dispatcher functions ------------------------------------------------
    def forward(self, row_ptr, col_idx, *inputs):
        out = self.run(row_ptr, col_idx, self.merge_aliases(inputs))
        # The operator is functional: its result may not alias an operand.
        for t in (row_ptr, col_idx, *inputs):
            if out is t or out._base is t:
                return out.clone()
        return out

    def fake_forward(self, row_ptr, col_idx, *inputs):
        return inputs[0].new_empty(self.out_shape, dtype=self.out_dtype)

    def backward(self, grad, row_ptr, col_idx, *rest):
        inputs, needs = rest[:-1], rest[-1]
        grads = [torch.zeros_like(t) for t in inputs]
        replay = self.merge_aliases([t.detach() for t in inputs])
        wanted: list[tuple[int, torch.Tensor]] = []
        for i, (t, need) in enumerate(zip(replay, needs)):
            # One leaf per distinct tensor: an operand bound twice gets its
            # whole gradient at its first position.
            if need and t.is_floating_point() and all(t is not w for _, w in wanted):
                wanted.append((i, t.requires_grad_(True)))
        if wanted:
            with torch.enable_grad():
                out = self.run(row_ptr, col_idx, replay)
                got = torch.autograd.grad(out, [t for _, t in wanted], grad,
                                          allow_unused=True)
            for (i, _), g in zip(wanted, got):
                if g is not None:
                    grads[i].copy_(g)   # keeps the layout the fake kernel promises
        return grads

    @staticmethod
    def fake_backward(grad, row_ptr, col_idx, *rest):
        return [torch.empty_like(t) for t in rest[:-1]]


def _op_name(kernel, graph, bindings, inputs, params, out_shape, out_dtype) -> str:
    """A stable operator name for a specialization: the kernel class and a
    digest of everything the specialization fixes."""
    key = (type(kernel).__module__, type(kernel).__qualname__, kernel.reducer.specialization_key(),
           graph.planning_key(), bindings,
           [(tuple(t.shape), str(t.dtype)) for t in inputs],
           sorted((k, repr(v)) for k, v in params.items()), out_shape, str(out_dtype))
    digest = hashlib.blake2b(repr(key).encode(), digest_size=10).hexdigest()
    stem = re.sub(r"[^0-9A-Za-z]+", "_", type(kernel).__name__).strip("_").lower() or "kernel"
    return f"mp_{stem}_{digest}"


def register_message_passing(kernel, *, graph, src: Mapping[str, Any], dst: Mapping[str, Any],
                             edge: Mapping[str, Any] | None = None, name: str | None = None,
                             **params: Any) -> RegisteredMessagePassingOp:
    """Register one MessagePassing specialization as a functional Torch
    operator.  The field tensors stay operands; the graph's topology, the
    field names and the non-tensor parameters are fixed by the registration."""
    edge = {} if edge is None else edge
    if graph.schema.realization != "materialized_csr":
        raise NotImplementedError(
            "torch.library registration currently requires a static CSR graph")
    groups = {"src": src, "dst": dst, "edge": edge}
    bindings = tuple((role, n) for role in _ROLES for n in sorted(groups[role]))
    inputs = [groups[role][n] for role, n in bindings]
    if not inputs or not all(isinstance(t, torch.Tensor) for t in inputs):
        raise TypeError("registered MessagePassing fields must be torch.Tensor values")
    if any(isinstance(v, torch.Tensor) for v in params.values()):
        raise TypeError("Tensor parameters must be expressed as src/dst/edge fields")
    with torch.no_grad():
        sample = kernel(graph=graph, src=src, dst=dst, edge=edge, **params)
    if not isinstance(sample, torch.Tensor):
        raise NotImplementedError("the torch.library facade requires one Tensor result")
    out_shape, out_dtype = tuple(sample.shape), sample.dtype
    op = name or _op_name(kernel, graph, bindings, inputs, params, out_shape, out_dtype)
    if not re.fullmatch(r"[A-Za-z][A-Za-z0-9_]*", op):
        raise ValueError("Torch op name must begin with a letter and be alphanumeric/_")
    qualified = f"tiga::{op}"
    if qualified in _OPS:
        return _OPS[qualified]

    spec = _Specialization(kernel, graph, bindings, params, out_shape, out_dtype)
    operands = ", ".join(["Tensor row_ptr", "Tensor col_idx"] +
                         [f"Tensor input_{i}" for i in range(len(bindings))])
    lib = torch.library.Library("tiga", "FRAGMENT")
    lib.define(f"{op}({operands}) -> Tensor")
    lib.define(f"{op}_backward(Tensor grad, {operands}, bool[] needs) -> Tensor[]")
    lib.impl(op, spec.forward, "CompositeExplicitAutograd")
    lib.impl(f"{op}_backward", spec.backward, "CompositeExplicitAutograd")
    torch.library.register_fake(qualified, spec.fake_forward, lib=lib)
    torch.library.register_fake(f"{qualified}_backward", spec.fake_backward, lib=lib)
    backward_op = getattr(torch.ops.tiga, f"{op}_backward").default

    def save_operands(ctx, inputs, output):
        ctx.save_for_backward(*inputs)

    def differentiate(ctx, grad):
        needs = [bool(n) for n in ctx.needs_input_grad[2:]]
        if not any(needs):
            return (None,) * len(ctx.needs_input_grad)
        grads = backward_op(grad, *ctx.saved_tensors, needs)
        return (None, None, *(g if n else None for g, n in zip(grads, needs)))

    torch.library.register_autograd(qualified, differentiate, setup_context=save_operands,
                                    lib=lib)
    registered = RegisteredMessagePassingOp(
        qualified_name=qualified, operation=getattr(torch.ops.tiga, op).default,
        topology=spec.topology, bindings=bindings, static_params=dict(params))
    _KEEP_ALIVE.append(lib)
    _OPS[qualified] = registered
    return registered


# The reference's interop.torch.Graph is the Torch-backed relation, which
# here is tiga.Graph itself.
from ..graph import Graph  # noqa: E402

__all__ = ["Graph", "RegisteredMessagePassingOp", "register_message_passing"]

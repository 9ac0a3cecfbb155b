"""``torch.library`` registration of MessagePassing specializations.

Mirrors the reference facade (python/tiga/interop/torch/library.py:23-208):
``register_message_passing(kernel, graph=..., src=..., dst=..., edge=...,
name=None, **params)`` defines one functional dispatcher op
``tiga::<name>(Tensor row_ptr, Tensor col_idx, Tensor input_0, ...) ->
Tensor`` whose operands are the field tensors in (src, dst, edge) order,
sorted by name, so ``torch.compile(fullgraph=True)``, FakeTensor tracing and
AOT autograd see one opaque op.

Implementation: the op's kernel calls the MessagePassing kernel itself, so
on ROCm tensors it runs this package's HIP path (below autograd).  Its
registered autograd formula recomputes the call with autograd enabled and
differentiates it: on the HIP path that replays the HIP forward and runs the
fused HIP backward (the reference replays its eager oracle instead).  The
fake kernel returns an empty tensor of the specialization's output shape and
dtype, taken from one call at registration.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass
from typing import Any, Mapping

import torch

_LIBRARIES: list[Any] = []
_REGISTERED: dict[str, "RegisteredMessagePassingOp"] = {}


def _ordered_fields(*groups: Mapping[str, Any]):
    return tuple((role, name)
                 for role, group in zip(("src", "dst", "edge"), groups, strict=True)
                 for name in sorted(group))


@dataclass(frozen=True)
class RegisteredMessagePassingOp:
    """One dispatcher binding for a MessagePassing specialization."""

    qualified_name: str
    operation: Any
    topology: tuple[Any, Any]
    bindings: tuple[tuple[str, str], ...]
    static_params: Mapping[str, Any]

    def __call__(self, *, src: Mapping[str, Any], dst: Mapping[str, Any],
                 edge: Mapping[str, Any] | None = None):
        edge = {} if edge is None else edge
        groups = {"src": src, "dst": dst, "edge": edge}
        expected = {role: {name for candidate, name in self.bindings if candidate == role}
                    for role in ("src", "dst", "edge")}
        for role, group in groups.items():
            if set(group) != expected[role]:
                raise ValueError(f"{role} fields must be {sorted(expected[role])}, "
                                 f"got {sorted(group)}")
        return self.operation(*self.topology,
                              *(groups[role][name] for role, name in self.bindings))

    def opcheck(self, *values: Any) -> dict[str, str]:
        """PyTorch's schema / autograd / FakeTensor / AOT conformance checks."""
        return torch.library.opcheck(self.operation, (*self.topology, *values))


def register_message_passing(kernel, *, graph, src: Mapping[str, Any], dst: Mapping[str, Any],
                             edge: Mapping[str, Any] | None = None, name: str | None = None,
                             **params: Any) -> RegisteredMessagePassingOp:
    """Register a MessagePassing specialization as a functional Torch op
    (reference library.py:63-205).  Tensor fields stay dispatcher operands;
    the graph topology, field names and non-Tensor parameters are fixed."""
    from ..graph import Graph

    edge = {} if edge is None else edge
    if graph.schema.realization != "materialized_csr":
        raise NotImplementedError(
            "torch.library registration currently requires a static CSR graph")
    row_ptr, col_idx = graph.resolve_csr()
    bindings = _ordered_fields(src, dst, edge)
    groups = {"src": src, "dst": dst, "edge": edge}
    values = tuple(groups[role][field] for role, field in bindings)
    if not values or any(not isinstance(value, torch.Tensor) for value in values):
        raise TypeError("registered MessagePassing fields must be torch.Tensor values")
    if any(isinstance(value, torch.Tensor) for value in params.values()):
        raise TypeError("Tensor parameters must be expressed as src/dst/edge fields")

    with torch.no_grad():
        sample = kernel(graph=graph, src=src, dst=dst, edge=edge, **params)
    if not isinstance(sample, torch.Tensor):
        raise NotImplementedError("the torch.library facade requires one Tensor result")
    output_shape, output_dtype = tuple(sample.shape), sample.dtype
    signature = repr((type(kernel).__module__, type(kernel).__qualname__,
                      kernel.reducer.specialization_key(), graph.planning_key(), bindings,
                      tuple((tuple(v.shape), str(v.dtype)) for v in values),
                      tuple(sorted((k, repr(v)) for k, v in params.items())),
                      output_shape, str(output_dtype)))
    op_name = name or f"message_passing_{hashlib.sha256(signature.encode()).hexdigest()[:20]}"
    if not op_name.replace("_", "").isalnum() or not op_name[0].isalpha():
        raise ValueError("Torch op name must begin with a letter and be alphanumeric/_")
    qualified = f"tiga::{op_name}"
    found = _REGISTERED.get(qualified)
    if found is not None:
        return found

    library = torch.library.Library("tiga", "FRAGMENT")
    arguments = ", ".join(["Tensor row_ptr", "Tensor col_idx",
                           *(f"Tensor input_{i}" for i in range(len(bindings)))])
    library.define(f"{op_name}({arguments}) -> Tensor")
    num_src = graph.schema.num_src

    def topology_key(rp, ci):
        return (rp.data_ptr(), ci.data_ptr(), tuple(rp.shape), tuple(ci.shape), str(rp.device))

    registered_key = topology_key(row_ptr, col_idx)

    def runtime_graph(flat):
        # The registered topology keeps its graph object, and with it the
        # per-graph device structures (row plans, transposed CSR).
        if topology_key(flat[0], flat[1]) == registered_key:
            return graph
        return Graph.from_csr(flat[0], flat[1], num_src=num_src, validate="basic")

    def canonical(values):
        """Operands that are one tensor (same storage, layout and dtype) become
        one object again, as the kernel saw them at registration (a field used
        as both src and dst, like GAT's h)."""
        seen, out = {}, []
        for value in values:
            key = (value.data_ptr(), tuple(value.shape), tuple(value.stride()), value.dtype,
                   str(value.device))
            out.append(seen.setdefault(key, value))
        return out

    def unpack(flat):
        groups_out = {"src": {}, "dst": {}, "edge": {}}
        for (role, field), value in zip(bindings, flat, strict=True):
            groups_out[role][field] = value
        return groups_out

    def implementation(*flat):
        fields = unpack(canonical(flat[2:]))
        out = kernel(graph=runtime_graph(flat), src=fields["src"], dst=fields["dst"],
                     edge=fields["edge"], **params)
        # A functional op must not return an alias of an operand.
        return out.clone() if any(out is t or out._base is t for t in flat) else out

    library.impl(op_name, implementation, "CompositeExplicitAutograd")

    def fake(*flat):
        return flat[2].new_empty(output_shape, dtype=output_dtype)

    torch.library.register_fake(qualified, fake, lib=library)

    # The backward is an opaque op of its own, so AOT autograd and
    # torch.compile trace it like the forward instead of tracing into the
    # HIP calls it makes.
    library.define(f"{op_name}_backward(Tensor grad, {arguments}, bool[] needs) -> Tensor[]")

    def backward_implementation(grad, *rest):
        flat, needs = rest[:-1], rest[-1]
        replay = list(flat[:2]) + canonical([t.detach() for t in flat[2:]])
        differentiable, positions = [], []
        for index, need in enumerate(needs):
            local = replay[2 + index]
            # A tensor given at several positions gets its whole gradient at
            # the first one that needs it (the others stay zero).
            if need and (local.is_floating_point() or local.is_complex()) and \
                    not any(local is d for d in differentiable):
                local.requires_grad_(True)
                differentiable.append(local)
                positions.append(index)
        gradients = [torch.zeros_like(t) for t in flat[2:]]
        if differentiable:
            fields = unpack(replay[2:])
            with torch.enable_grad():
                output = kernel(graph=runtime_graph(replay), src=fields["src"],
                                dst=fields["dst"], edge=fields["edge"], **params)
                computed = torch.autograd.grad(output, differentiable, grad,
                                               allow_unused=True)
            # Copied into zeros_like(input) so the result has exactly the
            # layout the fake kernel promises.
            for position, gradient in zip(positions, computed, strict=True):
                if gradient is not None:
                    gradients[position].copy_(gradient)
        return gradients

    library.impl(f"{op_name}_backward", backward_implementation, "CompositeExplicitAutograd")

    def backward_fake(grad, *rest):
        return [torch.empty_like(t) for t in rest[2:-1]]

    torch.library.register_fake(f"{qualified}_backward", backward_fake, lib=library)
    backward_op = getattr(getattr(torch.ops.tiga, f"{op_name}_backward"), "default")

    def setup_context(ctx, inputs, output):
        del output
        ctx.save_for_backward(*inputs)

    def backward(context, grad_output):
        needs = [bool(n) for n in context.needs_input_grad[2:]]
        if not any(needs):
            return (None,) * len(context.needs_input_grad)
        grads = backward_op(grad_output, *context.saved_tensors, needs)
        return (None, None, *(g if need else None for g, need in zip(grads, needs)))

    torch.library.register_autograd(qualified, backward, setup_context=setup_context,
                                    lib=library)
    operation = getattr(getattr(torch.ops.tiga, op_name), "default")
    registered = RegisteredMessagePassingOp(qualified_name=qualified, operation=operation,
                                            topology=(row_ptr, col_idx), bindings=bindings,
                                            static_params=dict(params))
    _LIBRARIES.append(library)   # dispatcher registrations live as long as the Library
    _REGISTERED[qualified] = registered
    return registered


__all__ = ["RegisteredMessagePassingOp", "register_message_passing"]

"""``tiga.MessagePassing``: the Torch-facing facade of the HIP provider.

Call form and validation follow the reference adapter
(python/tiga/interop/torch/message_passing.py:1490-1651, 3565-3586):
``K()(graph=G, src={...}, dst={...}, edge={...}, **params) -> torch.Tensor``,
``edge(self, src, dst, edge, **params)`` and ``node(self, dst, aggregate,
**params)``.

Dispatch: the edge function is captured once per parameter structure and
matched against the patterns that have gfx950 kernels (``capture.py``).  A
recognized pattern on ROCm tensors of a supported dtype/shape runs through
``torch.autograd.Function`` bridges over libtgx_hip.so and nothing else: if
the library is missing it raises.  Edge functions no kernel covers (and CPU
tensors) run on the eager Torch evaluator, which restates the reference's own
fallback (``_evaluate_reference`` 2848-2894); ``explain()`` reports which path
ran.  Setting ``tiga.config.strict = True`` turns that fallback into an error.
"""

from __future__ import annotations

import functools
import inspect
from collections.abc import Mapping
from types import SimpleNamespace
from typing import Any

import torch

from . import _eager, _native
from . import capture as cap
from .graph import Graph
from .kernel import CompiledVariant, Kernel
from .reducer import OnlineSoftmaxReducer, SumReducer


class _Config:
    strict = False


config = _Config()


@functools.lru_cache(maxsize=512)
def _parameter_names(function) -> tuple[bool, frozenset]:
    """(takes **kwargs, parameter names) of a function, computed once."""
    signature = inspect.signature(function)
    accepts_rest = any(p.kind is inspect.Parameter.VAR_KEYWORD
                       for p in signature.parameters.values())
    return accepts_rest, frozenset(signature.parameters)


def _call_region(method, positional: tuple, params: Mapping[str, Any]):
    accepts_rest, names = _parameter_names(getattr(method, "__func__", method))
    selected = params if accepts_rest else {
        name: value for name, value in params.items() if name in names}
    return method(*positional, **selected)


class MessagePassing(Kernel):
    reducer = SumReducer()

    def __init__(self) -> None:
        super().__init__()

    def edge(self, src, dst, edge, **params):
        raise NotImplementedError

    def node(self, dst, aggregate, **params):
        return aggregate

    # ------------------------------------------------------------------
    @staticmethod
    def _validate_fields(role: str, fields, entity_count: int, device) -> None:
        if not isinstance(fields, Mapping):
            raise TypeError(f"{role} fields must be a mapping")
        for name, value in fields.items():
            if not isinstance(value, torch.Tensor):
                raise TypeError(f"{role}.{name} must be a torch.Tensor")
            if value.ndim == 0 or value.shape[0] != entity_count:
                raise ValueError(
                    f"{role}.{name} leading dimension must be {entity_count}, "
                    f"got shape {tuple(value.shape)}")
            if value.device != device:
                raise ValueError(f"{role}.{name} is on {value.device}, but graph is on {device}")

    def _captured(self, params):
        # Captured afresh on every call: the tree holds the module's current
        # tensors (e.g. attention vectors), which a cache could leave stale.
        return cap.capture(lambda s, d, e, p: _call_region(self.edge, (s, d, e), p), params)

    def __call__(self, *, graph: Graph, src: Mapping[str, torch.Tensor],
                 dst: Mapping[str, torch.Tensor], edge: Mapping[str, torch.Tensor] | None = None,
                 **params: Any):
        if not getattr(graph, "_tiga_graph", False):
            raise TypeError("graph must be a tiga.Graph")
        edge = {} if edge is None else edge
        device = graph.device
        self._validate_fields("src", src, graph.schema.num_src, device)
        self._validate_fields("dst", dst, graph.schema.num_dst, device)
        prune = (self.reducer.block_prune_threshold
                 if isinstance(self.reducer, OnlineSoftmaxReducer) else None)
        if prune is not None and not graph.is_dense:
            # reference message_passing/core.py:500-505
            raise NotImplementedError(
                "block_prune_threshold is defined for dense relations only; refusing to "
                "run exact softmax on a CSR relation")
        captured = self._captured(params)
        result = None
        if device.type == "cuda" and captured is not None:
            result = self._execute_native(captured, graph, src, dst, edge, params)
        if result is None and prune is not None:
            # reference interop/torch/message_passing.py:1611-1616
            raise NotImplementedError(
                "block_prune_threshold requires the dense attention tile (dot-product "
                "score, bf16/fp16, head_dim 64 or 128, on the GPU); refusing to silently "
                "execute exact softmax or materialize the Cartesian relation")
        if result is None:
            if config.strict:
                raise RuntimeError(
                    f"{type(self).__qualname__}: no HIP kernel covers this edge function / "
                    "dtype / shape and tiga.config.strict is set")
            if not graph.is_varlen:
                self._validate_fields("edge", edge, graph.num_edges, device)
            self._record_variant(CompiledVariant(
                key=(type(self).__qualname__, "eager", graph.planning_key()),
                backend="torch-eager", provider="torch", pattern="generic",
                lowering="gather -> edge() -> scatter reduce (Torch ops)",
                remarks=("edge function not covered by a HIP kernel",)))
            aggregate = _eager.evaluate(self, graph, src, dst, edge, params)
        else:
            aggregate = result
        if type(self).node is MessagePassing.node:
            return aggregate
        return _call_region(self.node, (SimpleNamespace(**dst), aggregate), params)

    def reference(self, *, graph: Graph, src: Mapping[str, torch.Tensor],
                  dst: Mapping[str, torch.Tensor],
                  edge: Mapping[str, torch.Tensor] | None = None, **params: Any):
        """Run the eager Torch evaluator even where a HIP kernel exists
        (reference interop/torch/message_passing.py:2818-2894)."""
        if isinstance(self.reducer, OnlineSoftmaxReducer) and \
                self.reducer.block_prune_threshold is not None:
            raise NotImplementedError(
                "the schedule-dependent block-pruned approximation has no eager "
                "edge-materializing reference; compare against an exact online-softmax "
                "result with an explicit accuracy budget")
        if not getattr(graph, "_tiga_graph", False):
            raise TypeError("graph must be a tiga.Graph")
        edge = {} if edge is None else edge
        device = graph.device
        self._validate_fields("src", src, graph.schema.num_src, device)
        self._validate_fields("dst", dst, graph.schema.num_dst, device)
        if not graph.is_varlen:
            self._validate_fields("edge", edge, graph.num_edges, device)
        aggregate = _eager.evaluate(self, graph, src, dst, edge, params)
        if type(self).node is MessagePassing.node:
            return aggregate
        return _call_region(self.node, (SimpleNamespace(**dst), aggregate), params)

    # ------------------------------------------------------------------
    def _record_native(self, graph, pattern: str, entry_points, lowering, remarks=()):
        plan = graph._native_cache.get(("plan", 512, 512))
        # The record of a (kernel, pattern) on this graph is built once and
        # kept with the graph's other per-graph structures.
        memo = graph._native_cache.setdefault("variants", {})
        memo_key = (type(self).__qualname__, plan is not None, pattern, tuple(entry_points),
                    lowering, tuple(remarks))
        variant = memo.get(memo_key)
        if variant is None:
            extra = () if plan is None else (f"row plan: {plan.counts()}",)
            variant = CompiledVariant(
                key=(type(self).__qualname__, pattern, graph.planning_key()),
                backend="hip", provider="libtgx_hip.so (gfx950)", pattern=pattern,
                lowering=lowering, entry_points=tuple(entry_points),
                remarks=tuple(remarks) + extra)
            memo[memo_key] = variant
        self._record_variant(variant)

    def _execute_native(self, captured, graph, src, dst, edge, params):
        from . import _ops

        if isinstance(self.reducer, SumReducer):
            if self.reducer.identity_value != 0 or graph.is_varlen or graph.is_dense:
                return None
            pat = cap.recognize_weighted_sum(captured)
            if pat is None or pat.src_field not in src:
                return None
            x = src[pat.src_field]
            w = None
            if pat.edge_field is not None:
                if pat.edge_field not in edge:
                    return None
                w = edge[pat.edge_field]
                E = graph.num_edges
                if tuple(w.shape) not in ((E,), (E, 1)) or w.dtype != torch.float32:
                    return None
                if x.ndim == 1 and w.ndim == 2:
                    return None
            if x.dtype != torch.float32:
                return None
            _native.lib()
            out = _ops.CsrSumFunction.apply(x, w, graph)
            self._record_native(graph, "weighted-sum", ("tgx_csr_sum_fwd", "tgx_csr_sum_bwd"),
                                "degree-binned rows -> wave gather-FMA (fp32)")
            return out

        if not isinstance(self.reducer, OnlineSoftmaxReducer):
            return None
        gat = cap.recognize_gat(captured)
        if gat is not None and not graph.is_varlen and not graph.is_dense:
            h = src.get(gat.h_field)
            hd = dst.get(gat.dst_field)
            if h is None or hd is None or hd is not h:
                return None
            if graph.schema.num_src != graph.schema.num_dst or h.ndim != 3:
                return None
            N, H, D = h.shape
            if h.dtype != torch.float32 or tuple(gat.a_src.shape) not in ((H, D), (1, H, D)) \
                    or tuple(gat.a_dst.shape) not in ((H, D), (1, H, D)):
                return None
            if gat.a_src.dtype != torch.float32 or gat.a_dst.dtype != torch.float32:
                return None
            if gat.a_src.device != h.device or gat.a_dst.device != h.device:
                return None
            if H * D not in (64, 128, 256) or D % 4:
                return None
            if self.reducer.accumulation_dtype not in (None, torch.float32, "float32"):
                return None
            _native.lib()
            out = _ops.GatFunction.apply(h, gat.a_src, gat.a_dst, gat.slope, graph)
            self._record_native(graph, "gat-additive", ("tgx_gat_fwd", "tgx_gat_bwd"),
                                "online softmax per (row, head), logsumexp saved; "
                                "backward recomputes alpha over the transposed CSR")
            return out
        dot = cap.recognize_dot(captured)
        if dot is not None:
            return self._execute_dot(dot, graph, src, dst, edge)
        nn_item = cap.recognize_nn_attention(captured)
        if nn_item is not None:
            return self._execute_nn_attention(nn_item, graph, src, dst, edge)
        return None

    def _execute_nn_attention(self, item, graph, src, dst, edge):
        """tg.nn.trace-scored attention on the edge MLP kernels (reference
        interop/torch/message_passing.py:2372-2577, envelope: fp32, CSR
        relation, one score per edge, one gathered value field)."""
        from . import _ops

        if graph.is_varlen or graph.is_dense:
            return None
        if self.reducer.accumulation_dtype not in (None, torch.float32, "float32"):
            return None
        groups = {"src": src, "dst": dst, "edge": edge}
        rows = {"src": graph.schema.num_src, "dst": graph.schema.num_dst,
                "edge": graph.num_edges}
        fields, roles = [], []
        for role, name in item.inputs:
            t = groups[role].get(name)
            if t is None or t.dtype != torch.float32 or t.ndim not in (1, 2) or \
                    t.shape[0] != rows[role]:
                return None
            fields.append(t if t.ndim == 2 else t.unsqueeze(-1))
            roles.append(role)
        if len(fields) > 4 or sum(f.shape[1] for f in fields) > 64:
            return None
        value = src.get(item.value_field)
        if value is None or value.dtype != torch.float32:
            return None
        chain = item.module.chain()
        for layer in chain:
            for p in (layer.linear.weight, layer.linear.bias):
                if p is not None and (p.dtype != torch.float32 or p.device != value.device):
                    return None
        _native.lib()
        out = _ops.nn_attention(graph, chain, roles, fields, value)
        widths = "-".join(str(l.linear.in_features) for l in chain) + "-1"
        self._record_native(
            graph, "nn-attention",
            ("tgx_edge_mlp_scores", "tgx_segment_softmax_fwd", "tgx_csr_sum_fwd",
             "tgx_csr_sum_bwd", "tgx_segment_softmax_bwd", "tgx_edge_mlp_backward"),
            f"edge-parallel score network {widths} (one edge per lane, uniform weights), "
            "segment softmax per row, weighted CSR sum of the value; backward through the "
            "softmax Jacobian, per-edge network replay, weight gradients as GEMMs")
        return out

    def _execute_dot(self, dot, graph, src, dst, edge):
        from . import _ops

        q, k, v = dst.get(dot.q_field), src.get(dot.k_field), src.get(dot.v_field)
        if q is None or k is None or v is None:
            return None
        if q.ndim != 3 or k.shape[1:] != q.shape[1:] or v.shape[1:] != q.shape[1:]:
            return None
        _, H, D = q.shape
        if self.reducer.accumulation_dtype not in (None, torch.float32, "float32"):
            return None
        if graph.is_varlen or graph.is_dense:
            return self._execute_block_attention(dot, graph, q, k, v)
        if not (q.dtype == k.dtype == v.dtype == torch.bfloat16):
            return None
        if D % 8 or H * D not in (128, 256, 512):
            return None
        bias = None
        if dot.bias_field is not None:
            bias = edge.get(dot.bias_field)
            if bias is None or bias.dtype != torch.float32:
                return None
            if graph.is_varlen:
                return None
            if tuple(bias.shape) not in ((graph.num_edges, H), (graph.num_edges, H, 1)):
                return None
            bias = bias.reshape(graph.num_edges, H)
        if graph.is_varlen:
            return None
        _native.lib()
        out = _ops.DotAttnFunction.apply(q, k, v, bias, dot.scale, graph)
        self._record_native(graph, "dot-product", ("tgx_dot_attn_fwd", "tgx_dot_attn_bwd"),
                            "bf16 gathers, fp32 online softmax per (row, head); hub rows "
                            "split and merged; backward over CSR (dq, dbias) and transposed "
                            "CSR (dk, dv)")
        return out


    def _execute_block_attention(self, dot, graph, q, k, v):
        """Dot-product attention over Graph.cu_seqlens / dense / triangular
        on MFMA tiles (reference: eager oracle for varlen, compiled fp16
        dense streaming tile for dense/triangular, message_passing.py:
        1910-2020)."""
        from . import _ops

        if dot.bias_field is not None:
            return None
        if not (q.dtype == k.dtype == v.dtype) or q.dtype not in _ops._ATTN_DTYPES:
            return None
        _, H, D = q.shape
        if D not in (64, 128):
            return None
        if q.shape[0] != graph.schema.num_dst or k.shape[0] != graph.schema.num_src or \
                v.shape[0] != graph.schema.num_src:
            return None
        prune = self.reducer.block_prune_threshold
        if prune is not None and torch.is_grad_enabled() and \
                any(t.requires_grad for t in (q, k, v)):
            raise NotImplementedError(
                "block_prune_threshold is a forward-only approximation (no gradient); run "
                "it under torch.no_grad() or drop the threshold for exact softmax")
        _native.lib()
        out = _ops.BlockAttentionFunction.apply(q, k, v, dot.scale, float(prune or 0.0), graph)
        relation = ("cu_seqlens" if graph.is_varlen else graph.schema.origin)
        causal = graph._attn_blocks()[2]
        self._record_native(
            graph, "block-attention", ("tgx_attn_fwd", "tgx_attn_bwd"),
            f"MFMA 16x16x32 {str(q.dtype).split('.')[-1]} flash tiles over the implicit "
            f"{relation} relation ({'causal' if causal else 'all pairs'}); XCD-grouped "
            "tasks; atomic-free dK/dV and dQ passes",
            remarks=(("block-pruned tile admission (approximate)",) if prune else ()))
        return out


__all__ = ["MessagePassing", "config"]

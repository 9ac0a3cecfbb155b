"""``tiga.MessagePassing``: the Torch-facing facade of the HIP provider.

Call forms follow the reference (python/tiga/message_passing/core.py:32-50,
543-766 and python/tiga/interop/torch/message_passing.py:1490-1651,
3565-3586, 3827-3879):

* ``K()(graph=G, src={...}, dst={...}, edge={...}, **params) -> Tensor``,
  or ``ndata={...}`` in place of ``src``/``dst`` on a homogeneous relation;
* ``K().prepare(graph=G, ...)`` -> a zero-argument launch with the graph,
  the bindings, shapes and strides frozen (tensor contents stay live);
* ``edge(self, src, dst, edge, **params)``, ``node(self, dst, aggregate,
  **params)``; ``explain()``, ``last_variant``, ``cache_info``.

Dispatch.  A cold call validates the fields, captures ``edge()`` on symbolic
proxies and matches the capture against the patterns with gfx950 kernels
(``capture.py``).  A match on ROCm tensors of a supported dtype/shape becomes
a *launch*: the pattern's operands named by binding (``src.x``, ``edge.w``,
a tensor parameter) and a runner over ``torch.autograd.Function`` bridges
into libtgx_hip.so, which raises if the library is missing.  When every
operand comes from the call's own fields or parameters, the launch is kept
with guards (same graph object, same reducer, same parameter values, every
operand with the same dtype/shape/strides/device, required aliases, and
the same values for the scalars edge() reads from the kernel's attributes,
its module's globals and its closure); a warm call that passes the guards
runs it directly, skipping capture, recognition and validation, like the
reference's guarded executable (:974-1008).  A
launch that holds a tensor from outside the call (a closure or attribute)
is re-captured on every call instead, so rebinding that name is seen.

Edge functions no kernel covers (and CPU tensors) run the eager Torch
evaluator, the reference's own fallback (``_evaluate_reference``
2848-2894); ``explain()`` reports which path ran and
``tiga.config.strict = True`` turns that fallback into an error.
"""

from __future__ import annotations

import functools
import inspect
import numbers
import warnings
from collections.abc import Callable, Mapping
from dataclasses import dataclass
from types import CodeType, SimpleNamespace
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

_MISS = object()


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


def _resolve_node_fields(graph, src, dst, ndata):
    """``ndata=`` binds one mapping to both endpoint roles of a homogeneous
    relation (reference message_passing/core.py:32-50)."""
    if ndata is not None:
        if src is not None or dst is not None:
            raise TypeError("ndata= cannot be combined with src=/dst=")
        if graph.schema.num_src != graph.schema.num_dst:
            raise ValueError(
                "ndata= requires a homogeneous relation (num_src == num_dst); "
                "declare src= and dst= separately for bipartite graphs")
        src = dst = dict(ndata)
    if src is None or dst is None:
        raise TypeError("message passing requires ndata= or both src= and dst= mappings")
    return src, dst


def _spec(t: torch.Tensor) -> tuple:
    return (t.dtype, t.shape, t.stride(), t.device)


def _param_signature(params: Mapping[str, Any]) -> tuple:
    """Parameter names with the values a capture may have baked in: numbers
    and other hashable values by value, tensors by kind only (a launch
    reads its tensor operands from the call), anything else by identity."""
    sig = []
    for name in sorted(params):
        value = params[name]
        if isinstance(value, torch.Tensor):
            sig.append((name, "tensor"))
        elif isinstance(value, (numbers.Number, str, bytes, type(None))):
            sig.append((name, type(value), value))
        else:
            sig.append((name, "object", id(value)))
    return tuple(sig)


_SCALARS = (numbers.Number, str, bytes, type(None))


def _scalar(value) -> bool:
    """A value a capture bakes into the launch as a constant (a number, a
    string, or a tuple of them), as opposed to an operand it reads."""
    return isinstance(value, _SCALARS) or (
        isinstance(value, tuple) and all(isinstance(v, _SCALARS) for v in value))


@functools.lru_cache(maxsize=512)
def _code_names(function) -> tuple:
    """Attribute and global names read by `function`'s code and the code
    objects nested in it (lambdas, comprehensions)."""
    names, stack = set(), [function.__code__]
    while stack:
        code = stack.pop()
        names.update(code.co_names)
        stack.extend(c for c in code.co_consts if isinstance(c, CodeType))
    return tuple(sorted(names))


def _lookup(kernel, function, kind: str, name):
    """The current value of one outside name edge() reads: an attribute of
    the kernel (instance, then class; descriptors such as properties are
    not run), a global of edge()'s module, or a closure cell."""
    if kind == "attr":
        if name in kernel.__dict__:
            return kernel.__dict__[name]
        for cls in type(kernel).__mro__:
            if name in cls.__dict__:
                return cls.__dict__[name]
        return _MISS
    if kind == "global":
        return function.__globals__.get(name, _MISS)
    try:
        return function.__closure__[name].cell_contents
    except (TypeError, IndexError, ValueError):
        return _MISS


class _Environment:
    """The scalars edge() reads from outside the call: kernel attributes
    (self.slope), class attributes, module globals and closure variables
    that held a number or string when the launch was captured.  The capture
    bakes these in as constants (a LeakyReLU slope, a score scale), so a
    warm call re-runs the launch only while every one still has its value.
    Scalars reached other ways (through another object's attribute, or a
    helper function's globals) are not tracked."""

    def __init__(self, kernel):
        function = getattr(kernel.edge, "__func__", kernel.edge)
        keys = []
        for name in _code_names(function):
            for kind in ("attr", "global"):
                if _scalar(_lookup(kernel, function, kind, name)):
                    keys.append((kind, name))
        for index in range(len(function.__closure__ or ())):
            if _scalar(_lookup(kernel, function, "cell", index)):
                keys.append(("cell", index))
        self.keys = tuple(keys)
        self.values = self.snapshot(kernel)

    def snapshot(self, kernel) -> tuple:
        function = getattr(kernel.edge, "__func__", kernel.edge)
        return tuple(_lookup(kernel, function, kind, name) for kind, name in self.keys)

    def holds(self, kernel) -> bool:
        now = self.snapshot(kernel)
        # Compared by type and value: 1 and 1.0 can bake in differently.
        return all(type(a) is type(b) and a == b for a, b in zip(now, self.values))


@dataclass
class _Launch:
    """A recognized pattern bound to its HIP runner.

    operands: (role, name) per runner argument, role in src/dst/edge/param,
    or ("fixed", object) for something the capture took from outside the
    call.  aliases: pairs of bindings that must be the same tensor."""

    graph: Graph
    operands: tuple
    runner: Callable
    describe: Callable[[], CompiledVariant]
    aliases: tuple = ()
    variant: CompiledVariant | None = None
    # Optional: operands -> a zero-argument launch with its native arguments
    # bound (prepare()'s no-grad form), or None where that does not apply.
    bind: Callable | None = None

    @property
    def guardable(self) -> bool:
        return all(role != "fixed" for role, _ in self.operands)

    def gather(self, src, dst, edge, params) -> list:
        groups = {"src": src, "dst": dst, "edge": edge, "param": params}
        return [name if role == "fixed" else groups[role][name]
                for role, name in self.operands]


class _Guarded:
    """A launch plus the guards under which a warm call may re-run it."""

    def __init__(self, launch: _Launch, kernel, operands, params):
        self.launch = launch
        self.reducer = kernel.reducer
        self.specs = tuple(_spec(t) for t in operands)
        self.param_sig = _param_signature(params)
        self.environment = _Environment(kernel)
        self.names: tuple | None = None

    @staticmethod
    def _names(src, dst, edge) -> tuple:
        # Which fields are bound can steer Python code inside edge().
        return tuple(src), tuple(dst), tuple(edge)

    def try_run(self, kernel, graph, src, dst, edge, params):
        launch = self.launch
        if graph is not launch.graph or kernel.reducer is not self.reducer:
            return _MISS
        try:
            operands = launch.gather(src, dst, edge, params)
        except (KeyError, TypeError):
            return _MISS
        for t, spec in zip(operands, self.specs):
            if not isinstance(t, torch.Tensor) or _spec(t) != spec:
                return _MISS
        if launch.aliases:
            groups = {"src": src, "dst": dst, "edge": edge, "param": params}
            for (ra, na), (rb, nb) in launch.aliases:
                if groups[ra].get(na) is not groups[rb].get(nb):
                    return _MISS
        if self._names(src, dst, edge) != self.names or \
                _param_signature(params) != self.param_sig or \
                not self.environment.holds(kernel):
            return _MISS
        return launch.runner(*operands)


class MessagePassing(Kernel):
    reducer = SumReducer()
    _guarded: _Guarded | None = None
    _launch: _Launch | None = None

    def __init__(self) -> None:
        super().__init__()
        self._guarded: _Guarded | None = None
        self._launch: _Launch | None = None

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
        return cap.capture(lambda s, d, e, p: _call_region(self.edge, (s, d, e), p), params)

    def _epilogue(self, dst, aggregate, params):
        if type(self).node is MessagePassing.node:
            return aggregate
        return _call_region(self.node, (SimpleNamespace(**dst), aggregate), params)

    def __call__(self, *, graph: Graph, src: Mapping[str, torch.Tensor] | None = None,
                 dst: Mapping[str, torch.Tensor] | None = None,
                 edge: Mapping[str, torch.Tensor] | None = None,
                 ndata: Mapping[str, torch.Tensor] | None = None, **params: Any):
        if not getattr(graph, "_tiga_graph", False):
            raise TypeError("graph must be a tiga.Graph")
        src, dst = _resolve_node_fields(graph, src, dst, ndata)
        edge = {} if edge is None else edge
        guarded = self._guarded
        if guarded is not None:
            result = guarded.try_run(self, graph, src, dst, edge, params)
            if result is not _MISS:
                self._launch = guarded.launch
                self._record_warm(guarded.launch.variant)
                return self._epilogue(dst, result, params)
        return self._epilogue(dst, self._dispatch(graph, src, dst, edge, params), params)

    def _dispatch(self, graph, src, dst, edge, params):
        """The cold path: validate, capture, recognize, run."""
        device = graph.device
        self._validate_fields("src", src, graph.schema.num_src, device)
        self._validate_fields("dst", dst, graph.schema.num_dst, device)
        if edge:
            # Before any launch: a kernel would dereference a host pointer
            # (reference interop/torch/message_passing.py:1633-1634).
            self._validate_fields("edge", edge, graph.num_edges, device)
        prune = (self.reducer.block_prune_threshold
                 if isinstance(self.reducer, OnlineSoftmaxReducer) else None)
        if prune is not None and not graph.is_dense:
            # reference message_passing/core.py:500-505
            raise NotImplementedError(
                "block_prune_threshold is defined for dense relations only; refusing to "
                "run exact softmax on a CSR relation")
        captured = self._captured(params)
        launch = None
        if device.type == "cuda" and captured is not None:
            launch = self._plan_native(captured, graph, src, dst, edge, params)
        elif captured is not None:
            out = self._sparse_mm_sum(captured, graph, src, edge)
            if out is not None:
                self._launch = None
                return out
        if launch is None:
            self._launch = None
            if prune is not None:
                # reference interop/torch/message_passing.py:1611-1616
                raise NotImplementedError(
                    "block_prune_threshold requires the dense attention tile (dot-product "
                    "score, bf16/fp16, head_dim 32, 64 or 128, on the GPU); refusing to silently "
                    "execute exact softmax or materialize the Cartesian relation")
            if config.strict:
                raise RuntimeError(
                    f"{type(self).__qualname__}: no HIP kernel covers this edge function / "
                    "dtype / shape and tiga.config.strict is set")
            self._record_variant(CompiledVariant(
                key=(type(self).__qualname__, "eager", graph.planning_key()),
                backend="torch-eager", provider="torch", pattern="generic",
                lowering="gather -> edge() -> scatter reduce (Torch ops)",
                remarks=("edge function not covered by a HIP kernel",)))
            return _eager.evaluate(self, graph, src, dst, edge, params)
        operands = launch.gather(src, dst, edge, params)
        result = launch.runner(*operands)
        # Described after the first run, which builds the per-graph row plan
        # the description reports.
        launch.variant = launch.describe()
        self._launch = launch
        self._record_variant(launch.variant)
        if launch.guardable:
            guarded = _Guarded(launch, self, operands, params)
            guarded.names = _Guarded._names(src, dst, edge)
            self._guarded = guarded
        return result

    def _sparse_mm_sum(self, captured, graph, src, edge) -> torch.Tensor | None:
        """tg.sum() of edge.w * src.x on host tensors as the reference runs it
        there: one sparse CSR matrix of the weights times the features
        (torch.sparse.mm, reference interop/torch/message_passing.py:
        2903-2925, 3284-3345), same weight/feature conditions; None where the
        reference also falls back to its eager evaluator, and for a weight
        gradient over repeated (row, column) pairs, which the sparse
        matrix's backward cannot return per edge."""
        if not isinstance(self.reducer, SumReducer) or self.reducer.identity_value != 0 or \
                graph.is_varlen or graph.is_dense:
            return None
        pat = cap.recognize_weighted_sum(captured)
        if pat is None or pat.edge_field is None:
            return None
        x, w = src.get(pat.src_field), edge.get(pat.edge_field)
        if x is None or w is None or x.ndim not in (1, 2) or w.dtype != x.dtype or \
                not (w.ndim == 1 or (w.ndim == 2 and tuple(w.shape[1:]) == (1,))):
            return None
        row_ptr, col_idx = graph.resolve_csr()
        if w.requires_grad and torch.is_grad_enabled():
            # The sparse matrix's backward sums the gradients of repeated
            # (row, column) entries into one value, which does not map back
            # onto the edges of a multigraph: those stay eager.
            unique = graph._native_cache.get("unique_pairs")
            if unique is None:
                rows = torch.repeat_interleave(
                    torch.arange(graph.schema.num_dst, device=row_ptr.device),
                    row_ptr[1:] - row_ptr[:-1])
                keys = rows.to(torch.int64) * graph.schema.num_src + col_idx.to(torch.int64)
                unique = bool(torch.unique(keys).numel() == keys.numel())
                graph._native_cache["unique_pairs"] = unique
            if not unique:
                return None
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")   # sparse CSR support is marked beta
            matrix = torch.sparse_csr_tensor(
                row_ptr, col_idx, w.reshape(-1).contiguous(),
                size=(graph.schema.num_dst, graph.schema.num_src))
        out = torch.sparse.mm(matrix, (x[:, None] if x.ndim == 1 else x).contiguous())
        self._record_variant(CompiledVariant(
            key=(type(self).__qualname__, "sparse-mm", graph.planning_key()),
            backend=graph.device.type, provider="torch.sparse.mm", pattern="weighted-sum",
            lowering="dispatch-native-sparse-mm",
            remarks=("host tensors: the reference's native sparse dispatch",)))
        return out[:, 0] if x.ndim == 1 else out

    def prepare(self, *, graph: Graph, src: Mapping[str, torch.Tensor] | None = None,
                dst: Mapping[str, torch.Tensor] | None = None,
                edge: Mapping[str, torch.Tensor] | None = None,
                ndata: Mapping[str, torch.Tensor] | None = None, **params: Any):
        """One ordinary call (validation, capture, planning), then the HIP
        launch it ran frozen as a zero-argument callable: the graph object,
        the bound tensors, shapes and strides are fixed; their contents stay
        live, so in-place updates between launches are seen (reference
        message_passing/core.py:563-590, interop/torch/message_passing.py:
        3827-3879).  The callable carries ``.variant`` and ``.graph``.
        Raises NotImplementedError when the call ran the eager evaluator."""
        src, dst = _resolve_node_fields(graph, src, dst, ndata)
        edge = {} if edge is None else edge
        self(graph=graph, src=src, dst=dst, edge=edge, **params)
        launch = self._launch
        if launch is None or launch.graph is not graph:
            raise NotImplementedError(
                "prepared MessagePassing needs an edge function, dtype and shape that a HIP "
                f"kernel covers; this call ran {self.last_variant.backend} "
                f"({self.last_variant.provider})")
        operands = tuple(launch.gather(src, dst, edge, params))
        runner, epilogue = launch.runner, self._epilogue
        frozen_dst, frozen_params = dict(dst), dict(params)
        bound = launch.bind(*operands) if launch.bind is not None else None
        tensors = tuple(t for t in operands if isinstance(t, torch.Tensor))

        def run():
            if bound is not None and not any(t.requires_grad for t in tensors):
                return epilogue(frozen_dst, bound(), frozen_params)
            return epilogue(frozen_dst, runner(*operands), frozen_params)

        run.variant = launch.variant
        run.graph = graph
        return run

    def reference(self, *, graph: Graph, src: Mapping[str, torch.Tensor] | None = None,
                  dst: Mapping[str, torch.Tensor] | None = None,
                  edge: Mapping[str, torch.Tensor] | None = None,
                  ndata: Mapping[str, torch.Tensor] | None = None, **params: Any):
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
        src, dst = _resolve_node_fields(graph, src, dst, ndata)
        edge = {} if edge is None else edge
        device = graph.device
        self._validate_fields("src", src, graph.schema.num_src, device)
        self._validate_fields("dst", dst, graph.schema.num_dst, device)
        if edge:
            self._validate_fields("edge", edge, graph.num_edges, device)
        aggregate = _eager.evaluate(self, graph, src, dst, edge, params)
        return self._epilogue(dst, aggregate, params)

    # ------------------------------------------------------------------
    def _variant(self, graph, pattern: str, entry_points, lowering, remarks=()):
        """The variant record of a (kernel, pattern) on `graph`, built once and
        kept with the graph's other per-graph structures."""
        plan = graph._native_cache.get(("plan", 512, 512))
        memo = graph._native_cache.setdefault("variants", {})
        memo_key = (type(self).__qualname__, plan is not None, pattern, tuple(entry_points),
                    lowering, tuple(remarks))
        variant = memo.get(memo_key)
        if variant is None:
            extra = () if plan is None else (f"row plan: {plan.counts()}",
                                            *graph._reference_plan_remarks(
                                                type(self).node is not MessagePassing.node))
            variant = CompiledVariant(
                key=(type(self).__qualname__, pattern, graph.planning_key()),
                backend="hip", provider="libtgx_hip.so (gfx950)", pattern=pattern,
                lowering=lowering, entry_points=tuple(entry_points),
                remarks=tuple(remarks) + extra)
            memo[memo_key] = variant
        return variant

    @staticmethod
    def _binding(tensor, params) -> tuple:
        """Binding of a tensor the capture found inside the edge function: the
        parameter it was passed as, else ("fixed", tensor)."""
        for name, value in params.items():
            if value is tensor:
                return ("param", name)
        return ("fixed", tensor)

    def _plan_native(self, captured, graph, src, dst, edge, params) -> _Launch | None:
        if isinstance(self.reducer, SumReducer):
            return self._plan_sum(captured, graph, src, dst, edge)
        if not isinstance(self.reducer, OnlineSoftmaxReducer):
            return None
        if self.reducer.accumulation_dtype not in (None, torch.float32, "float32"):
            return None
        gat = cap.recognize_gat(captured)
        if gat is not None:
            return self._plan_gat(gat, graph, src, dst, params)
        dot = cap.recognize_dot(captured)
        if dot is not None:
            return self._plan_dot(dot, graph, src, dst, edge)
        nn_item = cap.recognize_nn_attention(captured)
        if nn_item is not None:
            return self._plan_nn_attention(nn_item, graph, src, dst, edge)
        raw = cap.recognize_score_softmax(captured)
        if raw is not None:
            return self._plan_score_softmax(raw, graph, src, dst, edge)
        return None

    def _plan_score_softmax(self, raw, graph, src, dst, edge) -> _Launch | None:
        """reducer(role.score [* c], src.value) on the gathered segment softmax
        and the weighted CSR sum (reference: the eager oracle for Torch
        tensors, reducer_oracle.py:60-137; its compiled stable-weighted row
        tile for 1-D f32 fields, message_passing.py:2579-2619).  Scalar
        scores (one lane); fp32, bf16 or fp16 score fields and values, with
        the oracle's arithmetic (scores and sums in fp32, the output in the
        value's type, reducer_oracle.py:22-41, 60-137); an empty row gives
        0, as the reference's Torch path does."""
        from . import _ops

        if graph.is_varlen or graph.is_dense:
            return None
        groups = {"src": src, "dst": dst, "edge": edge}
        rows = {"src": graph.schema.num_src, "dst": graph.schema.num_dst,
                "edge": graph.num_edges}
        table = groups[raw.score_role].get(raw.score_field)
        value = src.get(raw.value_field)
        if table is None or value is None:
            return None
        if table.dtype not in _ops._VALUE_DTYPES or value.dtype not in _ops._VALUE_DTYPES:
            return None
        if tuple(table.shape) not in ((rows[raw.score_role],), (rows[raw.score_role], 1)):
            return None
        _native.lib()
        role, scale = raw.score_role, raw.scale

        def run(table, value):
            return _ops.score_attention(graph, table, role, scale, value)

        describe = lambda: self._variant(
            graph, "score-softmax",
            ("tgx_segment_softmax_sum_fwd", "tgx_segment_softmax_gather_fwd", "tgx_csr_sum_fwd",
             "tgx_segment_softmax_bwd", "tgx_csr_sum_bwd"),
            f"segment softmax of the {role} score field per row and the weighted sum of "
            "src.value in one pass (fp32 values of at most 8 floats, no gradient), else the "
            "softmax weights and a weighted CSR sum; backward through the softmax Jacobian, "
            f"score gradient reduced per {role} row")
        return _Launch(graph, ((role, raw.score_field), ("src", raw.value_field)), run, describe)

    def _plan_sum(self, captured, graph, src, dst, edge) -> _Launch | None:
        from . import _ops

        if self.reducer.identity_value != 0 or graph.is_varlen or graph.is_dense:
            return None
        pat = cap.recognize_weighted_sum(captured)
        if pat is None:
            nn_sum = cap.recognize_nn_sum(captured)
            return None if nn_sum is None else self._plan_nn_sum(nn_sum, graph, src, dst, edge)
        if pat.src_field not in src:
            return None
        x = src[pat.src_field]
        floats = (torch.float32, torch.bfloat16, torch.float16)
        if x.dtype not in floats:
            return None
        out_dtype = x.dtype
        operands = [("src", pat.src_field)]
        if pat.edge_field is not None:
            w = edge.get(pat.edge_field)
            if w is None:
                return None
            E = graph.num_edges
            if tuple(w.shape) not in ((E,), (E, 1)) or w.dtype not in floats:
                return None
            if x.ndim == 1 and w.ndim == 2:
                return None
            # The message w * x has Torch's promoted dtype (bf16 * fp32 is
            # fp32), as in the reference's eager reduce_sum.
            out_dtype = torch.promote_types(x.dtype, w.dtype)
            operands.append(("edge", pat.edge_field))
        _native.lib()

        def run(x, w=None):
            # The kernels read x in the output dtype and fp32 weights; both
            # conversions are differentiable Torch ops (no-ops when the
            # dtypes already match).
            xk = x.to(out_dtype)
            wk = None if w is None else w.to(torch.float32)
            return _ops.csr_sum(xk, wk, graph)

        def bind(x, w=None):
            # Only where the kernel reads the bound tensors themselves (no
            # dtype conversion), so later in-place updates are seen.
            if x.dtype != out_dtype or (w is not None and w.dtype != torch.float32):
                return None
            return _ops.bind_csr_sum(x, w, graph)

        kind = {torch.float32: "fp32", torch.bfloat16: "bf16", torch.float16: "fp16"}[out_dtype]
        describe = lambda: self._variant(
            graph, "weighted-sum", ("tgx_csr_sum_fwd", "tgx_csr_sum_bwd"),
            f"degree-binned rows -> wave gather-FMA ({kind} features, fp32 sums)")
        return _Launch(graph, tuple(operands), run, describe, bind=bind)

    def _plan_gat(self, gat, graph, src, dst, params) -> _Launch | None:
        """The additive score on one feature tensor (src.h is dst.h) or two
        (bipartite src and dst tables of one shape per node), fp32, bf16 or
        fp16 features with fp32 arithmetic, any float a_src / a_dst (read as
        fp32); the reference evaluates it eagerly (reducer_oracle.py:60-137)."""
        from . import _ops

        if graph.is_varlen or graph.is_dense:
            return None
        h = src.get(gat.h_field)
        hd = dst.get(gat.dst_field)
        if h is None or hd is None or h.ndim != 3 or hd.ndim != 3:
            return None
        N, H, D = h.shape
        if hd.shape[1:] != h.shape[1:] or hd.dtype != h.dtype or \
                h.dtype not in _ops._VALUE_DTYPES:
            return None
        if tuple(gat.a_src.shape) not in ((H, D), (1, H, D)) \
                or tuple(gat.a_dst.shape) not in ((H, D), (1, H, D)):
            return None
        if not (gat.a_src.is_floating_point() and gat.a_dst.is_floating_point()):
            return None
        if gat.a_src.device != h.device or gat.a_dst.device != h.device:
            return None
        # Any head count: the kernels run heads in groups of at most 256
        # values per node; the head width is 4 * 2^k values, up to 256.
        if D % 4 or D > 256 or (D // 4) & (D // 4 - 1):
            return None
        _native.lib()
        slope = gat.slope

        def run(h, h_dst, a_src, a_dst):
            # One tensor object in both roles is a homogeneous relation; the
            # kernels read fp32 attention vectors (a no-op for fp32).
            return _ops.GatFunction.apply(h, None if h_dst is h else h_dst,
                                          a_src.to(torch.float32), a_dst.to(torch.float32),
                                          slope, graph)

        kind = {torch.float32: "fp32", torch.bfloat16: "bf16", torch.float16: "fp16"}[h.dtype]
        roles = "one feature table" if hd is h else "source and destination tables"
        describe = lambda: self._variant(
            graph, "gat-additive", ("tgx_gat_fwd", "tgx_gat_bwd"),
            f"{kind} {roles}, online softmax per (row, head), logsumexp and the positive-"
            "branch rows saved; backward recomputes alpha over the transposed CSR and "
            "forms the destination terms per node")
        operands = (("src", gat.h_field), ("dst", gat.dst_field),
                    self._binding(gat.a_src, params), self._binding(gat.a_dst, params))
        return _Launch(graph, operands, run, describe)

    @staticmethod
    def _nn_fields(inputs, graph, src, dst, edge):
        """(widths, roles) of an edge network's input fields if every one is a
        fp32 [rows] or [rows, k] tensor of its role, else None."""
        groups = {"src": src, "dst": dst, "edge": edge}
        rows = {"src": graph.schema.num_src, "dst": graph.schema.num_dst,
                "edge": graph.num_edges}
        widths, roles = [], []
        for role, name in inputs:
            t = groups[role].get(name)
            if t is None or t.dtype != torch.float32 or t.ndim not in (1, 2) or \
                    t.shape[0] != rows[role]:
                return None
            widths.append(1 if t.ndim == 1 else t.shape[1])
            roles.append(role)
        if len(widths) > 4:
            return None
        return widths, tuple(roles)

    @staticmethod
    def _nn_params_ok(layer, device) -> bool:
        """A layer's Linear and LayerNorm parameters are fp32 on `device`."""
        params = [layer.linear.weight, layer.linear.bias]
        if layer.norm is not None:
            params += [layer.norm.weight, layer.norm.bias]
        return all(p is None or (p.dtype == torch.float32 and p.device == device)
                   for p in params)

    @staticmethod
    def _scaled_chain(chain, out_scale):
        """The chain with a scalar applied to its output folded into its last
        layer."""
        if out_scale == 1.0:
            return chain
        import dataclasses

        last = chain[-1]
        return (*chain[:-1], dataclasses.replace(last, scale=last.scale * out_scale,
                                                 shift=last.shift * out_scale))

    def _plan_nn_sum(self, item, graph, src, dst, edge) -> _Launch | None:
        """tg.sum() over a tg.nn.trace message (reference edge-NN tile,
        interop/torch/message_passing.py:2134-2300; fp32 fields): the layers
        before the last per edge on the edge MLP kernels, summed per row, the
        last layer once per row."""
        from . import _ops

        got = self._nn_fields(item.inputs, graph, src, dst, edge)
        if got is None:
            return None
        widths, roles = got
        chain = item.module.chain(vector=True)
        if sum(widths) != chain[0].linear.in_features:
            return None     # the eager evaluator raises the network's own shape error
        if _ops._padded_width(chain, sum(widths), vector=True) > 32:
            return None
        device = graph.device
        for layer in chain:
            if not self._nn_params_ok(layer, device):
                return None
        _native.lib()
        out_scale = item.out_scale

        def run(module, *fields):
            return _ops.nn_message_sum(graph, self._scaled_chain(module.chain(vector=True),
                                                                 out_scale), roles,
                                       [f if f.ndim == 2 else f.unsqueeze(-1) for f in fields])

        layer_widths = "-".join(str(l.linear.in_features) for l in chain)
        describe = lambda: self._variant(
            graph, "edge-network-sum",
            ("tgx_edge_mlp_hidden", "tgx_csr_sum_fwd", "tgx_edge_mlp_backward_seeded",
             "tgx_csr_sum_bwd"),
            f"edge network {layer_widths}-{chain[-1].linear.out_features}: layers before the "
            "last evaluated per edge (one edge per lane), summed per row by the CSR sum, the "
            "last Linear applied once per row; backward seeds the per-edge replay with the "
            "last layer's input gradient gathered per row")
        return _Launch(graph, (("fixed", item.module), *item.inputs), run, describe)

    def _plan_nn_attention(self, item, graph, src, dst, edge) -> _Launch | None:
        """tg.nn.trace-scored attention on the edge MLP kernels (reference
        interop/torch/message_passing.py:2372-2577, envelope: fp32, CSR
        relation, one score per edge, one gathered value field)."""
        from . import _ops

        if graph.is_varlen or graph.is_dense:
            return None
        groups = {"src": src, "dst": dst, "edge": edge}
        rows = {"src": graph.schema.num_src, "dst": graph.schema.num_dst,
                "edge": graph.num_edges}
        widths, roles = [], []
        for role, name in item.inputs:
            t = groups[role].get(name)
            if t is None or t.dtype != torch.float32 or t.ndim not in (1, 2) or \
                    t.shape[0] != rows[role]:
                return None
            widths.append(1 if t.ndim == 1 else t.shape[1])
            roles.append(role)
        if len(widths) > 4 or sum(widths) > 64:
            return None
        chain = item.module.chain()
        if sum(widths) != chain[0].linear.in_features:
            # The eager evaluator raises the network's own shape error.
            return None
        value = src.get(item.value_field)
        if value is None or value.dtype != torch.float32:
            return None
        for layer in chain:
            if not self._nn_params_ok(layer, value.device):
                return None
        if any(l.norm is not None for l in chain) and _ops._padded_width(chain, sum(widths)) > 32:
            return None     # LayerNorm kernels cover padded widths up to 32
        _native.lib()
        roles = tuple(roles)

        out_scale = item.out_scale

        def run(module, value, *fields):
            return _ops.nn_attention(graph, self._scaled_chain(module.chain(), out_scale), roles,
                                     [f if f.ndim == 2 else f.unsqueeze(-1) for f in fields],
                                     value)

        layer_widths = "-".join(str(l.linear.in_features) for l in chain) + "-1"
        describe = lambda: self._variant(
            graph, "nn-attention",
            ("tgx_edge_mlp_scores", "tgx_segment_softmax_sum_fwd", "tgx_segment_softmax_fwd",
             "tgx_csr_sum_fwd", "tgx_edge_mlp_attention_backward", "tgx_csr_sum_bwd"),
            f"edge-parallel score network {layer_widths} (one edge per lane, uniform "
            "weights), segment softmax per row with the value sum in the same pass (value "
            "rows of at most 8 floats; else a weighted CSR sum); only each "
            "row's logsumexp and output are kept; backward replays the network per edge, "
            "recomputes the weights and the softmax Jacobian in the same kernel, on-chip "
            "weight-gradient sums, value gradient over the transposed CSR (a value that is "
            "also a source field of the score gets its edge term in the same kernel and "
            "one transposed reduction)")
        operands = (("fixed", item.module), ("src", item.value_field), *item.inputs)
        return _Launch(graph, operands, run, describe)

    def _plan_dot(self, dot, graph, src, dst, edge) -> _Launch | None:
        from . import _ops

        q, k, v = dst.get(dot.q_field), src.get(dot.k_field), src.get(dot.v_field)
        if q is None or k is None or v is None:
            return None
        if q.ndim != 3 or k.shape[1:] != q.shape[1:] or v.shape[1:] != q.shape[1:]:
            return None
        if graph.is_varlen or graph.is_dense:
            return self._plan_block_attention(dot, graph, q, k, v)
        _, H, D = q.shape
        # bf16, fp16 or fp32 q, k, v of one type: fp32 scores, softmax and
        # sums, the output in that type (the reference's eager path
        # accumulates 16-bit scores in fp32 and casts back to the value's
        # dtype, reducer_oracle.py:22-41, 137).
        if not (q.dtype == k.dtype == v.dtype) or q.dtype not in _ops._VALUE_DTYPES:
            return None
        # Any head count: the kernels run heads in groups of at most 512
        # values per node; the head width is 8 * 2^k values, up to 512.
        if D % 8 or D > 512 or (D // 8) & (D // 8 - 1):
            return None
        operands = [("dst", dot.q_field), ("src", dot.k_field), ("src", dot.v_field)]
        if dot.bias_field is not None:
            bias = edge.get(dot.bias_field)
            if bias is None or bias.dtype not in _ops._VALUE_DTYPES:
                return None
            if tuple(bias.shape) not in ((graph.num_edges, H), (graph.num_edges, H, 1)):
                return None
            operands.append(("edge", dot.bias_field))
        _native.lib()
        scale, E = dot.scale, graph.num_edges

        def run(q, k, v, bias=None):
            if bias is not None:
                # The kernels read an fp32 bias (a differentiable no-op for
                # fp32; a 16-bit bias widens exactly).
                bias = bias.reshape(E, H).to(torch.float32)
            return _ops.DotAttnFunction.apply(q, k, v, bias, scale, graph)

        kind = {torch.float32: "fp32", torch.bfloat16: "bf16", torch.float16: "fp16"}[q.dtype]
        describe = lambda: self._variant(
            graph, "dot-product", ("tgx_dot_attn_fwd", "tgx_dot_attn_bwd"),
            f"{kind} gathers, fp32 online softmax per (row, head); hub rows split and merged; "
            "backward over the transposed CSR (dk, dv, each edge's ds kept) and the CSR "
            "(dq, dbias from the kept ds)")
        return _Launch(graph, tuple(operands), run, describe)

    def _plan_block_attention(self, dot, graph, q, k, v) -> _Launch | None:
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
        if D not in (32, 64, 128):
            return None
        if q.shape[0] != graph.schema.num_dst or k.shape[0] != graph.schema.num_src or \
                v.shape[0] != graph.schema.num_src:
            return None
        prune = self.reducer.block_prune_threshold
        _native.lib()
        scale = dot.scale

        def run(q, k, v):
            if prune is not None and torch.is_grad_enabled() and \
                    any(t.requires_grad for t in (q, k, v)):
                raise NotImplementedError(
                    "block_prune_threshold is a forward-only approximation (no gradient); run "
                    "it under torch.no_grad() or drop the threshold for exact softmax")
            return _ops.BlockAttentionFunction.apply(q, k, v, scale, float(prune or 0.0), graph)

        relation = "cu_seqlens" if graph.is_varlen else graph.schema.origin
        causal = graph._attn_blocks()[2]
        describe = lambda: self._variant(
            graph, "block-attention", ("tgx_attn_fwd", "tgx_attn_bwd"),
            f"MFMA 16x16x32 {str(q.dtype).split('.')[-1]} flash tiles over the implicit "
            f"{relation} relation ({'causal' if causal else 'all pairs'}); XCD-grouped "
            "tasks; atomic-free dK/dV and dQ passes",
            remarks=(("block-pruned tile admission (approximate)",) if prune else ()))
        operands = (("dst", dot.q_field), ("src", dot.k_field), ("src", dot.v_field))
        return _Launch(graph, operands, run, describe)


__all__ = ["MessagePassing", "config"]

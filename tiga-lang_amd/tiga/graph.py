"""Destination-row CSR relation on Torch tensors.

Public constructors and queries mirror the reference Torch graph
(python/tiga/interop/torch/graph.py): ``from_csr`` 153-190 (validation
595-617), ``from_coo`` 193-231, ``regular`` 233-257, ``cu_seqlens`` 260-294,
``cat`` 297-340, ``transpose`` 675-685, ``destination_index`` 1212-1222,
degree statistics and ``planning_key`` 1224-1351.

On top of that, a graph caches the device-side structures the HIP kernels
need, built once per graph by the native planner (one host sync each):
the degree-binned row plan of the CSR, and the stable transpose
(row_ptr_t, col_t, perm) with its own row plan.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Literal

import torch

from . import _native

_INDEX_DTYPES = (torch.int32, torch.int64)

# Rows with at most WAVE_MAX edges run whole on one wavefront; longer rows are
# split into CHUNK_EDGES-edge chunks whose partial states are merged.
WAVE_MAX = 512
CHUNK_EDGES = 512


@dataclass(frozen=True)
class GraphSchema:
    """What a relation is, independent of its index values (reference
    interop/torch/graph.py:51-70); every relation here is static (built
    once, not regenerated per call like the reference's radius and kNN
    relations)."""

    num_src: int
    num_dst: int
    origin: str
    realization: str
    index_dtype: torch.dtype
    sorted_by_dst: bool = True
    lifecycle: str = "static"

    def specialization_key(self) -> tuple[object, ...]:
        return (self.num_src, self.num_dst, self.origin, self.lifecycle, self.realization,
                str(self.index_dtype), self.sorted_by_dst)


class RowPlanHandle:
    """A ``tgx_row_plan`` plus the device tensors it points into."""

    def __init__(self, plan: _native.RowPlan, rows: torch.Tensor, chunk_offsets: torch.Tensor):
        self.plan = plan
        self.rows = rows
        self.chunk_offsets = chunk_offsets

    @property
    def ref(self):
        return ctypes.byref(self.plan)

    def counts(self) -> dict[str, int]:
        p = self.plan
        return {"empty": p.n_empty, "wave": p.n_wave, "split": p.n_split,
                "chunks": p.n_chunks, "wave_max": p.wave_max,
                "chunk_edges": p.chunk_edges}


class Transposed:
    """Source-row CSR of a graph: row_ptr_t [num_src+1], col_t [E], perm [E]
    (original edge of each transposed edge) and inv_perm [E] (its inverse)."""

    def __init__(self, row_ptr_t, col_t, perm, inv_perm, plan):
        self.row_ptr_t = row_ptr_t
        self.col_t = col_t
        self.perm = perm
        self.inv_perm = inv_perm
        self.plan = plan


def build_row_plan(row_ptr: torch.Tensor, n_rows: int, *, wave_max: int = WAVE_MAX,
                   chunk_edges: int = CHUNK_EDGES) -> RowPlanHandle:
    """Run the native degree-bin partition (empty | wave | split) on row_ptr."""
    device = row_ptr.device
    bits = _native.idx_bits(row_ptr)
    stream = _native.stream_of(row_ptr)
    rows = torch.empty(max(n_rows, 1), dtype=torch.int32, device=device)
    ws_bytes = ctypes.c_size_t()
    _native.call("tgx_plan_degree_bins_workspace", n_rows, 3, ctypes.byref(ws_bytes))
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=device)
    bounds = (ctypes.c_int64 * 3)(0, wave_max, 1 << 62)
    offsets = (ctypes.c_int64 * 4)()
    _native.call("tgx_plan_degree_bins", _native.ptr(row_ptr), bits, n_rows, bounds, 3,
                 rows.data_ptr(), offsets, ws.data_ptr(), ws_bytes.value, stream)
    n_empty = offsets[1] - offsets[0]
    n_wave = offsets[2] - offsets[1]
    n_split = offsets[3] - offsets[2]
    chunk_offsets = torch.zeros(n_split + 1, dtype=torch.int32, device=device)
    n_chunks = ctypes.c_int64(0)
    if n_split:
        _native.call("tgx_plan_split_chunks", _native.ptr(row_ptr), bits,
                     rows.data_ptr() + 4 * offsets[2], n_split, chunk_edges,
                     chunk_offsets.data_ptr(), ctypes.byref(n_chunks), stream)
    plan = _native.RowPlan(n_rows, n_empty, n_wave, n_split, n_chunks.value, wave_max,
                           chunk_edges, rows.data_ptr(), chunk_offsets.data_ptr())
    return RowPlanHandle(plan, rows, chunk_offsets)


def build_transpose(row_ptr: torch.Tensor, col_idx: torch.Tensor, num_dst: int,
                    num_src: int):
    """Stable transpose on the device: (row_ptr_t, col_t, perm, inv_perm)."""
    device = row_ptr.device
    E = col_idx.numel()
    row_ptr_t = torch.empty(num_src + 1, dtype=torch.int32, device=device)
    col_t = torch.empty(max(E, 1), dtype=torch.int32, device=device)
    perm = torch.empty(max(E, 1), dtype=torch.int32, device=device)
    inv_perm = torch.empty(max(E, 1), dtype=torch.int32, device=device)
    ws_bytes = ctypes.c_size_t()
    _native.call("tgx_csr_transpose_workspace", num_dst, num_src, E, ctypes.byref(ws_bytes))
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=device)
    _native.call("tgx_csr_transpose", row_ptr.data_ptr(), col_idx.data_ptr(),
                 _native.idx_bits(row_ptr), num_dst, num_src, E, row_ptr_t.data_ptr(),
                 col_t.data_ptr(), perm.data_ptr(), inv_perm.data_ptr(), ws.data_ptr(),
                 ws_bytes.value, _native.stream_of(row_ptr))
    return row_ptr_t, col_t[:E], perm[:E], inv_perm[:E]


def _native_builder_ok(t: torch.Tensor, n_edges: int, n_rows: int) -> bool:
    """Device builders run for GPU tensors below 2^31 edges and rows; other
    cases (CPU tensors, larger graphs) use Torch ops, as the reference does."""
    return t.is_cuda and n_edges < 2**31 and n_rows < 2**31 - 1


def build_coo_csr(src: torch.Tensor, dst: torch.Tensor, num_dst: int):
    """(row_ptr in dst's dtype, col_idx in src's dtype) for ``from_coo``:
    stable sort of the edges by destination (reference graph.py:219-227)."""
    device = dst.device
    E = src.numel()
    row_ptr = torch.empty(num_dst + 1, dtype=dst.dtype, device=device)
    col = torch.empty(max(E, 1), dtype=src.dtype, device=device)
    ws_bytes = ctypes.c_size_t()
    _native.call("tgx_coo_to_csr_workspace", 0, num_dst, E, ctypes.byref(ws_bytes))
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=device)
    _native.call("tgx_coo_to_csr", _native.ptr(src), _native.idx_bits(src), _native.ptr(dst),
                 _native.idx_bits(dst), 0, num_dst, E, row_ptr.data_ptr(), col.data_ptr(),
                 None, ws.data_ptr(), ws_bytes.value, _native.stream_of(dst))
    return row_ptr, col[:E]


def build_varlen_csr(cu_seqlens: torch.Tensor, causal: bool, total: int, n_edges: int):
    """Materialized block-diagonal varlen CSR (reference graph.py:276-294)."""
    device, dtype = cu_seqlens.device, cu_seqlens.dtype
    n_seq = cu_seqlens.numel() - 1
    row_ptr = torch.empty(total + 1, dtype=dtype, device=device)
    col = torch.empty(max(n_edges, 1), dtype=dtype, device=device)
    ws_bytes = ctypes.c_size_t()
    _native.call("tgx_varlen_csr_workspace", n_seq, ctypes.byref(ws_bytes))
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=device)
    _native.call("tgx_varlen_csr", _native.ptr(cu_seqlens), _native.idx_bits(cu_seqlens),
                 n_seq, total, n_edges, int(causal), row_ptr.data_ptr(), col.data_ptr(),
                 ws.data_ptr(), ws_bytes.value, _native.stream_of(cu_seqlens))
    return row_ptr, col[:n_edges]


_PLAN_NAMES = ("row-neighbor-tile", "degree-bucketing-required", "high-degree-tail-split",
               "provider-deferred-high-degree", "bounded-row-preferred",
               "high-degree-tail-chunked", "high-degree-tail-split-rows")
_MAPPING_NAMES = ("worklist", "direct-filter", "worklist-chunked")


def reference_plan(n_rows: int, max_degree: int, degree_sum: int, histogram=None,
                   has_node_epilogue: bool = False) -> dict:
    """The reference's load-balance decision for a CSR with these degree
    statistics (native ``tgx_plan_reference_buckets``)."""
    hist = None
    if histogram is not None:
        hist = (ctypes.c_int64 * len(histogram))(*histogram)
    code, util = ctypes.c_int(), ctypes.c_int64()
    bounds = (ctypes.c_int64 * 64)()
    mapping = (ctypes.c_int * 64)()
    rows_in = (ctypes.c_int64 * 64)()
    n, per_row, active = ctypes.c_int(), ctypes.c_int64(), ctypes.c_int64()
    _native.call("tgx_plan_reference_buckets", n_rows, max_degree, degree_sum, hist,
                 int(bool(has_node_epilogue)), ctypes.byref(code), ctypes.byref(util), bounds,
                 mapping, rows_in, ctypes.byref(n), ctypes.byref(per_row), ctypes.byref(active))
    k = n.value
    plan = {"plan": _PLAN_NAMES[code.value], "utilization_milli": util.value,
            "bounds": list(bounds[:k]), "mapping": [_MAPPING_NAMES[m] for m in mapping[:k]],
            "rows_in_bucket": list(rows_in[:k]), "partials_per_row": per_row.value,
            "active_rows": active.value}
    # Launch sizing of the reference's bucket tasks (Translate.cpp:4728-4830):
    # rows per program min(16, 256 / nextpow2(bound)); a direct-filter bucket
    # scans every row, the others their worklist.
    grid = []
    for bound, how, rows in zip(plan["bounds"], plan["mapping"], plan["rows_in_bucket"]):
        per_program = max(1, min(16, 256 // (1 << max(0, (bound - 1).bit_length()))))
        scanned = n_rows if how == "direct-filter" else rows
        grid.append(-(-scanned // per_program))
    plan["grid_x"] = grid
    plan["worklist_elements"] = n_rows + 2 * k + 1
    plan["partial_bytes"] = 4 * plan["partials_per_row"] * plan["active_rows"]
    return plan


def describe_reference_plan(plan: dict) -> str:
    text = f"reference planner: {plan['plan']}"
    if plan["utilization_milli"] >= 0:
        text += f", padding utilization {plan['utilization_milli']}/1000"
    if plan["bounds"]:
        buckets = ", ".join(f"<={b} {m} ({r} rows)" for b, m, r in
                            zip(plan["bounds"], plan["mapping"], plan["rows_in_bucket"]))
        text += f"; buckets {buckets}"
    if plan["partials_per_row"]:
        text += (f"; row split {plan['partials_per_row']} partials x "
                 f"{plan['active_rows']} rows")
    return text


class Graph:
    """Torch realization of a Tiga relation (destination-row CSR)."""

    _tiga_graph = True

    def __init__(self, schema: GraphSchema, *, row_ptr=None, col_idx=None,
                 cu_seqlens=None, causal=True, device=None):
        self._schema = schema
        self._row_ptr = row_ptr
        self._col_idx = col_idx
        self._cu_seqlens = cu_seqlens
        self._causal = causal
        # Implicit dense relations: None (every pair) or "lower_inclusive".
        self._dense_boundary = None
        self._device = torch.device(device) if device is not None else None
        self._destination_index_cache = None
        self._degree_bounds_cache = None
        self._native_cache: dict[object, object] = {}

    # ---- constructors ----------------------------------------------------
    @staticmethod
    def _validate_index_tensor(name: str, value: torch.Tensor) -> None:
        if not isinstance(value, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if value.ndim != 1:
            raise ValueError(f"{name} must be one-dimensional")
        if value.dtype not in _INDEX_DTYPES:
            raise TypeError(f"{name} must have int32 or int64 dtype")

    @staticmethod
    def _validate_csr_values(row_ptr, col_idx, num_src: int) -> None:
        if int(row_ptr[0].item()) != 0:
            raise ValueError("row_ptr[0] must be zero")
        if int(row_ptr[-1].item()) != col_idx.numel():
            raise ValueError("row_ptr[-1] must equal the number of edges")
        if bool(torch.any(row_ptr[1:] < row_ptr[:-1]).item()):
            raise ValueError("row_ptr must be monotonic")
        if col_idx.numel():
            lo = int(col_idx.min().item())
            hi = int(col_idx.max().item())
            if lo < 0 or hi >= num_src:
                raise ValueError("col_idx contains an out-of-range source index")

    @classmethod
    def from_csr(cls, row_ptr: torch.Tensor, col_idx: torch.Tensor, *,
                 num_src: int | None = None, sorted_by_dst: bool = True,
                 validate: Literal["basic", "full"] = "basic") -> "Graph":
        cls._validate_index_tensor("row_ptr", row_ptr)
        cls._validate_index_tensor("col_idx", col_idx)
        if row_ptr.device != col_idx.device:
            raise ValueError("row_ptr and col_idx must be on the same device")
        if row_ptr.numel() == 0:
            raise ValueError("row_ptr must contain at least the initial zero")
        num_dst = row_ptr.numel() - 1
        if num_src is None:
            num_src = num_dst if col_idx.numel() == 0 else int(col_idx.max().item()) + 1
        if num_src < 0:
            raise ValueError("num_src must be non-negative")
        if validate == "full":
            cls._validate_csr_values(row_ptr, col_idx, num_src)
        elif validate != "basic":
            raise ValueError("validate must be 'basic' or 'full'")
        schema = GraphSchema(num_src=num_src, num_dst=num_dst, origin="explicit",
                             realization="materialized_csr", index_dtype=col_idx.dtype,
                             sorted_by_dst=sorted_by_dst)
        return cls(schema, row_ptr=row_ptr, col_idx=col_idx)

    @classmethod
    def from_coo(cls, src: torch.Tensor, dst: torch.Tensor, *, num_src: int | None = None,
                 num_dst: int | None = None) -> "Graph":
        cls._validate_index_tensor("src", src)
        cls._validate_index_tensor("dst", dst)
        if src.shape != dst.shape:
            raise ValueError("src and dst must have identical shapes")
        if src.device != dst.device:
            raise ValueError("src and dst must be on the same device")
        if num_src is None:
            num_src = int(src.max().item()) + 1 if src.numel() else 0
        if num_dst is None:
            num_dst = int(dst.max().item()) + 1 if dst.numel() else 0
        if not isinstance(num_src, int) or num_src < 0:
            raise ValueError("num_src must be a non-negative integer")
        if not isinstance(num_dst, int) or num_dst < 0:
            raise ValueError("num_dst must be a non-negative integer")
        if src.numel():
            if int(src.min().item()) < 0 or int(src.max().item()) >= num_src:
                raise ValueError("src contains an out-of-range source index")
            if int(dst.min().item()) < 0 or int(dst.max().item()) >= num_dst:
                raise ValueError("dst contains an out-of-range destination index")
        if _native_builder_ok(dst, src.numel(), num_dst):
            row_ptr, col_idx = build_coo_csr(src, dst, num_dst)
        else:
            order = torch.argsort(dst, stable=True)
            col_idx = src[order]
            counts = torch.bincount(dst.to(torch.int64), minlength=num_dst)
            row_ptr = torch.empty(num_dst + 1, device=dst.device, dtype=dst.dtype)
            row_ptr[0] = 0
            torch.cumsum(counts, dim=0, out=row_ptr[1:])
        return cls.from_csr(row_ptr, col_idx, num_src=num_src, validate="basic")

    @classmethod
    def regular(cls, num_nodes: int, degree: int, *, device="cpu") -> "Graph":
        if not isinstance(num_nodes, int) or num_nodes < 1:
            raise ValueError("num_nodes must be a positive integer")
        if not isinstance(degree, int) or degree < 0:
            raise ValueError("degree must be a non-negative integer")
        row_ptr = torch.arange(num_nodes + 1, device=device, dtype=torch.int64) * degree
        col_idx = torch.arange(num_nodes * degree, device=device, dtype=torch.int64) % num_nodes
        return cls.from_csr(row_ptr, col_idx, num_src=num_nodes)

    @classmethod
    def cu_seqlens(cls, cu_seqlens: torch.Tensor, *, causal: bool = True) -> "Graph":
        """Block-diagonal packed varlen relation; kept implicit until needed.

        Row i of sequence k relates to sources [s_k, i] (causal) or
        [s_k, s_{k+1}) — the reference materializes this CSR at construction;
        here it is materialized only if an edge function needs the CSR.
        """
        cls._validate_index_tensor("cu_seqlens", cu_seqlens)
        if not isinstance(causal, bool):
            raise TypeError("causal must be bool")
        if cu_seqlens.numel() == 0 or int(cu_seqlens[0].item()) != 0:
            raise ValueError("cu_seqlens must start at zero")
        if bool(torch.any(cu_seqlens[1:] < cu_seqlens[:-1]).item()):
            raise ValueError("cu_seqlens must be monotonic")
        total = int(cu_seqlens[-1].item())
        schema = GraphSchema(num_src=total, num_dst=total, origin="cu_seqlens",
                             realization="implicit_varlen", index_dtype=cu_seqlens.dtype)
        return cls(schema, cu_seqlens=cu_seqlens, causal=causal, device=cu_seqlens.device)

    @classmethod
    def dense(cls, num_src: int, num_dst: int | None = None, *, device=None,
              index_dtype: torch.dtype = torch.int64) -> "Graph":
        """Implicit Cartesian relation: every (dst, src) pair, no adjacency
        stored (reference graph.py:535-574).  Dot-product attention over it
        runs in MFMA tiles; other edge functions materialize the CSR."""
        if not isinstance(num_src, int) or num_src < 0:
            raise ValueError("num_src must be a non-negative integer")
        if num_dst is None:
            num_dst = num_src
        if not isinstance(num_dst, int) or num_dst < 0:
            raise ValueError("num_dst must be a non-negative integer")
        if index_dtype not in _INDEX_DTYPES:
            raise TypeError("index_dtype must be torch.int32 or torch.int64")
        resolved = torch.device("cpu" if device is None else device)
        if resolved.type == "cuda" and resolved.index is None and torch.cuda.is_available():
            resolved = torch.device("cuda", torch.cuda.current_device())
        schema = GraphSchema(num_src=num_src, num_dst=num_dst, origin="cartesian",
                             realization="implicit_dense", index_dtype=index_dtype)
        return cls(schema, device=resolved)

    @classmethod
    def triangular(cls, num_entities: int, *, device=None,
                   index_dtype: torch.dtype = torch.int64) -> "Graph":
        """Lower-inclusive dense relation: row i relates to sources 0..i
        (reference graph.py:576-592)."""
        graph = cls.dense(num_entities, num_entities, device=device, index_dtype=index_dtype)
        graph._schema = GraphSchema(num_src=num_entities, num_dst=num_entities,
                                    origin="lower_triangular", realization="implicit_dense",
                                    index_dtype=index_dtype)
        graph._dense_boundary = "lower_inclusive"
        return graph

    @classmethod
    def cat(cls, graphs) -> "Graph":
        blocks = list(graphs)
        if not blocks:
            raise ValueError("graphs must be a non-empty sequence")
        for block in blocks:
            if not isinstance(block, Graph):
                raise TypeError("graphs must contain only Graph instances")
        device = blocks[0].device
        if any(str(block.device) != str(device) for block in blocks):
            raise ValueError("all blocks must share a device")
        # Causal (or all-pairs) square blocks stay implicit: their cat is one
        # cu_seqlens relation.
        for causal in (True, False):
            if all(b._square_blocks(causal) is not None for b in blocks):
                parts = [torch.zeros(1, dtype=torch.int64, device=device)]
                offset = 0
                for b in blocks:
                    cu = b._square_blocks(causal)
                    parts.append(cu[1:] + offset)
                    offset += int(cu[-1].item())
                return cls.cu_seqlens(torch.cat(parts), causal=causal)
        # Materialized blocks: every block's CSR shifted by the edges and
        # sources of the blocks before it; the block edge counts come back in
        # one host transfer.
        dtype = (torch.int64 if any(b.schema.index_dtype == torch.int64 for b in blocks)
                 else torch.int32)
        csrs = [b.resolve_csr() for b in blocks]
        ends = torch.stack([rp[-1].to(torch.int64) for rp, _ in csrs]).cpu().tolist()
        edge_base = [0]
        src_base = [0]
        for b, n in zip(blocks, ends):
            edge_base.append(edge_base[-1] + int(n))
            src_base.append(src_base[-1] + b.schema.num_src)
        row_ptr = torch.cat([torch.zeros(1, dtype=dtype, device=device)] +
                            [rp[1:].to(dtype) + eb for (rp, _), eb in zip(csrs, edge_base)])
        col_idx = torch.cat([ci.to(dtype) + sb for (_, ci), sb in zip(csrs, src_base)])
        return cls.from_csr(row_ptr, col_idx, num_src=src_base[-1])

    # ---- queries ---------------------------------------------------------
    @property
    def schema(self) -> GraphSchema:
        return self._schema

    @property
    def device(self) -> torch.device:
        if self._col_idx is not None:
            return self._col_idx.device
        if self._cu_seqlens is not None:
            return self._cu_seqlens.device
        return self._device or torch.device("cpu")

    @property
    def is_varlen(self) -> bool:
        return self._schema.realization == "implicit_varlen"

    @property
    def is_dense(self) -> bool:
        return self._schema.realization == "implicit_dense"

    def _square_blocks(self, causal: bool):
        """cu_seqlens (int64, on the graph's device) of an implicit relation
        made of square blocks with the given boundary, else None."""
        if self._row_ptr is not None:
            return None
        if self.is_varlen and self._causal == causal:
            return self._cu_seqlens.to(torch.int64)
        if self.is_dense and (self._dense_boundary == "lower_inclusive") == causal and \
                self._schema.num_src == self._schema.num_dst:
            return torch.tensor([0, self._schema.num_dst], dtype=torch.int64, device=self.device)
        return None

    @property
    def num_edges(self) -> int:
        if self.is_dense and self._row_ptr is None:
            n = self._schema.num_dst
            if self._dense_boundary == "lower_inclusive":
                return n * (n + 1) // 2
            return self._schema.num_src * n
        if self.is_varlen and self._row_ptr is None:
            lengths = (self._cu_seqlens[1:] - self._cu_seqlens[:-1]).to(torch.int64)
            if self._causal:
                return int((lengths * (lengths + 1) // 2).sum().item())
            return int((lengths * lengths).sum().item())
        return self._col_idx.numel()

    def resolve_csr(self) -> tuple[torch.Tensor, torch.Tensor]:
        if self._row_ptr is None and self.is_dense:
            # Only an edge function no tile covers gets here (eager path).
            dtype, dev = self._schema.index_dtype, self.device
            n_dst, n_src = self._schema.num_dst, self._schema.num_src
            if self._dense_boundary == "lower_inclusive":
                cu = torch.tensor([0, n_dst], dtype=dtype, device=dev)
                if _native_builder_ok(cu, self.num_edges, n_dst):
                    self._row_ptr, self._col_idx = build_varlen_csr(cu, True, n_dst,
                                                                    self.num_edges)
                else:
                    self._row_ptr, self._col_idx = _varlen_csr(cu, True)
            else:
                self._row_ptr = torch.arange(n_dst + 1, dtype=dtype, device=dev) * n_src
                self._col_idx = torch.arange(n_src, dtype=dtype, device=dev).repeat(n_dst)
            return self._row_ptr, self._col_idx
        if self._row_ptr is None and self.is_varlen:
            total = self._schema.num_dst
            n_edges = self.num_edges
            n_seq = self._cu_seqlens.numel() - 1
            if _native_builder_ok(self._cu_seqlens, n_edges, max(total, n_seq)):
                self._row_ptr, self._col_idx = build_varlen_csr(
                    self._cu_seqlens, self._causal, total, n_edges)
            else:
                self._row_ptr, self._col_idx = _varlen_csr(self._cu_seqlens, self._causal)
        return self._row_ptr, self._col_idx

    def transpose(self) -> "Graph":
        row_ptr, col_idx = self.resolve_csr()
        destination = self.destination_index(row_ptr)
        return type(self).from_coo(destination.to(col_idx.dtype), col_idx,
                                   num_src=self._schema.num_dst, num_dst=self._schema.num_src)

    def destination_index(self, row_ptr: torch.Tensor | None = None) -> torch.Tensor:
        if row_ptr is None and self._destination_index_cache is not None:
            return self._destination_index_cache
        if row_ptr is None:
            row_ptr, _ = self.resolve_csr()
        native = False
        if row_ptr.is_cuda and row_ptr.numel() == self._schema.num_dst + 1 > 1:
            # One sync: the edge count, and whether row_ptr is well formed
            # (starts at 0, non-decreasing) so the kernel's writes stay in
            # [0, row_ptr[-1]).
            stats = torch.stack([row_ptr[-1].to(torch.int64),
                                 (row_ptr[0] == 0).to(torch.int64),
                                 (row_ptr[1:] >= row_ptr[:-1]).all().to(torch.int64)]).cpu()
            n_edges = int(stats[0])
            native = bool(stats[1]) and bool(stats[2]) and _native_builder_ok(
                row_ptr, n_edges, self._schema.num_dst)
        if native:
            dst = torch.empty(n_edges, dtype=torch.int64, device=row_ptr.device)
            _native.call("tgx_destination_index", _native.ptr(row_ptr),
                         _native.idx_bits(row_ptr), self._schema.num_dst, n_edges,
                         _native.ptr(dst), 64, _native.stream_of(row_ptr))
        else:
            degree = row_ptr[1:] - row_ptr[:-1]
            dst = torch.repeat_interleave(
                torch.arange(self._schema.num_dst, device=row_ptr.device), degree)
        if self._row_ptr is row_ptr:
            self._destination_index_cache = dst
        return dst

    def _degree_stats(self) -> tuple[int, int, int]:
        """(min, max, sum) of the destination-row degrees: closed forms for
        implicit relations, else one device reduction and one host transfer,
        cached for the graph (an immutable snapshot)."""
        got = self._degree_bounds_cache
        if got is not None:
            return got
        n_dst, n_src = self._schema.num_dst, self._schema.num_src
        if self.is_dense and self._row_ptr is None:
            if self._dense_boundary == "lower_inclusive":
                got = (1, n_dst, n_dst * (n_dst + 1) // 2) if n_dst else (0, 0, 0)
            else:
                got = (n_src, n_src, n_src * n_dst)
        elif self.is_varlen and self._row_ptr is None:
            lengths = (self._cu_seqlens[1:] - self._cu_seqlens[:-1]).to(torch.int64).cpu()
            lengths = lengths[lengths > 0]
            if lengths.numel() == 0:
                got = (0, 0, 0)
            elif self._causal:
                got = (1, int(lengths.max()), int((lengths * (lengths + 1) // 2).sum()))
            else:
                got = (int(lengths.min()), int(lengths.max()), int((lengths * lengths).sum()))
        elif n_dst == 0:
            got = (0, 0, 0)
        else:
            row_ptr, _ = self.resolve_csr()
            degree = (row_ptr[1:] - row_ptr[:-1]).to(torch.int64)
            got = tuple(int(v) for v in torch.stack(
                (degree.min(), degree.max(), row_ptr[-1].to(torch.int64))).cpu())
        self._degree_bounds_cache = got
        return got

    def degree_bounds(self) -> tuple[int, int]:
        """(minimum, maximum) destination-row degree (reference graph.py:1224-1245;
        the first call may synchronize the device)."""
        return self._degree_stats()[:2]

    def degree_statistics(self) -> tuple[int, int, int]:
        """(minimum, maximum, sum) of the destination-row degrees (reference
        graph.py:1247-1256)."""
        return self._degree_stats()

    def degree_histogram(self) -> tuple[int, ...]:
        """Exact row counts indexed by degree 0..max (reference graph.py:
        1258-1277); limited to a maximum degree of 4096, as there."""
        _, maximum, _ = self._degree_stats()
        if maximum > 4096:
            raise ValueError("exact degree histogram is limited to degree_max <= 4096")
        got = self._native_cache.get("histogram")
        if got is None:
            n_dst = self._schema.num_dst
            if self.is_dense and self._row_ptr is None:
                counts = [0] * (maximum + 1)
                if self._dense_boundary == "lower_inclusive":
                    counts[1:] = [1] * maximum
                else:
                    counts[maximum] = n_dst
            else:
                row_ptr, _ = self.resolve_csr() if not self.is_varlen else (None, None)
                if row_ptr is None:
                    cu = self._cu_seqlens.to(torch.int64).cpu()
                    counts = [0] * (maximum + 1)
                    for length in (cu[1:] - cu[:-1]).tolist():
                        if self._causal:
                            for d in range(1, length + 1):
                                counts[d] += 1
                        else:
                            counts[length] += length
                    counts[0] += n_dst - sum(counts)
                else:
                    degree = (row_ptr[1:] - row_ptr[:-1]).to(torch.int64)
                    counts = torch.bincount(degree, minlength=maximum + 1).cpu().tolist()
            got = tuple(int(c) for c in counts)
            self._native_cache["histogram"] = got
        return got

    def source_index_span_ratio(self, samples: int = 4096) -> float:
        """Locality of the gathers (reference graph.py:1279-1311): the mean
        |source id - destination id| over `samples` evenly spaced edge slots,
        over max(1, num_src, num_dst), clipped to [0, 1]; about 1/3 for random
        numbering, near 0 for index-local graphs.  Planning information only."""
        key = ("span_ratio", samples)
        got = self._native_cache.get(key)
        if got is not None:
            return got
        if self.is_dense and self._row_ptr is None:
            return 1.0 / 3.0
        row_ptr, col_idx = self.resolve_csr()
        E = col_idx.numel()
        if E == 0:
            ratio = 0.0
        else:
            count = min(samples, E)
            step = (E - 1) / (count - 1) if count > 1 else 0.0
            slots = torch.floor(torch.arange(count, dtype=torch.float64) * step)
            slots = slots.clamp_(max=E - 1).to(torch.int64).to(col_idx.device)
            rows = torch.searchsorted(row_ptr[1:].to(torch.int64), slots, right=True)
            span = (col_idx[slots].to(torch.int64) - rows).abs().to(torch.float64).mean()
            scale = max(1, self._schema.num_src, self._schema.num_dst)
            ratio = min(1.0, max(0.0, float(span.cpu()) / scale))
        self._native_cache[key] = ratio
        return ratio

    def planning_key(self) -> tuple[object, ...]:
        """What a specialization depends on (reference graph.py:1317-1351):
        the relation's kind and sizes, index dtype and device, the degree
        statistics, the gather locality and the dense boundary."""
        s = self._schema
        locality = (self.source_index_span_ratio()
                    if self._row_ptr is not None else "implicit")
        return (s.origin, s.realization, s.num_src, s.num_dst, str(s.index_dtype),
                str(self.device), self.degree_statistics(), locality, self._dense_boundary)

    def _reference_plan_remarks(self, has_node_epilogue: bool = False) -> tuple[str, ...]:
        """The reference planner's decision for this CSR
        (tgx_plan_reference_buckets: SelectKernelSchedule.cpp:136-163,
        PlanDegreeBuckets.cpp:32-143, PlanSplitRows.cpp:84-147), given the
        degree statistics and, up to degree 4096, the exact histogram."""
        key = ("reference_plan", bool(has_node_epilogue))
        got = self._native_cache.get(key)
        if got is None:
            got = (describe_reference_plan(self.reference_plan(has_node_epilogue)),)
            self._native_cache[key] = got
        return got

    def reference_plan(self, has_node_epilogue: bool = False) -> dict:
        """The reference planner's decision for this graph as a dict: plan name,
        padding utilization (per mille, -1 when not computed), bucket upper
        bounds, their mappings and row counts, row-split sizing."""
        _, maximum, total = self._degree_stats()
        histogram = self.degree_histogram() if maximum <= 4096 else None
        return reference_plan(self._schema.num_dst, maximum, total, histogram,
                              has_node_epilogue)

    def __repr__(self) -> str:
        # The reference's summary line (interop/torch/graph.py:1444-1478).
        s = self._schema
        return (f"Graph(origin={s.origin}, lifecycle={s.lifecycle}, "
                f"realization={s.realization}, src={s.num_src:,}, dst={s.num_dst:,}, "
                f"edges={self.num_edges:,}, device={self.device})")

    def explain(self) -> str:
        """The reference's summary line, then this provider's row plan and
        the reference planner's decision once a HIP launch has built them."""
        lines = [repr(self), f"relation: {self._schema.realization}",
                 f"num_src: {self._schema.num_src}", f"num_dst: {self._schema.num_dst}"]
        plan = self._native_cache.get(("plan", WAVE_MAX, CHUNK_EDGES))
        if plan is not None:
            lines.append(f"row plan: {plan.counts()}")
            lines.extend(self._reference_plan_remarks())
        return "\n".join(lines)

    # ---- native device structures (built once per graph) -----------------
    def _kernel_csr(self) -> tuple[torch.Tensor, torch.Tensor]:
        """(row_ptr, col_idx) as the HIP kernels read them: one index dtype
        for both arrays, values checked once per graph.

        A kernel that gathered through an out-of-range column id would read
        outside the source table, so the first native use of a graph checks
        what ``validate="basic"`` leaves unchecked (one host sync, cached).
        """
        got = self._native_cache.get("csr")
        if got is None:
            row_ptr, col_idx = self.resolve_csr()
            if col_idx.dtype != row_ptr.dtype:
                col_idx = col_idx.to(row_ptr.dtype)
            E = col_idx.numel()
            checks = [row_ptr[0], row_ptr[-1]]
            if self._schema.num_dst:
                checks.append((row_ptr[1:] < row_ptr[:-1]).any().to(row_ptr.dtype))
            if E:
                checks += [col_idx.min(), col_idx.max()]
            vals = torch.stack([c.to(torch.int64) for c in checks]).cpu().tolist()
            if vals[0] != 0 or vals[1] != E:
                raise ValueError("row_ptr must start at 0 and end at the number of edges")
            if self._schema.num_dst and vals[2]:
                raise ValueError("row_ptr must be monotonic")
            if E and (vals[-2] < 0 or vals[-1] >= self._schema.num_src):
                raise ValueError("col_idx contains an out-of-range source index")
            if E >= (1 << 31) or max(self._schema.num_src, self._schema.num_dst) >= (1 << 31):
                raise ValueError("the HIP provider supports fewer than 2**31 edges and nodes")
            got = (row_ptr, col_idx)
            self._native_cache["csr"] = got
        return got

    def _dst_index32(self) -> torch.Tensor:
        """Destination row of every edge, int32, on the device (cached)."""
        got = self._native_cache.get("dst32")
        if got is None:
            row_ptr, col_idx = self._kernel_csr()
            E = col_idx.numel()
            got = torch.empty(max(E, 1), dtype=torch.int32, device=row_ptr.device)
            _native.call("tgx_destination_index", row_ptr.data_ptr(), _native.idx_bits(row_ptr),
                         self._schema.num_dst, E, got.data_ptr(), 32,
                         _native.stream_of(row_ptr))
            self._native_cache["dst32"] = got
        return got

    def _attn_blocks(self):
        """(cu_q, cu_k, causal) of a block-diagonal relation as int32 host
        arrays: cu_seqlens for varlen, one block for dense/triangular."""
        import numpy as np

        if self.is_varlen:
            cu = np.ascontiguousarray(self._cu_seqlens.cpu().numpy(), dtype=np.int64)
            if cu.size and cu[-1] >= 2**31:
                raise ValueError("the HIP attention tiles support fewer than 2**31 tokens")
            cu = cu.astype(np.int32)
            return cu, cu, bool(self._causal)
        n_dst, n_src = self._schema.num_dst, self._schema.num_src
        if max(n_dst, n_src) >= 2**31:
            raise ValueError("the HIP attention tiles support fewer than 2**31 tokens")
        return (np.array([0, n_dst], dtype=np.int32), np.array([0, n_src], dtype=np.int32),
                self._dense_boundary == "lower_inclusive")

    def _attn_tasks(self, kind: int, block: int, heads: int):
        """(cu_q, cu_k on device, tasks [n, 4] int32 on device, n, causal) for
        the attention tiles of a `heads`-head launch; kind 0 = query tiles,
        1 = key tiles (tgx_attn_tasks: XCD-grouped dispatch order)."""
        key = ("attn", kind, block, heads)
        got = self._native_cache.get(key)
        if got is None:
            import numpy as np

            cu_q, cu_k, causal = self._attn_blocks()
            n = ctypes.c_int64()
            args = (cu_q.ctypes.data, cu_k.ctypes.data, cu_q.size - 1, heads, block, kind,
                    int(causal))
            _native.call("tgx_attn_tasks", *args, None, ctypes.byref(n))
            tasks = np.zeros(4 * max(n.value, 1), dtype=np.int32)
            _native.call("tgx_attn_tasks", *args, tasks.ctypes.data, ctypes.byref(n))
            dev = self.device
            got = (torch.as_tensor(cu_q, device=dev), torch.as_tensor(cu_k, device=dev),
                   torch.as_tensor(tasks, device=dev), n.value, causal)
            self._native_cache[key] = got
        return got

    def _attn_fwd_split(self, heads: int):
        """The forward's split-key-range task lists for a `heads`-head launch
        (tgx_attn_fwd_split_tasks with two resident workgroups per CU):
        (tasks, n_tasks, merge, n_merge, chunk_tiles, max_chunks) on the
        device, or None when no tile is worth splitting."""
        key = ("attn-split", heads)
        if key not in self._native_cache:
            import numpy as np

            cu_q, cu_k, causal = self._attn_blocks()
            slots = 2 * torch.cuda.get_device_properties(self.device).multi_processor_count
            n, n_merge = ctypes.c_int64(), ctypes.c_int64()
            chunk, max_chunks = ctypes.c_int32(), ctypes.c_int32()
            args = (cu_q.ctypes.data, cu_k.ctypes.data, cu_q.size - 1, heads, int(causal),
                    slots)
            _native.call("tgx_attn_fwd_split_tasks", *args, None, ctypes.byref(n), None,
                         ctypes.byref(n_merge), ctypes.byref(chunk), ctypes.byref(max_chunks))
            got = None
            if n_merge.value > 0:
                tasks = np.zeros(4 * max(n.value, 1), dtype=np.int32)
                merge = np.zeros(4 * n_merge.value, dtype=np.int32)
                _native.call("tgx_attn_fwd_split_tasks", *args, tasks.ctypes.data,
                             ctypes.byref(n), merge.ctypes.data, ctypes.byref(n_merge),
                             ctypes.byref(chunk), ctypes.byref(max_chunks))
                dev = self.device
                got = (torch.as_tensor(tasks, device=dev), n.value,
                       torch.as_tensor(merge, device=dev), n_merge.value, chunk.value,
                       max_chunks.value)
            self._native_cache[key] = got
        return self._native_cache[key]

    def _attn_ds_tiles(self, heads: int) -> int | None:
        """Stored dS tiles of a `heads`-head attention backward
        (tgx_attn_ds_tiles), None when the relation has too many."""
        key = ("attn-ds", heads)
        if key not in self._native_cache:
            cu_q, cu_k, causal = self._attn_blocks()
            n = ctypes.c_int64()
            try:
                _native.call("tgx_attn_ds_tiles", cu_q.ctypes.data, cu_k.ctypes.data,
                             cu_q.size - 1, heads, int(causal), ctypes.byref(n))
                self._native_cache[key] = n.value
            except NotImplementedError:
                self._native_cache[key] = None
        return self._native_cache[key]

    def _row_plan(self, wave_max: int = WAVE_MAX, chunk_edges: int = CHUNK_EDGES) -> RowPlanHandle:
        key = ("plan", wave_max, chunk_edges)
        handle = self._native_cache.get(key)
        if handle is None:
            row_ptr, _ = self._kernel_csr()
            handle = build_row_plan(row_ptr, self._schema.num_dst, wave_max=wave_max,
                                    chunk_edges=chunk_edges)
            self._native_cache[key] = handle
        return handle

    def _transposed(self, wave_max: int = WAVE_MAX, chunk_edges: int = CHUNK_EDGES) -> Transposed:
        key = ("transpose", wave_max, chunk_edges)
        t = self._native_cache.get(key)
        if t is None:
            row_ptr, col_idx = self._kernel_csr()
            row_ptr_t, col_t, perm, inv_perm = build_transpose(
                row_ptr, col_idx, self._schema.num_dst, self._schema.num_src)
            plan = build_row_plan(row_ptr_t, self._schema.num_src, wave_max=wave_max,
                                  chunk_edges=chunk_edges)
            t = Transposed(row_ptr_t, col_t, perm, inv_perm, plan)
            self._native_cache[key] = t
        return t


def _varlen_csr(cu_seqlens: torch.Tensor, causal: bool):
    """The block-diagonal relation of `cu_seqlens` as an explicit CSR, for
    the tensors the device builder does not take (CPU tensors).  Same
    relation as the reference's materialization (graph.py:260-294): row i of
    sequence [s, e) reads columns s..i when causal, s..e-1 otherwise.

    Built one sequence block at a time: a causal block of length L is the
    lower triangle of an L x L block, whose columns in row order are the
    second row of ``torch.tril_indices(L, L)``; a full block repeats its L
    columns once per row."""
    device, dtype = cu_seqlens.device, cu_seqlens.dtype
    bounds = cu_seqlens.tolist()
    degrees, columns = [], []
    for first, stop in zip(bounds[:-1], bounds[1:]):
        length = stop - first
        if length <= 0:
            continue
        if causal:
            degrees.append(torch.arange(1, length + 1, device=device, dtype=dtype))
            block = torch.tril_indices(length, length, device=device, dtype=dtype)[1]
        else:
            degrees.append(torch.full((length,), length, device=device, dtype=dtype))
            block = torch.arange(length, device=device, dtype=dtype).repeat(length)
        columns.append(block.add_(first))
    row_ptr = torch.zeros(bounds[-1] + 1 if bounds else 1, device=device, dtype=dtype)
    if degrees:
        torch.cumsum(torch.cat(degrees), 0, out=row_ptr[1:])
    col_idx = torch.cat(columns) if columns else torch.zeros(0, device=device, dtype=dtype)
    return row_ptr, col_idx


__all__ = ["Graph", "GraphSchema", "build_coo_csr", "build_row_plan", "build_transpose",
           "build_varlen_csr", "describe_reference_plan", "reference_plan"]

"""CPU tests of the product's host side: the C-ABI library loads and exports
every declared entry point, the native planner matches the reference lit
vectors, Graph validation/constructors, and edge-function recognition."""

import ctypes
import json
import re
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import tiga as tg
from tiga import _native, capture as cap
from oracle import ref, planner

ROOT = Path(__file__).resolve().parents[1]
GOLD = json.loads((ROOT / "tests" / "golden" / "reference_vectors.json").read_text())


def declared_symbols():
    names = set()
    for header in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(tgx_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_native.exported_symbols())
    assert lib.tgx_abi_version() == 13
    assert lib.tgx_status_string(1) == b"invalid argument"


def declared_arities():
    """Parameter count of every tgx_* function declared in include/*.h."""
    arity = {}
    for header in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        for m in re.finditer(r"\b(tgx_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
            params = m.group(2).strip()
            arity[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return arity


def test_binding_signatures_match_the_header():
    """Every ctypes signature has as many arguments as its declaration (an
    entry point whose parameters change without the binding would pass
    arguments in the wrong places)."""
    arity = declared_arities()
    assert len(arity) >= 10
    table = {**_native._SIGNATURES, **_native._OPTIONAL}
    for name, argtypes in table.items():
        assert name in arity, name
        assert len(argtypes) == arity[name], (name, len(argtypes), arity[name])


def _native_plan(case):
    lib = _native.lib()
    hist = case["histogram"]
    harr = (ctypes.c_int64 * len(hist))(*hist) if hist is not None else None
    code = ctypes.c_int()
    util = ctypes.c_int64()
    bounds = (ctypes.c_int64 * 64)()
    mapping = (ctypes.c_int * 64)()
    rows_in = (ctypes.c_int64 * 64)()
    nb = ctypes.c_int()
    ppr = ctypes.c_int64()
    active = ctypes.c_int64()
    st = lib.tgx_plan_reference_buckets(case["rows"], case["max"], case["sum"], harr,
                                        int(case["has_node"]), ctypes.byref(code),
                                        ctypes.byref(util), bounds, mapping, rows_in,
                                        ctypes.byref(nb), ctypes.byref(ppr),
                                        ctypes.byref(active))
    assert st == 0
    n = nb.value
    return {"plan": planner.PLAN_NAMES[code.value], "utilization_milli": util.value,
            "bounds": list(bounds[:n]), "mapping": [planner.MAPPING_NAMES[m] for m in mapping[:n]],
            "rows_in_bucket": list(rows_in[:n]), "partials_per_row": ppr.value,
            "active_rows": active.value}


@pytest.mark.parametrize("case", GOLD["planner"], ids=lambda c: c["cite"].split(":")[0].split("/")[-1])
def test_native_planner_matches_lit_vectors(case):
    res = _native_plan(case)
    for key, value in case["expect"].items():
        if key in res:
            assert res[key] == value, (key, res[key], value)
    # and the native planner agrees with the oracle planner on every field
    o = planner.plan(case["rows"], case["max"], case["sum"], case["histogram"], case["has_node"])
    for key in res:
        assert res[key] == o[key], key


def test_native_planner_random_histograms_agree_with_oracle():
    rng = np.random.default_rng(7)
    for _ in range(200):
        max_deg = int(rng.integers(1, 300))
        rows = int(rng.integers(1, 600))
        hist = np.zeros(max_deg + 1, dtype=np.int64)
        degs = rng.integers(0, max_deg + 1, size=rows)
        degs[0] = max_deg
        np.add.at(hist, degs, 1)
        case = {"rows": rows, "max": max_deg, "sum": int(degs.sum()),
                "histogram": hist.tolist() if rng.random() < 0.8 else None,
                "has_node": bool(rng.random() < 0.5)}
        res = _native_plan(case)
        o = planner.plan(case["rows"], case["max"], case["sum"], case["histogram"],
                         case["has_node"])
        for key in res:
            assert res[key] == o[key], (case, key)


def test_graph_from_csr_validation_messages():
    rp = torch.tensor([0, 2, 3, 5])
    col = torch.tensor([0, 2, 1, 0, 1])
    g = tg.Graph.from_csr(rp, col, validate="full")
    assert g.schema.num_src == 3 and g.schema.num_dst == 3
    bad = [
        (torch.tensor([1, 2, 3, 5]), col, "row_ptr\\[0\\] must be zero"),
        (torch.tensor([0, 2, 3, 4]), col, "row_ptr\\[-1\\] must equal"),
        (torch.tensor([0, 3, 2, 5]), col, "monotonic"),
        (rp, torch.tensor([0, 2, 1, 0, 7]), "out-of-range"),
    ]
    for r, c, msg in bad:
        with pytest.raises(ValueError, match=msg):
            tg.Graph.from_csr(r, c, num_src=3, validate="full")
        # the oracle restatement raises the same message
        with pytest.raises(ValueError, match=msg):
            ref.validate_csr(r.numpy(), c.numpy(), 3)
    with pytest.raises(TypeError):
        tg.Graph.from_csr(rp.float(), col)
    with pytest.raises(ValueError):
        tg.Graph.from_csr(rp.reshape(2, 2), col)


def test_graph_constructors_match_oracle():
    rng = np.random.default_rng(8)
    src = rng.integers(0, 9, size=40)
    dst = rng.integers(0, 7, size=40)
    g = tg.Graph.from_coo(torch.tensor(src), torch.tensor(dst), num_src=9, num_dst=7)
    rp, col, _ = ref.from_coo(src, dst, 9, 7)
    r2, c2 = g.resolve_csr()
    assert r2.tolist() == rp.tolist() and c2.tolist() == col.tolist()
    t = g.transpose()
    rpt, colt, _ = ref.transpose(rp, col, 9)
    r3, c3 = t.resolve_csr()
    assert r3.tolist() == rpt.tolist() and c3.tolist() == colt.tolist()
    cu = torch.tensor([0, 3, 4, 9])
    gv = tg.Graph.cu_seqlens(cu)
    rp4, col4 = ref.cu_seqlens_csr(cu.numpy())
    r4, c4 = gv.resolve_csr()
    assert r4.tolist() == rp4.tolist() and c4.tolist() == col4.tolist()
    assert gv.num_edges == int(rp4[-1])
    gc = tg.Graph.cat([tg.Graph.regular(3, 2), tg.Graph.regular(2, 1)])
    r5, c5 = gc.resolve_csr()
    assert r5.tolist() == [0, 2, 4, 6, 7, 8] and c5.tolist() == [0, 1, 2, 0, 1, 2, 3, 4]


class WeightedSum(tg.MessagePassing):
    reducer = tg.sum()

    def edge(self, src, dst, edge):
        return edge.weight * src.x


class WithBias(tg.MessagePassing):
    reducer = tg.sum()

    def edge(self, src, dst, edge):
        return edge.conductivity * src.temperature

    def node(self, dst, incoming):
        return incoming + dst.bias


class GAT(tg.MessagePassing):
    reducer = tg.online_softmax()

    def __init__(self, a_s, a_d, slope=0.2):
        super().__init__()
        self.a_s, self.a_d, self.slope = a_s, a_d, slope

    def edge(self, src, dst, edge):
        s = F.leaky_relu((src.h * self.a_s).sum(-1) + (dst.h * self.a_d).sum(-1), self.slope)
        return self.reducer(s, src.h)


class Dot(tg.MessagePassing):
    reducer = tg.online_softmax()

    def edge(self, src, dst, edge, scale):
        return self.reducer((src.k * dst.q).sum(dim=-1) * scale + edge.bias, src.v)


class Generic(tg.MessagePassing):
    reducer = tg.online_softmax()

    def edge(self, src, dst, edge):
        return self.reducer(src.score.exp(), src.value)


def test_recognizer_patterns():
    assert cap.recognize_weighted_sum(WeightedSum()._captured({})) == cap.WeightedSum("x", "weight")
    a = torch.zeros(2, 4)
    g = cap.recognize_gat(GAT(a, a)._captured({}))
    assert g is not None and g.h_field == "h" and g.slope == 0.2
    d = cap.recognize_dot(Dot()._captured({"scale": 0.125}))
    assert d == cap.DotProduct("q", "k", "v", 0.125, "bias")
    assert Generic()._captured({}) is None


def test_readme_and_quickstart_on_cpu():
    g = GOLD["readme_weighted_sum"]
    graph = tg.Graph.from_csr(torch.tensor(g["row_ptr"]), torch.tensor(g["col_idx"]), num_src=3)
    x = torch.tensor(g["x"], requires_grad=True)
    w = torch.tensor(g["weight"], requires_grad=True)
    k = WeightedSum()
    out = k(graph=graph, src={"x": x}, dst={}, edge={"weight": w})
    dx, dw = torch.autograd.grad(out.sum(), (x, w))
    assert out.tolist() == g["out"] and dx.tolist() == g["dx"] and dw.tolist() == g["dw"]
    # The reference's dispatch for host tensors: the sparse CSR product.
    assert k.last_variant.provider == "torch.sparse.mm"
    q = GOLD["quickstart_node_bias"]
    bias = torch.tensor(q["bias"], requires_grad=True)
    out = WithBias()(graph=graph, src={"temperature": x}, dst={"bias": bias},
                     edge={"conductivity": w})
    np.testing.assert_allclose(out.detach().numpy(), q["out"], rtol=1e-6)


def test_strict_mode_refuses_eager():
    graph = tg.Graph.from_csr(torch.tensor([0, 1]), torch.tensor([0]), num_src=1)
    tg.config.strict = True
    try:
        with pytest.raises(RuntimeError, match="strict"):
            Generic()(graph=graph, src={"score": torch.ones(1), "value": torch.ones(1)}, dst={})
    finally:
        tg.config.strict = False


def test_block_prune_threshold_rejected_on_csr():
    class Pruned(tg.MessagePassing):
        reducer = tg.online_softmax(block_prune_threshold=0.5)

        def edge(self, src, dst, edge):
            return self.reducer(src.s, src.v)

    graph = tg.Graph.from_csr(torch.tensor([0, 1]), torch.tensor([0]), num_src=1)
    with pytest.raises(NotImplementedError):
        Pruned()(graph=graph, src={"s": torch.ones(1), "v": torch.ones(1)}, dst={})


def test_kernel_csr_unifies_dtypes_and_rejects_bad_columns():
    rp = torch.tensor([0, 2, 3, 5], dtype=torch.int64)
    g = tg.Graph.from_csr(rp, torch.tensor([0, 2, 1, 0, 1], dtype=torch.int32), num_src=3)
    r, c = g._kernel_csr()
    assert r.dtype == c.dtype == torch.int64 and c.tolist() == [0, 2, 1, 0, 1]
    for col, msg in (([0, 2, 1, 0, 3], "out-of-range"), ([0, -1, 1, 0, 1], "out-of-range")):
        bad = tg.Graph.from_csr(rp, torch.tensor(col), num_src=3)
        with pytest.raises(ValueError, match=msg):
            bad._kernel_csr()
    bad_rp = tg.Graph.from_csr(torch.tensor([0, 3, 2, 5]), torch.tensor([0, 2, 1, 0, 1]),
                               num_src=3)
    with pytest.raises(ValueError, match="monotonic"):
        bad_rp._kernel_csr()


def _attn_tasks(cu_q, cu_k, H, block, kind, causal):
    n = ctypes.c_int64()
    cq = np.ascontiguousarray(cu_q, dtype=np.int32)
    ck = np.ascontiguousarray(cu_k, dtype=np.int32)
    args = (cq.ctypes.data, ck.ctypes.data, cq.size - 1, H, block, kind, int(causal))
    _native.call("tgx_attn_tasks", *args, None, ctypes.byref(n))
    tasks = np.zeros(4 * max(n.value, 1), dtype=np.int32)
    _native.call("tgx_attn_tasks", *args, tasks.ctypes.data, ctypes.byref(n))
    return tasks[: 4 * n.value].reshape(n.value, 4)


@pytest.mark.parametrize("kind,block", [(0, 128), (1, 64)])
@pytest.mark.parametrize("causal,rect", [(True, False), (False, False), (False, True)])
def test_attn_tasks_cover_once_grouped_per_xcd(kind, block, causal, rect):
    """Host-side work list of the attention tiles: every (block, tile, head)
    exactly once; all tiles of one (block, head) on one XCD (slot % 8),
    consecutive in that XCD's queue and heaviest first; XCD loads balanced."""
    cu_q = np.array([0, 3, 300, 300, 301, 1500, 1700, 4000], dtype=np.int32)
    cu_k = (np.array([0, 10, 10, 90, 91, 1000, 1300, 1310], dtype=np.int32) if rect else cu_q)
    H = 3
    t = _attn_tasks(cu_q, cu_k, H, block, kind, causal)
    assert t.shape[0] % 8 == 0
    real = t[t[:, 0] >= 0]
    assert (t[t[:, 0] < 0][:, 1:] == 0).all()
    rows = cu_q if kind == 0 else cu_k
    expect = sorted((b, r0, h) for b in range(len(rows) - 1) for h in range(H)
                    for r0 in range(rows[b], rows[b + 1], block))
    assert sorted(map(tuple, real[:, :3].tolist())) == expect
    # tile0: the first stored dS tile of (block, head) (tgx_attn_ds_tiles).
    nt = [(-(-(cu_q[b + 1] - cu_q[b]) // 64)) * (-(-(cu_q[b + 1] - cu_q[b]) // 64) + 1) // 2
          if causal else -(-(cu_q[b + 1] - cu_q[b]) // 64) * -(-(cu_k[b + 1] - cu_k[b]) // 64)
          for b in range(len(cu_q) - 1)]
    base = np.concatenate([[0], np.cumsum(np.array(nt) * H)])
    for b, _, h, t0 in real.tolist():
        assert t0 == base[b] + h * nt[b]
    n = ctypes.c_int64()
    _native.call("tgx_attn_ds_tiles", cu_q.ctypes.data, cu_k.ctypes.data, len(cu_q) - 1, H,
                 int(causal), ctypes.byref(n))
    assert n.value == base[-1]

    def work(b, r0):
        q0, q1, k0, k1 = (int(x) for x in (cu_q[b], cu_q[b + 1], cu_k[b], cu_k[b + 1]))
        if kind == 0:
            return (min(r0 + block, q1) - k0) if causal else (k1 - k0)
        return (q1 - r0) if causal else (q1 - q0)

    loads = [0] * 8
    for x in range(8):
        queue = [tuple(row[:3]) for row in t[x::8] if row[0] >= 0]
        col = t[x::8, 0]
        assert all(col[i] >= 0 for i in range(len(queue)))   # padding only at the end
        groups = []
        for b, r0, h in queue:
            if not groups or groups[-1][0] != (b, h):
                groups.append(((b, h), []))
            groups[-1][1].append(work(b, r0))
        keys = [gr[0] for gr in groups]
        assert len(keys) == len(set(keys)), "a group's tiles are split in the queue"
        for _, ws in groups:
            assert ws == sorted(ws, reverse=True)
            loads[x] += max(sum(ws), 1)
    group_work = {}
    for b, r0, h in expect:
        group_work[(b, h)] = group_work.get((b, h), 0) + work(b, r0)
    assert max(loads) - min(loads) <= max(max(group_work.values()), 1)
    where = {}
    for slot, row in enumerate(t):
        if row[0] >= 0:
            where.setdefault((row[0], row[2]), set()).add(slot % 8)
    assert all(len(v) == 1 for v in where.values())
    with pytest.raises(RuntimeError, match="square"):
        _attn_tasks(cu_q, np.array([0, 1, 2, 3, 4, 5, 6, 7]), H, block, kind, True)


def test_torch_library_registration_reference_example():
    """The reference's torch.library test (tests/python/test_torch_provider.py:
    80-112, examples/torch_library.py) on CPU tensors (eager path): call,
    gradients, opcheck and torch.compile(fullgraph=True)."""

    class Weighted(tg.MessagePassing):
        reducer = tg.sum()

        def edge(self, src, dst, edge):
            return edge.weight * src.x

    row_ptr = torch.tensor([0, 2, 4], dtype=torch.int64)
    col_idx = torch.tensor([0, 1, 1, 2], dtype=torch.int64)
    graph = tg.Graph.from_csr(row_ptr, col_idx, num_src=3)
    x = torch.tensor([1.0, 2.0, 4.0], requires_grad=True)
    weight = torch.tensor([2.0, 3.0, 5.0, 7.0], requires_grad=True)
    registered = tg.interop.torch.register_message_passing(
        Weighted(), graph=graph, src={"x": x}, dst={}, edge={"weight": weight})
    assert registered.qualified_name.startswith("tiga::")
    output = registered(src={"x": x}, dst={}, edge={"weight": weight})
    assert output.tolist() == [8.0, 38.0]
    dx, dweight = torch.autograd.grad(output.sum(), (x, weight))
    torch.testing.assert_close(dx, torch.tensor([2.0, 8.0, 7.0]))
    torch.testing.assert_close(dweight, torch.tensor([1.0, 2.0, 2.0, 4.0]))
    checked = registered.opcheck(x.detach(), weight.detach())
    assert all(result == "SUCCESS" for result in checked.values()), checked
    compiled = torch.compile(
        lambda a, b: registered(src={"x": a}, dst={}, edge={"weight": b}), fullgraph=True)
    cx = x.detach().clone().requires_grad_(True)
    cw = weight.detach().clone().requires_grad_(True)
    out_c = compiled(cx, cw)
    grads_c = torch.autograd.grad(out_c.sum(), (cx, cw))
    torch.testing.assert_close(out_c, output)
    torch.testing.assert_close(grads_c[0], dx)
    torch.testing.assert_close(grads_c[1], dweight)
    # the same specialization registers once; field names are checked
    again = tg.interop.torch.register_message_passing(
        Weighted(), graph=graph, src={"x": x}, dst={}, edge={"weight": weight})
    assert again is registered
    with pytest.raises(ValueError, match="edge fields"):
        registered(src={"x": x}, dst={}, edge={"w": weight})
    with pytest.raises(NotImplementedError, match="static CSR"):
        tg.interop.torch.register_message_passing(
            Weighted(), graph=tg.Graph.dense(3), src={"x": x}, dst={}, edge={})


def test_reference_method_runs_eager_even_when_covered():
    class Weighted(tg.MessagePassing):
        reducer = tg.sum()

        def edge(self, src, dst, edge):
            return edge.weight * src.x

    graph = tg.Graph.from_csr(torch.tensor([0, 2, 4]), torch.tensor([0, 1, 1, 2]), num_src=3)
    out = Weighted().reference(graph=graph, src={"x": torch.tensor([1.0, 2.0, 4.0])}, dst={},
                               edge={"weight": torch.tensor([2.0, 3.0, 5.0, 7.0])})
    assert out.tolist() == [8.0, 38.0]

    class Pruned(tg.MessagePassing):
        reducer = tg.online_softmax(block_prune_threshold=0.5)

        def edge(self, src, dst, edge):
            return self.reducer((src.k * dst.q).sum(-1), src.k)

    with pytest.raises(NotImplementedError, match="no eager"):
        Pruned().reference(graph=tg.Graph.dense(2), src={"k": torch.ones(2, 3)},
                           dst={"q": torch.ones(2, 3)})


def test_edge_mlp_validation_of_layer_widths():
    """tgx_edge_mlp: out_width beyond the padded width, or a last layer with
    more than one output, is rejected before anything is launched."""
    lib = _native.lib()
    buf = torch.zeros(2, 32 * 32 + 32)
    seg = torch.zeros(4, 8)

    def mlp(out_width):
        m = _native.EdgeMlp()
        m.n_layers, m.width = 2, 32
        m.act[0] = 1
        m.weights_dev = buf.data_ptr()
        m.n_segments = 1
        m.seg_role[0], m.seg_width[0], m.seg_stride[0] = 0, 8, 8
        m.seg_dev[0] = seg.data_ptr()
        for i, w in enumerate(out_width):
            m.out_width[i] = w
        return m

    size = ctypes.c_size_t()
    for bad in ((40, 1), (16, 2), (-1, 1)):
        m = mlp(bad)
        assert lib.tgx_edge_mlp_backward_workspace(0, ctypes.byref(m), ctypes.byref(size)) == 1
        assert b"width" in lib.tgx_last_error() or b"output" in lib.tgx_last_error()
    for good in ((16, 1), (0, 0), (32, 1)):
        m = mlp(good)
        assert lib.tgx_edge_mlp_backward_workspace(0, ctypes.byref(m), ctypes.byref(size)) == 0


def test_attention_backward_fold_segment_is_checked_before_any_launch():
    """tgx_edge_mlp_attention_backward: fold_segment must name a segment
    whose width is value_width (or be -1); a bad one is rejected on the host
    before any HIP call."""
    lib = _native.lib()
    buf = torch.zeros(2, 32 * 32 + 32)
    segs = [torch.zeros(4, 8), torch.zeros(4, 3)]
    m = _native.EdgeMlp()
    m.n_layers, m.width = 2, 32
    m.act[0] = 1
    m.weights_dev = buf.data_ptr()
    m.n_segments = 2
    for i, t in enumerate(segs):
        m.seg_role[i], m.seg_width[i], m.seg_stride[i] = 0, t.shape[1], t.shape[1]
        m.seg_dev[i] = t.data_ptr()
    m.out_width[0], m.out_width[1] = 16, 1
    for fold, match in ((2, b"fold_segment"), (-2, b"fold_segment"), (1, b"value_width")):
        status = lib.tgx_edge_mlp_attention_backward(
            None, None, 64, 0, ctypes.byref(m), None, None, None, None, 8, None, fold, None,
            None, None, 0, None)
        assert status == 1 and match in lib.tgx_last_error(), (fold, lib.tgx_last_error())


def test_sum_rejects_source_tables_past_32_bit_rows():
    """The sum kernels hold gathered row indices in 32 bits: a source table of
    2^31 rows or more is refused before anything is launched."""
    lib = _native.lib()
    plan = _native.RowPlan(4, 0, 4, 0, 0, 512, 512, 0x1000, 0x1000)
    dummy = 0x1000   # never dereferenced: validation fails first
    st = lib.tgx_csr_sum_fwd(dummy, dummy, 64, ctypes.byref(plan), dummy, None, dummy, 4,
                             1 << 31, 1, _native.DTYPE_F32, None, None)
    assert st == 1 and b"2^31 rows" in lib.tgx_last_error()
    st = lib.tgx_csr_edge_dot(dummy, dummy, 64, ctypes.byref(plan), dummy, dummy, dummy, 4,
                              1 << 31, 1, _native.DTYPE_F32, None)
    assert st == 1 and b"2^31 rows" in lib.tgx_last_error()


@pytest.mark.parametrize("cu,H,causal", [
    ([0, 4096], 16, 1),                 # one causal block: two chunks for the long tiles
    ([0, 8192], 2, 1),                  # up to eight chunks
    ([0, 4096], 4, 0),                  # non-causal, few equal tiles
    ([0, 700, 705, 3000], 3, 1),        # several blocks, a short one
    ([0, 512, 1024], 16, 1),            # balanced: nothing split
])
def test_attn_fwd_split_tasks_cover_every_key_tile_once(cu, H, causal):
    """tgx_attn_fwd_split_tasks: every (query tile, head) is one whole task or
    chunks that cover its 64-key tiles exactly once, each chunk at most
    chunk_tiles long, with one merge entry per split tile naming its chunks."""
    lib = _native.lib()
    cu = np.asarray(cu, dtype=np.int32)
    n, nm = ctypes.c_int64(), ctypes.c_int64()
    chunk, mc = ctypes.c_int32(), ctypes.c_int32()
    args = (cu.ctypes.data, cu.ctypes.data, cu.size - 1, H, causal, 512)
    assert lib.tgx_attn_fwd_split_tasks(*args, None, ctypes.byref(n), None, ctypes.byref(nm),
                                        ctypes.byref(chunk), ctypes.byref(mc)) == 0
    tasks = np.zeros(4 * max(n.value, 1), dtype=np.int32)
    merge = np.zeros(4 * max(nm.value, 1), dtype=np.int32)
    assert lib.tgx_attn_fwd_split_tasks(*args, tasks.ctypes.data, ctypes.byref(n),
                                        merge.ctypes.data, ctypes.byref(nm),
                                        ctypes.byref(chunk), ctypes.byref(mc)) == 0
    tasks = tasks.reshape(-1, 4)[:n.value]
    merge = merge.reshape(-1, 4)[:nm.value]
    assert n.value % 8 == 0
    covered = {}
    for blk, q0, h, code in tasks:
        if blk < 0:
            continue
        k0, k1 = cu[blk], cu[blk + 1]
        nk = -(-((min(q0 + 128, k1) if causal else k1) - k0) // 64)
        if code < 0:
            assert nk <= chunk.value
            tiles = range(nk)
        else:
            m, c = divmod(int(code), mc.value)
            assert tuple(merge[m][:3]) == (blk, q0, h) and c < merge[m][3]
            tiles = range(c * chunk.value, min(nk, (c + 1) * chunk.value))
            assert len(tiles) > 0
        for t in tiles:
            key = (int(blk), int(q0), int(h), t)
            assert key not in covered
            covered[key] = True
    expect = 0
    for b in range(cu.size - 1):
        for q0 in range(cu[b], cu[b + 1], 128):
            nk = -(-((min(q0 + 128, cu[b + 1]) if causal else cu[b + 1]) - cu[b]) // 64)
            expect += nk * H
    assert len(covered) == expect
    if cu.tolist() == [0, 512, 1024]:
        assert nm.value == 0


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus N > 1 exits with a message before any
    GPU work."""
    import subprocess
    import sys

    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
def test_cpu_varlen_csr_matches_the_oracle_with_empty_sequences(causal, idx):
    """The CPU materialization of Graph.cu_seqlens against the oracle's
    per-position loop, with empty sequences at the start, middle and end,
    in the index dtype of cu_seqlens."""
    cu = torch.tensor([0, 0, 5, 5, 6, 13, 13], dtype=idx)
    g = tg.Graph.cu_seqlens(cu, causal=causal)
    rp, col = ref.cu_seqlens_csr(cu.numpy(), causal=causal)
    r, c = g.resolve_csr()
    assert r.dtype == idx and c.dtype == idx
    assert r.tolist() == rp.tolist() and c.tolist() == col.tolist()
    assert g.num_edges == int(rp[-1])
